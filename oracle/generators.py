"""The reference's deterministic input generators, restated.

matrix()  Tests/TritonMetalCoreTests/DotTests.swift:32-34
tensor()  Tests/TritonMetalCoreTests/AttentionTests.swift:56-62
          (same formula in AttentionBackwardTests.swift:199-204)
ramp()    bench inputs (i % p)/p - 0.5, AttentionBenchmark.swift:354
synthetic()  the SAE encoder's inputs, Tests/TritonMetalMLXTests/MLXTestSupport.swift:82-90
          (same formula in Sources/tmsae/main.swift and python/examples/sae_encode.py:64-69)
"""

import numpy as np


def matrix(count: int, seed: int) -> np.ndarray:
    """((i*7 + seed*13) % 17) * 0.25 - 2, as float32."""
    i = np.arange(count, dtype=np.int64)
    return (((i * 7 + seed * 13) % 17).astype(np.float32) * np.float32(0.25) - np.float32(2))


def tensor(count: int, seed: int, spread: float = 1.0) -> np.ndarray:
    """(((i*31 + seed*17) % 23) / 23 * 2 - 1) * spread, as float32 (each step in
    float32, as the Swift expression evaluates it)."""
    i = np.arange(count, dtype=np.int64)
    bucket = ((i * 31 + seed * 17) % 23).astype(np.float32)
    unit = bucket / np.float32(23)
    return (unit * np.float32(2) - np.float32(1)) * np.float32(spread)


def ramp(count: int, period: int) -> np.ndarray:
    i = np.arange(count, dtype=np.int64)
    return (i % period).astype(np.float32) / np.float32(period) - np.float32(0.5)


def normal(shape, seed: int, scale: float = 1.0) -> np.ndarray:
    """Seeded N(0, scale^2) float32 (numpy's PCG64 Generator)."""
    return np.random.default_rng(seed).standard_normal(shape, dtype=np.float32) * np.float32(scale)


def uniform(shape, seed: int, low=-1.0, high=1.0) -> np.ndarray:
    return np.random.default_rng(seed).uniform(low, high, size=shape).astype(np.float32)


def synthetic(shape, offset: int = 0, modulus: int = 71) -> np.ndarray:
    """Float(((i + offset) * 13) % modulus) / Float(modulus) - 0.5, each step in
    float32 as the Swift expression evaluates it, reshaped to `shape`."""
    shape = tuple(shape)
    count = int(np.prod(shape)) if shape else 1
    i = np.arange(count, dtype=np.int64)
    bucket = (((i + offset) * 13) % modulus).astype(np.float32)
    return (bucket / np.float32(modulus) - np.float32(0.5)).reshape(shape)
