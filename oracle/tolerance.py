"""The reference's error metrics.

hybrid_error    |a - b| / max(1, |b|), worst element
                (Tests/TritonMetalCoreTests/GPUHarness.swift:146)
relative_error  max|a - b| / max|b|   (python/examples/attention_training.py:250-252)
summation_bound n * u * A * max|b|    (AttentionBackwardTests.swift:17-23, :301-324)
lse_bound       the forward L tolerance for 16-bit elements (see its docstring)
"""

import numpy as np


def hybrid_error(actual, expected) -> float:
    a = np.asarray(actual, dtype=np.float64)
    b = np.asarray(expected, dtype=np.float64)
    if a.shape != b.shape:
        raise ValueError(f"shape {a.shape} != {b.shape}")
    if np.any(np.isnan(a) != np.isnan(b)):
        return float("inf")
    ok = ~np.isnan(b)
    if not ok.any():
        return 0.0
    return float(np.max(np.abs(a[ok] - b[ok]) / np.maximum(1.0, np.abs(b[ok]))))


def relative_error(actual, expected) -> float:
    a = np.asarray(actual, dtype=np.float64)
    b = np.asarray(expected, dtype=np.float64)
    scale = max(float(np.max(np.abs(b))), 1e-30)
    return float(np.max(np.abs(a - b))) / scale


def max_abs_error(actual, expected) -> float:
    return float(np.max(np.abs(np.asarray(actual, np.float64) - np.asarray(expected, np.float64))))


def summation_bound(expected, terms: int, unit_roundoff: float, amplification: float) -> float:
    peak = max(float(np.max(np.abs(expected))), 1e-30)
    return terms * unit_roundoff * amplification * peak


U_F32 = 2.0 ** -24
U_F16 = 2.0 ** -11
U_BF16 = 2.0 ** -8


def lse_bound(element: str) -> float:
    """Tolerance on L (log2 units) for a 16-bit forward.  2e-3 covers the
    scores of rounded inputs; the HIP forward also takes its row sums l from
    the P it rounded to the element type (the weights P V uses), where the
    reference sums the unrounded P: each rounded P is within a factor 1 +- u of
    the unrounded one, so log2 of the sum moves by at most log2(1 + u)."""
    u = U_BF16 if element == "bf16" else U_F16
    return 2e-3 + float(np.log2(1.0 + u))
