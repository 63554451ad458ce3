"""matmul_kernel on the device against the oracle (reference DotTests.swift:318-646,
python/examples/matmul.py:66-79) and benchmark configs 1 and 3.

Tolerance metric: the reference's |a - b| / max(1, |b|) (GPUHarness.swift:146),
with the reference computed from inputs already rounded to the element type
(DotTests.swift:533-553)."""

import numpy as np
import pytest

from oracle import generators as G
from oracle import native as N
from oracle import tolerance as T
from triton_metal import _core, ops
from triton_metal.buffer import DeviceBuffer, round_to

pytestmark = pytest.mark.gpu

DT = {"f32": "float32", "f16": "float16", "bf16": "bfloat16"}


UNIT_ROUNDOFF = {"f32": 2.0 ** -24, "f16": 2.0 ** -11, "bf16": 2.0 ** -8}


def _assert_column_checksum(a, b, c, element):
    """1^T C = (1^T A) B over every column, within the error the output rounding
    alone can contribute (u * sum_i |C_ij|) plus the f32 accumulation bound
    (K * 2^-24 * sum_i (|A||B|)_ij): a property that sees every tile of C."""
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    colsum = a64.sum(0) @ b64
    got = c.astype(np.float64).sum(0)
    k = a.shape[1]
    bound = (UNIT_ROUNDOFF[element] * np.abs(c.astype(np.float64)).sum(0)
             + k * 2.0 ** -24 * (np.abs(a64).sum(0) @ np.abs(b64)))
    worst = np.max(np.abs(got - colsum) / bound)
    print(f"column checksum: worst error / bound = {worst:.3f}")
    assert worst <= 1.0


def run_matmul(a_flat, b_flat, m, n, k, strides, element="f32", c_elems=None, c_init=None,
               threads=128):
    """Upload flat A/B, run one matmul_kernel dispatch, return C (flat, f32)."""
    dtype = DT[element]
    sam, sak, sbk, sbn, scm, scn = strides
    a = DeviceBuffer.from_numpy(np.asarray(a_flat, np.float32), dtype)
    b = DeviceBuffer.from_numpy(np.asarray(b_flat, np.float32), dtype)
    c = DeviceBuffer(c_elems or m * n, dtype)
    if c_init is not None:
        c.write(np.asarray(c_init, np.float32))
    lib = ops.library(element)
    kernel = lib.kernels["matmul_kernel"]
    try:
        grid, kinds, values = ops.matmul_args(a, b, c, m, n, k, strides)
        _core.launch(kernel, grid, threads, kinds, values)
        return c.float32(), _core.kernel_variant(kernel)
    finally:
        for x in (a, b, c):
            x.free()


@pytest.mark.parametrize("m,n,k", [(64, 64, 64), (129, 257, 65), (1, 1, 1), (37, 8, 96),
                                   (100, 100, 3), (65, 33, 129), (16, 16, 16), (5, 3, 7)])
def test_tutorial_matmul_is_exact_on_the_reference_inputs(device, m, n, k):
    """DotTests.swift:369-396.  The matrix() inputs make every partial sum exact,
    so any summation order gives the exact answer: equality, not a tolerance."""
    a = G.matrix(m * k, 3)
    b = G.matrix(k * n, 11)
    c, _ = run_matmul(a, b, m, n, k, (k, 1, n, 1, n, 1))
    want = N.gemm(a, b, m, n, k, k, 1, n, 1)
    assert np.array_equal(c.reshape(m, n).astype(np.float64), want)


@pytest.mark.parametrize("m,n,k,lda,ldb", [(70, 36, 40, 40, 36), (33, 40, 27, 30, 43),
                                           (64, 64, 64, 65, 67)])
def test_awkward_row_strides(device, m, n, k, lda, ldb):
    """DotTests.swift:403-437."""
    a = G.matrix(m * lda, 5)
    b = G.matrix(k * ldb, 7)
    c, _ = run_matmul(a, b, m, n, k, (lda, 1, ldb, 1, n, 1))
    want = N.gemm(a, b, m, n, k, lda, 1, ldb, 1)
    assert T.hybrid_error(c.reshape(m, n), want) <= 1e-5


def test_non_unit_innermost_stride(device):
    """DotTests.swift:439-461."""
    m = n = k = 40
    col, lda, ldb = 3, 120, 120
    a = G.matrix(m * lda, 5)
    b = G.matrix(k * ldb, 7)
    c, _ = run_matmul(a, b, m, n, k, (lda, col, ldb, col, n, 1))
    want = N.gemm(a, b, m, n, k, lda, col, ldb, col)
    assert T.hybrid_error(c.reshape(m, n), want) <= 1e-5


@pytest.mark.parametrize("element,tol", [("f16", 5e-3), ("bf16", 1.0 / 256)])
def test_half_operands_accumulate_in_float(device, element, tol):
    """DotTests.swift:466-554: f16 at 5e-3, bf16 at 1/256, reference from rounded inputs."""
    m, n, k = 70, 66, 34
    a = (np.arange(m * k) % 11).astype(np.float32) * 0.125 - 0.5
    b = (np.arange(k * n) % 7).astype(np.float32) * 0.25 - 0.75
    c, _ = run_matmul(a, b, m, n, k, (k, 1, n, 1, n, 1), element)
    want = N.gemm(round_to(a, element), round_to(b, element), m, n, k, k, 1, n, 1)
    assert T.hybrid_error(c.reshape(m, n), want) <= tol


@pytest.mark.parametrize("threads", [32, 64, 128, 256, 512, 1024])
def test_matmul_at_every_requested_workgroup_size(device, threads):
    """DotTests.swift:585-605: the answer does not depend on the threads asked for."""
    m, n, k = 48, 40, 40
    a, b = G.matrix(m * k, 2), G.matrix(k * n, 9)
    c, _ = run_matmul(a, b, m, n, k, (k, 1, n, 1, n, 1), threads=threads)
    assert np.array_equal(c.reshape(m, n).astype(np.float64), N.gemm(a, b, m, n, k, k, 1, n, 1))


@pytest.mark.parametrize("element", ["f32", "bf16"])
def test_matmul_does_not_write_outside_the_logical_matrix(device, element):
    """DotTests.swift:609-646: padding columns of a strided C keep their sentinel."""
    m, n, k, stride = 17, 19, 23, 24
    a, b = G.matrix(m * k, 4), G.matrix(k * n, 6)
    sentinel = -1232.0  # exactly representable in f32, f16 and bf16
    c, _ = run_matmul(a, b, m, n, k, (k, 1, n, 1, stride, 1), element, c_elems=m * stride,
                      c_init=np.full(m * stride, sentinel, np.float32))
    c = c.reshape(m, stride)
    want = N.gemm(round_to(a, element), round_to(b, element), m, n, k, k, 1, n, 1)
    assert np.all(c[:, n:] == sentinel)
    assert T.hybrid_error(c[:, :n], want) <= (1e-5 if element == "f32" else 1 / 256)


def test_numpy_tutorial_known_answer(device):
    """matmul.py:66-79: 256^3 standard normal from default_rng(0); the reference
    asserts max|triton - numpy| < 1e-3 (and measured 0 on its summation order)."""
    rng = np.random.default_rng(0)
    a = rng.standard_normal((256, 256), dtype=np.float32)
    b = rng.standard_normal((256, 256), dtype=np.float32)
    c, _ = run_matmul(a.reshape(-1), b.reshape(-1), 256, 256, 256, (256, 1, 256, 1, 256, 1))
    assert np.max(np.abs(c.reshape(256, 256) - a @ b)) < 1e-3


def test_config1_fp32_256_uniform(device):
    """Config 1: fp32 256^3, U[-1,1] from seed 0, 1e-5 (hybrid) vs fp64."""
    a = G.uniform((256, 256), seed=0)
    b = G.uniform((256, 256), seed=1)
    c, variant = run_matmul(a.reshape(-1), b.reshape(-1), 256, 256, 256, (256, 1, 256, 1, 256, 1))
    assert variant == "tm_gemm_fast_t64_k4_f32"  # 16 tiles of 64 x 64, K over 4 wave groups
    want = a.astype(np.float64) @ b.astype(np.float64)
    assert T.hybrid_error(c.reshape(256, 256), want) <= 1e-5


@pytest.mark.parametrize("m,n,k,lda,ldb,ldc,variant", [
    (2048, 1024, 32, None, None, None, "fast"),      # 128 tiles: half the compute units
    (1536, 2048, 96, 100, 2052, 2056, "fast_k2"),   # padded, 16-byte aligned rows; 3 k-steps, 2 groups
    (2048, 2048, 1024, None, None, None, "fast_k2"),  # one tile per CU: K over 2 wave groups
    (1024, 1024, 1024, None, None, None, "fast_t64_k2"),  # 64 tiles of 128: 64 x 64 tiles instead
    (192, 320, 64, 196, 324, 324, "fast_t64_k2"),
    (256, 256, 160, None, None, None, "fast_t64_k4"),  # 5 k-steps over 4 wave groups
    (160, 128, 32, None, None, None, "generic"),     # M not a multiple of 64
    (2048, 2048, 30, None, None, None, "generic"),    # rows not 16-byte aligned
    (1984, 2048, 32, None, None, None, "fast_t64"),   # M a multiple of 64 only
])
def test_fp32_gemm_kernels(device, m, n, k, lda, ldb, ldc, variant):
    _check_fp32_gemm(m, n, k, lda, ldb, ldc, variant, "nn")


@pytest.mark.parametrize("layout", ["nt", "tn"])
@pytest.mark.parametrize("m,n,k,ld_t,variant", [
    (2048, 1024, 64, None, "fast"),
    (1536, 2048, 96, 2052, "fast"),     # padded rows of the transposed operand
    (1024, 1024, 256, None, "fast_t64"),  # 64 x 64 tiles
])
def test_fp32_transposed_operand(device, layout, m, n, k, ld_t, variant):
    """One operand stored transposed: B with unit stride along K (nt) or A
    with unit stride along M (tn)."""
    _check_fp32_gemm(m, n, k, None, None, None, variant, layout, ld_t)


def _check_fp32_gemm(m, n, k, lda, ldb, ldc, variant, layout, ld_t=None):
    """fp32 on the fp32 MFMA kernel for whole 128 x 128 x 32 tiles and the
    generic one otherwise, against fp64: every element within the fp32
    accumulation bound K * 2^-24 * (|A||B|)_ij (deep K exceeds the reference's
    1e-5 hybrid figure through summation alone: 2.8e-5 at K = 1024 on U[-1, 1]),
    and the 1e-5 hybrid figure itself for K <= 256; C's padding columns stay
    untouched."""
    lda, ldb, ldc = lda or k, ldb or n, ldc or n
    rng = np.random.default_rng(11)
    a = rng.uniform(-1, 1, (m, lda)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, ldb)).astype(np.float32)
    a_flat, b_flat, strides = a.reshape(-1), b.reshape(-1), (lda, 1, ldb, 1, ldc, 1)
    if layout == "nt":   # B^T [n, ld_t]
        ld_t = ld_t or k
        bt = np.full((n, ld_t), np.inf, np.float32)
        bt[:, :k] = b[:, :n].T
        b_flat, strides = bt.reshape(-1), (lda, 1, 1, ld_t, ldc, 1)
    elif layout == "tn":  # A^T [k, ld_t]
        ld_t = ld_t or m
        at = np.full((k, ld_t), np.inf, np.float32)
        at[:, :m] = a[:, :k].T
        a_flat, strides = at.reshape(-1), (1, ld_t, ldb, 1, ldc, 1)
    c, got = run_matmul(a_flat, b_flat, m, n, k, strides,
                        c_elems=m * ldc, c_init=np.full(m * ldc, -7.0, np.float32))
    if variant == "generic":
        assert got == "tm_gemm_generic_f32"
    else:
        kind, _, tile = variant.partition("_")
        suffix = ("" if layout == "nn" else "_" + layout) + ("_" + tile if tile else "")
        assert got == f"tm_gemm_{kind}{suffix}_f32"
    c = c.reshape(m, ldc)
    a64, b64 = a[:, :k].astype(np.float64), b[:, :n].astype(np.float64)
    want = a64 @ b64
    bound = k * 2.0 ** -24 * (np.abs(a64) @ np.abs(b64))
    assert np.all(np.abs(c[:, :n] - want) <= bound)
    if k <= 256:
        assert T.hybrid_error(c[:, :n], want) <= 1e-5
    assert np.all(c[:, n:] == -7.0)


@pytest.mark.parametrize("element", ["bf16", "f16"])
def test_large_aligned_gemm_hybrid_and_checksums(device, element):
    """A 1024x768x512 aligned half GEMM: every element vs fp64 from rounded
    inputs (2e-2 hybrid), plus the column-sum checksum 1^T C = (1^T A) B."""
    m, n, k = 1024, 768, 512
    a = round_to(G.normal((m, k), seed=3), element)
    b = round_to(G.normal((k, n), seed=4), element)
    c, variant = run_matmul(a.reshape(-1), b.reshape(-1), m, n, k, (k, 1, n, 1, n, 1), element)
    c = c.reshape(m, n)
    want = a.astype(np.float64) @ b.astype(np.float64)
    assert T.hybrid_error(c, want) <= 2e-2
    _assert_column_checksum(a, b, c, element)


def test_config3_bf16_8192_cube(device):
    """Config 3: bf16 8192^3, N(0,1) from seed, f32 accumulate, bf16 out.
    Full size: 256 sampled rows against fp64 (from the bf16-rounded inputs) under
    the 2e-2 hybrid metric, the column-sum checksum over all rows, and every
    element against an fp32 BLAS product under the same metric."""
    m = n = k = 8192
    a = round_to(G.normal((m, k), seed=0), "bf16")
    b = round_to(G.normal((k, n), seed=1), "bf16")
    c, variant = run_matmul(a.reshape(-1), b.reshape(-1), m, n, k, (k, 1, n, 1, n, 1), "bf16")
    c = c.reshape(m, n)
    assert np.all(np.isfinite(c))
    rows = np.random.default_rng(7).choice(m, 256, replace=False)
    want = a[rows].astype(np.float64) @ b.astype(np.float64)
    err = T.hybrid_error(c[rows], want)
    print(f"config3 variant={variant} hybrid={err:.3e} max_abs={T.max_abs_error(c[rows], want):.3e}")
    assert err <= 2e-2
    _assert_column_checksum(a, b, c, "bf16")
    # every element: against an fp32 BLAS product of the same rounded inputs
    # (bf16 products are exact in fp32; its own summation error, measured on
    # the sampled rows against fp64, is a few units of 2^-24 relative)
    want32 = a @ b
    assert T.hybrid_error(want32[rows], want) <= 1e-4
    err_all = T.hybrid_error(c, want32)
    print(f"config3 all rows vs fp32 BLAS: hybrid={err_all:.3e}")
    assert err_all <= 2e-2
