"""The specialised gfx950 kernels: which shapes take them, and parity at their
edges (tiny and ragged sequence lengths, padded strides, non-square GEMMs).
Every case is checked against the fp64 oracle; the variant each dispatch ran is
read back through tm_kernel_variant."""

import math

import numpy as np
import pytest

from oracle import generators as G
from oracle import reference as R
from oracle import tolerance as T
from triton_metal import _core, ops
from triton_metal.buffer import DeviceBuffer, round_to

pytestmark = pytest.mark.gpu

DT = {"f32": "float32", "f16": "float16", "bf16": "bfloat16"}


def _attention(heads, seq, dim, element, causal, stride_seq=None, stride_head=None, seed=0):
    """Forward + backward through the ABI with optional padded strides; returns
    (outputs dict, variants, inputs)."""
    ss = stride_seq or dim
    sh = stride_head or seq * ss
    total = (heads - 1) * sh + (seq - 1) * ss + dim
    rng = np.random.default_rng(seed)
    dense = [round_to(rng.standard_normal((heads, seq, dim), dtype=np.float32), element)
             for _ in range(4)]

    def scatter(x):
        flat = np.zeros(total, np.float32)
        for h in range(heads):
            for i in range(seq):
                flat[h * sh + i * ss: h * sh + i * ss + dim] = x[h, i]
        return flat

    def gather(flat):
        return np.stack([np.stack([flat[h * sh + i * ss: h * sh + i * ss + dim] for i in range(seq)])
                         for h in range(heads)])

    lib = ops.library(element, dim, causal)
    dtype = DT[element]
    bufs = {k: DeviceBuffer.from_numpy(scatter(x), dtype) for k, x in zip(("q", "k", "v", "do"), dense)}
    for k in ("o", "dq", "dk", "dv"):
        bufs[k] = DeviceBuffer.from_numpy(np.zeros(total, np.float32), dtype)
    bufs["lse"] = DeviceBuffer((heads, seq), "float32")
    bufs["delta"] = DeviceBuffer((heads, seq), "float32")
    h = lambda k: bufs[k].tm_handle
    scale = 1 / math.sqrt(dim)
    B, I, F = _core.ARG_BUFFER, _core.ARG_I32, _core.ARG_F32
    kern = lib.kernels
    variants = []
    try:
        _core.launch(kern["attn_fwd"], (1, heads, 1), 128, [B, B, B, B, F, I, I, I, B, I],
                     [h("q"), h("k"), h("v"), h("o"), _core.float_bits(scale), sh, ss, seq,
                      h("lse"), seq])
        variants.append(_core.kernel_variant(kern["attn_fwd"]))
        _core.launch(kern["attn_bwd_preprocess"], (1, heads, 1), 128, [B, B, B, I, I, I, I],
                     [h("o"), h("do"), h("delta"), sh, ss, seq, seq])
        variants.append(_core.kernel_variant(kern["attn_bwd_preprocess"]))
        _core.launch(kern["attn_bwd_dq"], (1, heads, 1), 128, [B] * 7 + [F, I, I, I, I],
                     [h(x) for x in ("q", "k", "v", "do", "dq", "lse", "delta")] +
                     [_core.float_bits(scale), sh, ss, seq, seq])
        variants.append(_core.kernel_variant(kern["attn_bwd_dq"]))
        _core.launch(kern["attn_bwd_dkdv"], (1, heads, 1), 128, [B] * 8 + [F, I, I, I, I],
                     [h(x) for x in ("q", "k", "v", "do", "dk", "dv", "lse", "delta")] +
                     [_core.float_bits(scale), sh, ss, seq, seq])
        variants.append(_core.kernel_variant(kern["attn_bwd_dkdv"]))
        out = {k: gather(bufs[k].float32()) for k in ("o", "dq", "dk", "dv")}
        out["lse"] = bufs["lse"].float32()
        out["delta"] = bufs["delta"].float32()
        out["padding"] = [bufs[k].float32() for k in ("o", "dq", "dk", "dv")]
    finally:
        for b in bufs.values():
            b.free()
    return out, variants, dense, (total, sh, ss)


def _check(out, dense, dim, causal, tol=2e-2, element="bf16"):
    q, k, v, d_out = dense
    want = R.attention_backward(q, k, v, d_out, 1 / math.sqrt(dim), causal)
    assert T.max_abs_error(out["o"], want["o"]) <= tol
    assert T.max_abs_error(out["lse"], want["lse"]) <= (2e-3 if element == "f32" else T.lse_bound(element))
    # Delta = rowsum(dO * O) over the O the forward wrote (already rounded to
    # the element type), in fp32: within the summation bound of D products
    o64, do64 = out["o"].astype(np.float64), d_out.astype(np.float64)
    delta_want = np.sum(do64 * o64, -1)
    bound = dim * 2.0 ** -23 * np.sum(np.abs(do64 * o64), -1) + 1e-30
    assert np.all(np.abs(out["delta"] - delta_want) <= bound)
    for name in ("dq", "dk", "dv"):
        assert T.hybrid_error(out[name], want[name]) <= tol, name


@pytest.mark.parametrize("element", ["bf16", "f16"])
@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("seq", [1, 2, 3, 63, 64, 65, 129])
def test_fast_attention_edges(element, dim, causal, seq, device):
    out, variants, dense, _ = _attention(2, seq, dim, element, causal)
    assert all("_fast_" in v for v in variants), variants
    _check(out, dense, dim, causal, element=element)


def _random_attention_cases(count=16, seed=7):
    """Seeded sweep: sequence lengths up to 600, D 64 or 128, causal or not,
    bf16 or f16, rows padded by 0-24 elements (kept 16-byte aligned) and a
    head stride padded by 0-3 rows."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        seq = int(rng.integers(1, 600))
        dim = (64, 128)[i % 2]
        ss = dim + 8 * int(rng.integers(0, 4))
        sh = (seq + int(rng.integers(0, 4))) * ss
        out.append((int(rng.integers(1, 4)), seq, dim, ("bf16", "f16")[(i // 2) % 2], bool(i % 3 == 0),
                    ss, sh))
    return out


@pytest.mark.parametrize("heads,seq,dim,element,causal,ss,sh", _random_attention_cases())
def test_fast_attention_sweep(heads, seq, dim, element, causal, ss, sh, device):
    out, variants, dense, _ = _attention(heads, seq, dim, element, causal, stride_seq=ss,
                                         stride_head=sh, seed=seq)
    assert all("_fast_" in v for v in variants), variants
    _check(out, dense, dim, causal, element=element)


@pytest.mark.parametrize("causal", [False, True])
def test_fast_attention_padded_strides_leave_padding_untouched(causal, device):
    """Rows padded to stride_seq = D + 8 and heads to a padded stride_head: the
    fast kernels run (16-byte aligned rows) and never write the padding."""
    heads, seq, dim = 3, 100, 64
    out, variants, dense, (total, sh, ss) = _attention(heads, seq, dim, "bf16", causal,
                                                        stride_seq=dim + 8,
                                                        stride_head=seq * (dim + 8) + 16)
    assert all("_fast_" in v for v in variants), variants
    _check(out, dense, dim, causal)
    mask = np.ones(total, bool)
    for h in range(heads):
        for i in range(seq):
            mask[h * sh + i * ss: h * sh + i * ss + dim] = False
    for flat in out["padding"]:
        assert np.all(flat[mask] == 0)


@pytest.mark.parametrize("element,dim,stride_seq,expect", [
    ("bf16", 80, 80, "generic"),    # head_dim without a specialised kernel
    ("bf16", 64, 68, "generic"),    # rows not 16-byte aligned
    ("f32", 64, 64, "generic"),     # f32 runs the exact-f32 MFMA kernels
    ("f16", 128, 128, "fast"),
    ("bf16", 64, 72, "fast"),      # padded rows, 16-byte aligned
])
def test_variant_selection(element, dim, stride_seq, expect, device):
    out, variants, dense, _ = _attention(1, 70, dim, element, False, stride_seq=stride_seq)
    assert all(f"_{expect}_" in v for v in variants), variants
    _check(out, dense, dim, False, tol=2e-2 if element != "f32" else 1e-4, element=element)


def _gemm(m, n, k, element, lda=None, ldb=None, ldc=None, seed=0, poison=False, extra_rows=0):
    """C = A B with leading dimensions lda/ldb/ldc.  `poison` fills the padding
    columns of A (k..lda) with inf and of B (n..ldb) with NaN: a kernel that
    lets them reach a stored output element fails.  C gets `extra_rows` rows
    past row m, preset to -7 like its padding columns."""
    lda, ldb, ldc = lda or k, ldb or n, ldc or n
    rng = np.random.default_rng(seed)
    a = round_to(rng.standard_normal((m, lda), dtype=np.float32), element)
    b = round_to(rng.standard_normal((k, ldb), dtype=np.float32), element)
    if poison:
        a[:, k:] = np.inf
        b[:, n:] = np.nan
    dtype = DT[element]
    A = DeviceBuffer.from_numpy(a, dtype)
    B = DeviceBuffer.from_numpy(b, dtype)
    C = DeviceBuffer.from_numpy(np.full((m + extra_rows, ldc), -7.0, np.float32), dtype)
    kern = ops.library(element).kernels["matmul_kernel"]
    try:
        grid, kinds, values = ops.matmul_args(A, B, C, m, n, k, (lda, 1, ldb, 1, ldc, 1))
        _core.launch(kern, grid, 128, kinds, values)
        variant = _core.kernel_variant(kern)
        c = C.float32()
    finally:
        for x in (A, B, C):
            x.free()
    want = a[:, :k].astype(np.float64) @ b[:, :n].astype(np.float64)
    return c, want, variant


def _tile_suffix(m, n, cus=256, k=None):
    """The planner's tile choice on an MI355X (256 compute units): rounds of
    resident 256 x 256 tiles (one per CU) at 31 against rounds of 128 x 128
    pairs (two per CU) at 21; with fewer 128 x 128 tiles than CUs, 64 x 64
    tiles ("_t64").  Given k >= 128 (whole row-major tiles only), the K loop
    is split over wave groups: 128 x 128 tiles fewer than two per CU over 2
    ("_k2"); 64 x 64 tiles over 4 ("_k4") up to one per CU, over 2 ("_k2")
    up to two."""
    cd = lambda a, b: -(-a // b)
    big = cd(cd(m, 256) * cd(n, 256), cus) * 31 <= cd(cd(m, 128) * cd(n, 128), 2 * cus) * 21
    if big:
        return ""
    small = cd(m, 128) * cd(n, 128) < cus
    tile = 64 if small else 128
    suffix = "_t64" if small else "_t128"
    tiles = cd(m, tile) * cd(n, tile)
    if k is not None and k >= 128:
        if small and tiles <= cus:
            suffix += "_k4"
        elif small and tiles <= 2 * cus or not small and tiles < 2 * cus:
            suffix += "_k2"
    return suffix
@pytest.mark.parametrize("element", ["bf16", "f16"])
@pytest.mark.parametrize("m,n,k,lda,ldb,ldc,tile", [
    (256, 512, 64, None, None, None, "_t64"),
    (512, 256, 192, None, None, None, "_t64_k4"),   # 3 k-steps over 4 wave groups
    (768, 1024, 320, 328, 1032, 1040, "_t64_k4"),  # padded leading dimensions, 16-byte aligned
    (256, 8192, 256, None, None, None, "_t64_k2"),  # 512 tiles of 64 x 64: two per CU
    (2048, 2048, 64, None, None, None, "_t128"),
    (2560, 2048, 128, 136, 2056, 2052, "_t128_k2"),
    (2048, 2048, 2048, None, None, None, "_t128_k2"),
    (1024, 1024, 1024, None, None, None, "_t64_k4"),
    (4096, 4096, 128, None, None, None, ""),
    (4096, 4096, 64, 72, 4104, 4100, ""),
])
def test_fast_gemm_shapes_and_strides(element, m, n, k, lda, ldb, ldc, tile, device):
    c, want, variant = _gemm(m, n, k, element, lda, ldb, ldc)
    assert tile == _tile_suffix(m, n, k=k)
    # whole row-major 256 x 256 tiles run the 4-wave kernel
    assert variant == (f"tm_gemm_w4_{element}" if tile == "" else f"tm_gemm_fast{tile}_{element}")
    assert T.hybrid_error(c[:, :n], want) <= 2e-2
    if ldc:
        assert np.all(c[:, n:] == -7.0)


@pytest.mark.parametrize("element", ["bf16", "f16"])
@pytest.mark.parametrize("m,n,k,lda,ldb,ldc", [
    (255, 256, 64, None, None, None),    # M short of a tile
    (256, 264, 64, None, None, None),    # N one chunk past a tile
    (256, 256, 72, None, None, None),    # K past the last whole k-step
    (129, 257, 65, 72, 264, 260),        # the reference's ragged shape (DotTests), padded rows
    (1, 1, 1, 8, 8, 4),                  # one element
    (300, 1000, 136, None, None, None),
    (513, 777, 1000, 1000, 784, 780),
    (4000, 4100, 200, 200, 4104, 4100),  # 272 tiles of 256 x 256
    (4096, 4096, 72, None, None, None),  # whole 256 x 256 tiles, ragged K
    (2000, 2100, 72, None, 2104, 2100),  # 128 x 128 tiles
])
def test_ragged_gemm(element, m, n, k, lda, ldb, ldc, device):
    """Any M, N, K with 16-byte aligned rows of A and B run the ragged
    specialised kernel: masked to the matrix, with inf/NaN in the operands'
    padding and sentinel rows and columns around C."""
    c, want, variant = _gemm(m, n, k, element, lda, ldb, ldc, poison=True, extra_rows=3)
    tile = _tile_suffix(m, n)
    # the main dispatch (64 x 64 tiles that leave the chip idle run with K
    # ranges, "_ks", and a reduce dispatch)
    assert variant.split(" + ")[0] in (f"tm_gemm_ragged{tile}_{element}",
                                       f"tm_gemm_ragged{tile}_ks_{element}")
    assert np.all(np.isfinite(c[:m, :n]))
    assert T.hybrid_error(c[:m, :n], want) <= 2e-2
    assert np.all(c[:m, n:] == -7.0) and np.all(c[m:] == -7.0)


@pytest.mark.parametrize("element", ["bf16", "f16"])
@pytest.mark.parametrize("m,n,k,lda,ldb,ldc,main,ranges", [
    (16, 1024, 4096, None, None, None, "tm_gemm_ragged_t64", 16),     # a few rows, long K
    (64, 2048, 8192, None, None, None, "tm_gemm_fast_t64_k4", 8),     # whole tiles, K groups too
    (512, 512, 8192, 8200, 520, 516, "tm_gemm_fast_t64_k4", 4),       # padded rows
    (100, 300, 1000, 1000, 304, 300, "tm_gemm_ragged_t64", 8),        # ragged M, N and K
    (1, 8, 8192, 8192, 8, 8, "tm_gemm_ragged_t64", 16),               # one row
    (64, 64, 65536, None, None, None, "tm_gemm_fast_t64_k4", 16),     # one tile, K of 1024 steps
    (1, 1, 65536, 65536, 8, 4, "tm_gemm_ragged_t64", 16),             # one element, long K
])
def test_gemm_k_ranges(element, m, n, k, lda, ldb, ldc, main, ranges, device):
    """64 x 64-tile problems with too few tiles to fill the chip split K
    across workgroups: each range writes an fp32 partial and a reduce
    dispatch sums them into C (operand padding poisoned, C fenced with
    sentinels)."""
    c, want, variant = _gemm(m, n, k, element, lda, ldb, ldc, poison=True, extra_rows=3)
    assert variant == (f"{main}_ks_{element} + tm_gemm_split_reduce_{element} ({ranges} K ranges)")
    assert np.all(np.isfinite(c[:m, :n]))
    assert T.hybrid_error(c[:m, :n], want) <= 2e-2
    assert np.all(c[:m, n:] == -7.0) and np.all(c[m:] == -7.0)


def test_gemm_k_ranges_queued_back_to_back(device):
    """Three K-range GEMMs queued without waiting, each needing more work
    memory than the last (the library grows its workspace between them, after
    the queued dispatches drain), then one synchronize: every result is
    right."""
    kern = ops.library("bf16").kernels["matmul_kernel"]
    rng = np.random.default_rng(11)
    shapes = ((16, 256, 4096), (64, 1024, 4096), (200, 2000, 3000))
    bufs, wants = [], []
    try:
        for m, n, k in shapes:
            a = round_to(rng.standard_normal((m, k), dtype=np.float32), "bf16")
            b = round_to(rng.standard_normal((k, n), dtype=np.float32), "bf16")
            A, B = DeviceBuffer.from_numpy(a, "bfloat16"), DeviceBuffer.from_numpy(b, "bfloat16")
            C = DeviceBuffer.from_numpy(np.full((m, n), -7.0, np.float32), "bfloat16")
            bufs.append((A, B, C))
            wants.append(a.astype(np.float64) @ b.astype(np.float64))
        for (m, n, k), (A, B, C) in zip(shapes, bufs):
            grid, kinds, values = ops.matmul_args(A, B, C, m, n, k)
            _core.launch_async(kern, grid, 128, kinds, values)
            assert "K ranges" in _core.kernel_variant(kern), _core.kernel_variant(kern)
        _core.synchronize()
        for (A, B, C), want in zip(bufs, wants):
            assert T.hybrid_error(C.float32(), want) <= 2e-2
    finally:
        for trio in bufs:
            for x in trio:
                x.free()


def _gemm_nt(m, n, k, element, lda=None, ldbt=None, ldc=None, seed=0):
    """C = A B with B stored transposed (bt[n, k], row stride ldbt: the
    x @ W^T layout); the padding columns of A and of B^T hold inf, and C is
    fenced with -7 sentinels like _gemm's."""
    lda, ldbt, ldc = lda or k, ldbt or k, ldc or n
    rng = np.random.default_rng(seed)
    a = round_to(rng.standard_normal((m, lda), dtype=np.float32), element)
    bt = round_to(rng.standard_normal((n, ldbt), dtype=np.float32), element)
    a[:, k:] = np.inf
    bt[:, k:] = np.inf
    dtype = DT[element]
    A = DeviceBuffer.from_numpy(a, dtype)
    B = DeviceBuffer.from_numpy(bt, dtype)
    C = DeviceBuffer.from_numpy(np.full((m + 3, ldc), -7.0, np.float32), dtype)
    kern = ops.library(element).kernels["matmul_kernel"]
    try:
        grid, kinds, values = ops.matmul_args(A, B, C, m, n, k, (lda, 1, 1, ldbt, ldc, 1))
        _core.launch(kern, grid, 128, kinds, values)
        variant = _core.kernel_variant(kern)
        c = C.float32()
    finally:
        for x in (A, B, C):
            x.free()
    want = a[:, :k].astype(np.float64) @ bt[:, :k].astype(np.float64).T
    return c, want, variant


@pytest.mark.parametrize("element", ["bf16", "f16"])
@pytest.mark.parametrize("m,n,k,lda,ldbt,ldc,kind", [
    (256, 256, 64, None, None, None, "fast"),
    (4096, 4096, 128, None, None, None, "w4"),
    (129, 257, 65, 72, 72, 260, "ragged"),
    (300, 1000, 136, None, None, None, "ragged"),
    (4000, 4100, 200, 200, 208, 4100, "ragged"),
])
def test_transposed_b_gemm(element, m, n, k, lda, ldbt, ldc, kind, device):
    """B stored transposed (stride_bk = 1) runs the specialised kernels too,
    B's tile copied and read like A's."""
    c, want, variant = _gemm_nt(m, n, k, element, lda, ldbt, ldc)
    assert variant == f"tm_gemm_{kind}_nt{_tile_suffix(m, n)}_{element}"
    assert np.all(np.isfinite(c[:m, :n]))
    assert T.hybrid_error(c[:m, :n], want) <= 2e-2
    assert np.all(c[:m, n:] == -7.0) and np.all(c[m:] == -7.0)


def _gemm_tn(m, n, k, element, ldat=None, ldb=None, ldc=None, seed=0):
    """C = A B with A stored transposed (at[k, m], row stride ldat: the dY^T X
    layout); A^T's padding columns hold inf, and C is fenced with -7."""
    ldat, ldb, ldc = ldat or m, ldb or n, ldc or n
    rng = np.random.default_rng(seed)
    at = round_to(rng.standard_normal((k, ldat), dtype=np.float32), element)
    b = round_to(rng.standard_normal((k, ldb), dtype=np.float32), element)
    at[:, m:] = np.inf
    b[:, n:] = np.nan
    dtype = DT[element]
    A = DeviceBuffer.from_numpy(at, dtype)
    B = DeviceBuffer.from_numpy(b, dtype)
    C = DeviceBuffer.from_numpy(np.full((m + 3, ldc), -7.0, np.float32), dtype)
    kern = ops.library(element).kernels["matmul_kernel"]
    try:
        grid, kinds, values = ops.matmul_args(A, B, C, m, n, k, (1, ldat, ldb, 1, ldc, 1))
        _core.launch(kern, grid, 128, kinds, values)
        variant = _core.kernel_variant(kern)
        c = C.float32()
    finally:
        for x in (A, B, C):
            x.free()
    want = at[:, :m].astype(np.float64).T @ b[:, :n].astype(np.float64)
    return c, want, variant


@pytest.mark.parametrize("element", ["bf16", "f16"])
@pytest.mark.parametrize("m,n,k,ldat,ldb,ldc,kind", [
    (256, 256, 64, None, None, None, "fast"),
    (4096, 4096, 128, None, None, None, "w4"),
    (129, 257, 65, 136, 264, 260, "ragged"),
    (1000, 300, 136, None, 304, None, "ragged"),
    (4100, 4000, 200, 4104, 4000, 4000, "ragged"),
])
def test_transposed_a_gemm(element, m, n, k, ldat, ldb, ldc, kind, device):
    """A stored transposed (stride_am = 1) runs the specialised kernels too,
    A's tile copied and read like B's."""
    c, want, variant = _gemm_tn(m, n, k, element, ldat, ldb, ldc)
    assert variant == f"tm_gemm_{kind}_tn{_tile_suffix(m, n)}_{element}"
    assert np.all(np.isfinite(c[:m, :n]))
    assert T.hybrid_error(c[:m, :n], want) <= 2e-2
    assert np.all(c[:m, n:] == -7.0) and np.all(c[m:] == -7.0)


def _random_gemm_cases(count=36, seed=123):
    """Seeded shapes for the layout sweep: M, N, K up to 700, each operand
    row-major or (one of them) transposed, leading dimensions padded by 0-16
    elements to a multiple of 8."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        m, n, k = (int(x) for x in rng.integers(1, 700, 3))
        layout = ("nn", "nt", "tn")[i % 3]
        pad = lambda x: -(-(x + int(rng.integers(0, 17))) // 8) * 8
        cases.append((m, n, k, layout, pad, ("bf16", "f16")[i % 2]))
    return [(m, n, k, layout, pad(k), pad(n), pad(m), el) for m, n, k, layout, pad, el in cases]


def _random_k_range_cases(count=18, seed=7):
    """Seeded shapes that take K ranges: M and N up to 300 (few 64 x 64
    tiles), K from 1000 to 6000, every layout, padded leading dimensions."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        m, n = (int(x) for x in rng.integers(1, 300, 2))
        k = int(rng.integers(1000, 6000))
        pad = lambda x: -(-(x + int(rng.integers(0, 17))) // 8) * 8
        out.append((m, n, k, ("nn", "nt", "tn")[i % 3], pad(k), pad(n), pad(m), ("bf16", "f16")[i % 2]))
    return out


@pytest.mark.parametrize("m,n,k,layout,pk,pn,pm,element", _random_k_range_cases())
def test_gemm_k_range_sweep(m, n, k, layout, pk, pn, pm, element, device):
    """Seeded small-M-N, long-K shapes: every one runs K ranges across
    workgroups and a reduce, against fp64 with inf/NaN in the padding."""
    if layout == "nn":
        c, want, variant = _gemm(m, n, k, element, pk, pn, pn, poison=True, extra_rows=3)
    elif layout == "nt":
        c, want, variant = _gemm_nt(m, n, k, element, pk, pk, pn)
    else:
        c, want, variant = _gemm_tn(m, n, k, element, pm, pn, pn)
    assert "_ks_" in variant and "K ranges" in variant, variant
    assert np.all(np.isfinite(c[:m, :n]))
    assert T.hybrid_error(c[:m, :n], want) <= 2e-2
    assert np.all(c[:m, n:] == -7.0) and np.all(c[m:] == -7.0)


@pytest.mark.parametrize("m,n,k,layout,pk,pn,pm,element", _random_gemm_cases())
def test_gemm_layout_sweep(m, n, k, layout, pk, pn, pm, element, device):
    """Seeded random shapes and layouts through the specialised kernels,
    each against fp64 with inf/NaN in every operand's padding."""
    if layout == "nn":
        c, want, variant = _gemm(m, n, k, element, pk, pn, pn, poison=True, extra_rows=3)
    elif layout == "nt":
        c, want, variant = _gemm_nt(m, n, k, element, pk, pk, pn)
    else:
        c, want, variant = _gemm_tn(m, n, k, element, pm, pn, pn)
    assert "generic" not in variant, variant
    assert np.all(np.isfinite(c[:m, :n]))
    assert T.hybrid_error(c[:m, :n], want) <= 2e-2
    assert np.all(c[:m, n:] == -7.0) and np.all(c[m:] == -7.0)


@pytest.mark.parametrize("m,n,k,lda,ldb,variant", [
    (256, 256, 60, None, None, "generic"),    # rows of A not 16-byte aligned
    (300, 200, 100, None, None, "generic"),
    (255, 256, 64, None, None, "ragged_t64"),
    (512, 256, 128, None, None, "fast_t64_k4"),
    (2048, 2048, 64, None, None, "fast_t128"),
    (2000, 2100, 72, None, 2104, "ragged_t128"),
    (4096, 4096, 64, None, None, "w4"),
])
def test_gemm_kernel_choice(m, n, k, lda, ldb, variant, device):
    c, want, got = _gemm(m, n, k, "bf16", lda, ldb)
    assert got == f"tm_gemm_{variant}_bf16"
    assert T.hybrid_error(c[:, :n], want) <= 2e-2


@pytest.mark.parametrize("seq,expect", [(1024, "fast"), (1025, "generic")])
def test_head_span_at_the_buffer_resource_limit(seq, expect, device):
    """The fast kernels copy tiles through a buffer resource based at a head's
    first row, so a head whose rows span 2^31 bytes or more takes the generic
    kernel.  Rows 2 MiB apart put the boundary between 1024 rows (2^31 - 2 MiB
    + 128 bytes: fast, with 32-bit lane offsets up to 2^31 - 2 MiB) and 1025
    rows (2^31 + 128 bytes: generic).  Only the rows themselves are written and
    read back; the buffers (about 2 GiB each) are never touched elsewhere."""
    from triton_metal.buffer import bf16_bits, bf16_values
    dim, ss = 64, 1 << 20
    extent = (seq - 1) * ss + dim
    rng = np.random.default_rng(7)
    dense = [round_to(rng.standard_normal((1, seq, dim), dtype=np.float32), "bf16")
             for _ in range(3)]
    handles = [_core.alloc_buffer(extent * 2) for _ in range(4)]
    lse = DeviceBuffer((1, seq), "float32")
    try:
        for handle, x in zip(handles, dense):
            bits = bf16_bits(x[0])
            for i in range(seq):
                row = np.ascontiguousarray(bits[i])
                _core.buffer_write(handle, i * ss * 2, row.ctypes.data, dim * 2)
        kern = ops.library("bf16", dim, False).kernels["attn_fwd"]
        B, I, F = _core.ARG_BUFFER, _core.ARG_I32, _core.ARG_F32
        _core.launch(kern, (1, 1, 1), 128, [B, B, B, B, F, I, I, I, B, I],
                     handles + [_core.float_bits(1 / math.sqrt(dim)), seq * ss, ss, seq,
                                lse.tm_handle, seq])
        variant = _core.kernel_variant(kern)
        o_bits = np.zeros((seq, dim), np.uint16)
        for i in range(seq):
            _core.buffer_read(handles[3], i * ss * 2, o_bits[i].ctypes.data, dim * 2)
        o = bf16_values(o_bits)[None]
        lse_got = lse.float32()
    finally:
        for handle in handles:
            _core.free_buffer(handle)
        lse.free()
    assert f"_{expect}_" in variant, variant
    q, k, v = dense
    o_want, _, lse_want = R.attention_forward(q, k, v, 1 / math.sqrt(dim), False)
    assert T.max_abs_error(o, o_want) <= 2e-2
    assert T.max_abs_error(lse_got, lse_want) <= 2e-3


@pytest.mark.parametrize("element", ["bf16", "f16"])
@pytest.mark.parametrize("m,n,k,lda,ldb,ldc", [
    (4096, 4096, 64, None, None, None),        # one K step: no copy of a next step
    (4096, 4096, 128, None, None, None),       # two steps: each stage buffer once
    (4096, 4608, 192, None, None, None),       # odd step count; 16 x 18 tiles
    (5120, 4096, 1024, 1032, 4104, 4100),      # padded, poisoned leading dimensions
    (8192, 4096, 320, None, None, None),
])
def test_four_wave_gemm(element, m, n, k, lda, ldb, ldc, device):
    """The 4-wave 256 x 256-tile kernel (whole row-major tiles, K a multiple of
    64): every element against fp64, padding columns of A and B poisoned
    (inf, NaN) so a read past K or N reaches an output, C's padding and extra
    rows untouched."""
    c, want, variant = _gemm(m, n, k, element, lda, ldb, ldc, seed=k, poison=lda is not None,
                             extra_rows=8)
    assert variant == f"tm_gemm_w4_{element}"
    assert np.all(np.isfinite(c[:m, :n]))
    assert T.hybrid_error(c[:m, :n], want) <= 2e-2
    assert np.all(c[:m, n:] == -7.0) and np.all(c[m:] == -7.0)


@pytest.mark.parametrize("element", ["bf16", "f16"])
@pytest.mark.parametrize("layout,m,n,k,lda,ldb,ldc", [
    ("nt", 4096, 4096, 64, None, None, None),    # one K step
    ("nt", 4096, 4608, 192, None, None, None),   # odd step count, 16 x 18 tiles
    ("nt", 5120, 4096, 1024, 1032, 1040, 4100),  # padded, poisoned leading dimensions
    ("tn", 4096, 4096, 64, None, None, None),
    ("tn", 4608, 4096, 192, None, None, None),
    ("tn", 4096, 5120, 1024, 4104, 5128, 5124),
])
def test_four_wave_gemm_transposed(element, layout, m, n, k, lda, ldb, ldc, device):
    """The 4-wave kernel with B stored transposed (both operands K-contiguous,
    read by ds_read_b128) or A stored transposed (both read transposed):
    every element against fp64, operand padding poisoned, C's padding and
    extra rows untouched."""
    if layout == "nt":
        c, want, variant = _gemm_nt(m, n, k, element, lda, ldb, ldc, seed=k)
    else:
        c, want, variant = _gemm_tn(m, n, k, element, lda, ldb, ldc, seed=k)
    assert variant == f"tm_gemm_w4_{layout}_{element}"
    assert np.all(np.isfinite(c[:m, :n]))
    assert T.hybrid_error(c[:m, :n], want) <= 2e-2
    assert np.all(c[:m, n:] == -7.0) and np.all(c[m:] == -7.0)


@pytest.mark.parametrize("operand,stride,expect", [
    ("b", 16777208, "w4"),    # B row-major: 64 rows at this stride span just under 2^31 bytes
    ("b", 16777216, "fast"),  # one 8-element step further: past the 32-bit range
    ("a", 4194296, "w4"),     # A row-major: 256 rows at this stride span just under 2^31 bytes
    ("a", 4194304, "fast"),
])
def test_four_wave_gemm_buffer_range_limit(operand, stride, expect, device):
    """The 4-wave kernel addresses a step's tile of each operand through one
    buffer resource with 32-bit offsets: 256 stored rows of a K-contiguous
    operand (A row-major), 64 of the other kind (B row-major).  At the largest
    row stride whose offsets and range stay below 2^31 bytes the planner takes
    it, and every element is right; one step further it takes the 8-wave
    kernel, whose copies use 64-bit addresses.  Only the rows the GEMM reads
    are written (the A buffers span about 34 GB, the B buffers 2 GB)."""
    from triton_metal.buffer import bf16_bits
    m = n = 4096
    k = 64
    rng = np.random.default_rng(stride)
    a = round_to(rng.standard_normal((m, k), dtype=np.float32), "bf16")
    b = round_to(rng.standard_normal((k, n), dtype=np.float32), "bf16")
    lda, ldb = (stride, n) if operand == "a" else (k, stride)
    rows, ld, dense = (m, lda, a) if operand == "a" else (k, ldb, b)
    strided = _core.alloc_buffer(((rows - 1) * ld + dense.shape[1]) * 2)
    other = DeviceBuffer.from_numpy(b if operand == "a" else a, "bfloat16")
    c = DeviceBuffer((m, n), "bfloat16")
    try:
        bits = bf16_bits(dense)
        for i in range(rows):
            row = np.ascontiguousarray(bits[i])
            _core.buffer_write(strided, i * ld * 2, row.ctypes.data, row.nbytes)
        ha, hb = (strided, other.tm_handle) if operand == "a" else (other.tm_handle, strided)
        kern = ops.library("bf16").kernels["matmul_kernel"]
        kinds = [_core.ARG_BUFFER] * 3 + [_core.ARG_I32] * 9
        _core.launch(kern, (m // 64, n // 64, 1), 128, kinds,
                     [ha, hb, c.tm_handle, m, n, k, lda, 1, ldb, 1, n, 1])
        variant = _core.kernel_variant(kern)
        got = c.float32()
    finally:
        _core.free_buffer(strided)
        other.free()
        c.free()
    assert variant == f"tm_gemm_{expect}_bf16"
    want = a.astype(np.float64) @ b.astype(np.float64)
    assert T.hybrid_error(got, want) <= 2e-2
