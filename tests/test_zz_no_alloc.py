"""tm_launch_noalloc, the launch that allocates nothing: its dispatches take
their work buffer (attn_bwd_fused's fp32 dQ accumulator) from a static device
array instead of library-owned memory.  Checked against tm_launch on the same
inputs, two calls in a row with the second smaller (the array keeps the first
call's contents, so a missing clear would show), a request larger than the
array refused before anything runs, a built-in with no work buffer, and the
generic kernels' range split and the GEMM's K ranges, whose partials also
come from the array."""

import ctypes
import math

import numpy as np
import pytest

from oracle import reference as R
from oracle import tolerance as T
from triton_metal import _core, ops
from triton_metal.buffer import DeviceBuffer, round_to

pytestmark = pytest.mark.gpu

B, I, F = _core.ARG_BUFFER, _core.ARG_I32, _core.ARG_F32
SCRATCH_BYTES = 64 << 20


def _raw_launch(entry, kernel, grid, kinds, values):
    """Call a launch entry point of the C ABI directly."""
    n = len(kinds)
    return getattr(_core._lib, entry)(kernel, grid[0], grid[1], grid[2], 128,
                                      (ctypes.c_int32 * n)(*kinds), (ctypes.c_int64 * n)(*values), n)


class _Problem:
    def __init__(self, heads, seq, dim, seed):
        self.heads, self.seq, self.dim = heads, seq, dim
        rng = np.random.default_rng(seed)
        self.inputs = [round_to(rng.standard_normal((heads, seq, dim), dtype=np.float32), "bf16")
                       for _ in range(4)]
        self.bufs = {k: DeviceBuffer.from_numpy(x, "bfloat16")
                     for k, x in zip(("q", "k", "v", "do"), self.inputs)}
        for k in ("o", "dq", "dk", "dv"):
            self.bufs[k] = DeviceBuffer((heads, seq, dim), "bfloat16")
        self.bufs["lse"] = DeviceBuffer((heads, seq), "float32")
        self.bufs["delta"] = DeviceBuffer((heads, seq), "float32")
        self.scale = 1 / math.sqrt(dim)
        self.lib = ops.library("bf16", dim, True, bwd="atomic")
        self.tail = [_core.float_bits(self.scale), seq * dim, dim, seq, seq]
        kern = self.lib.kernels
        _core.launch(kern["attn_fwd"], (1, heads, 1), 128, [B, B, B, B, F, I, I, I, B, I],
                     [self.h("q"), self.h("k"), self.h("v"), self.h("o"),
                      _core.float_bits(self.scale), seq * dim, dim, seq, self.h("lse"), seq])
        _core.launch(kern["attn_bwd_preprocess"], (1, heads, 1), 128, [B, B, B, I, I, I, I],
                     [self.h("o"), self.h("do"), self.h("delta"), seq * dim, dim, seq, seq])

    def h(self, name):
        return self.bufs[name].tm_handle

    def fused(self, entry):
        kern = self.lib.kernels["attn_bwd_fused"]
        for k in ("dq", "dk", "dv"):
            self.bufs[k].write(np.zeros((self.heads, self.seq, self.dim), np.float32))
        rc = _raw_launch(entry, kern, (1, self.heads, 1), [B] * 9 + [F, I, I, I, I],
                         [self.h(x) for x in ("q", "k", "v", "do", "dq", "dk", "dv", "lse",
                                              "delta")] + self.tail)
        assert rc == 0, _core.last_error()
        assert "tm_attn_fused_fast_" in _core.kernel_variant(kern)
        return {k: self.bufs[k].float32() for k in ("dq", "dk", "dv")}

    def free(self):
        for b in self.bufs.values():
            b.free()


def test_noalloc_fused_backward_matches_tm_launch_twice(device):
    # the first call fills 3 MiB of the array; the second, smaller one must
    # not see its leftovers
    for heads, seq, dim in ((6, 1024, 128), (2, 300, 64)):
        print(f"noalloc fused backward heads={heads} seq={seq} dim={dim}", flush=True)
        p = _Problem(heads, seq, dim, seed=heads * seq)
        try:
            want = p.fused("tm_launch")
            got = p.fused("tm_launch_noalloc")
        finally:
            p.free()
        assert np.array_equal(got["dk"], want["dk"])
        assert np.array_equal(got["dv"], want["dv"])
        # dQ: the same partials summed by atomics in another order
        assert T.hybrid_error(got["dq"], want["dq"]) <= 2 * T.U_BF16
        q, k, v, d_out = p.inputs
        ref = R.attention_backward(q, k, v, d_out, p.scale, True)
        assert T.hybrid_error(got["dq"], ref["dq"]) <= 2e-2


def test_noalloc_refuses_an_accumulator_larger_than_the_array(device):
    # 9 * 16384 * 128 * 4 bytes = 72 MiB of accumulator
    heads, seq, dim = 9, 16384, 128
    assert heads * seq * dim * 4 > SCRATCH_BYTES
    lib = ops.library("bf16", dim, True, bwd="atomic")
    kern = lib.kernels["attn_bwd_fused"]
    bufs = [DeviceBuffer((heads, seq, dim), "bfloat16") for _ in range(7)]
    stats = [DeviceBuffer((heads, seq), "float32") for _ in range(2)]
    try:
        rc = _raw_launch("tm_launch_noalloc", kern, (1, heads, 1), [B] * 9 + [F, I, I, I, I],
                         [b.tm_handle for b in bufs + stats] +
                         [_core.float_bits(1 / math.sqrt(dim)), seq * dim, dim, seq, seq])
        assert rc == -1
        assert "static scratch holds 67108864 bytes" in _core.last_error()
    finally:
        for b in bufs + stats:
            b.free()


def test_noalloc_runs_kernels_without_a_work_buffer(device):
    """A dispatch with no work buffer (the GEMM) runs the same device function
    with the same result through either entry point."""
    n = 256
    rng = np.random.default_rng(3)
    a = DeviceBuffer.from_numpy(round_to(rng.standard_normal((n, n), dtype=np.float32), "bf16"),
                                "bfloat16")
    b = DeviceBuffer.from_numpy(round_to(rng.standard_normal((n, n), dtype=np.float32), "bf16"),
                                "bfloat16")
    c1, c2 = DeviceBuffer((n, n), "bfloat16"), DeviceBuffer((n, n), "bfloat16")
    lib = ops.library("bf16", 64, False)
    mm = lib.kernels["matmul_kernel"]
    try:
        for entry, c in (("tm_launch", c1), ("tm_launch_noalloc", c2)):
            grid, kinds, values = ops.matmul_args(a, b, c, n, n, n)
            assert _raw_launch(entry, mm, grid, kinds, values) == 0, _core.last_error()
        assert np.array_equal(c1.float32(), c2.float32())
    finally:
        for x in (a, b, c1, c2):
            x.free()


def test_noalloc_range_split_matches_tm_launch_twice(device):
    """The generic kernels' range split (small fp32 grids) takes its partials
    from the static array too: forward, dq and dkdv through either entry
    point, two problems in a row with the second smaller, give the same
    answers bit for bit (the same dispatches over the same inputs)."""
    for heads, seq, dim in ((2, 700, 64), (1, 300, 32)):
        print(f"noalloc range split heads={heads} seq={seq} dim={dim}", flush=True)
        rng = np.random.default_rng(seq)
        layer = ops.AttentionLayer(heads, seq, dim, "f32", causal=True)
        try:
            for name in ("q", "k", "v", "do"):
                layer.upload(name, rng.standard_normal((heads, seq, dim), dtype=np.float32))
            kern = layer.lib.kernels
            results = {}
            for entry in ("tm_launch", "tm_launch_noalloc"):
                out = {}
                for name, (grid, kinds, values), reads in (
                        ("attn_fwd", layer.fwd_args(True), ("o", "lse")),
                        ("attn_bwd_preprocess", layer.pre_args(), ("delta",)),
                        ("attn_bwd_dq", layer.dq_args(), ("dq",)),
                        ("attn_bwd_dkdv", layer.dkdv_args(), ("dk", "dv"))):
                    for r in reads:
                        layer.buffers[r].write(np.full(layer.buffers[r].shape, 5.0, np.float32))
                    assert _raw_launch(entry, kern[name], grid, kinds, values) == 0, _core.last_error()
                    if name != "attn_bwd_preprocess":
                        assert "ranges" in _core.kernel_variant(kern[name]), _core.kernel_variant(kern[name])
                    out.update({r: layer.read(r) for r in reads})
                results[entry] = out
            for r, want in results["tm_launch"].items():
                assert np.array_equal(results["tm_launch_noalloc"][r], want), r
            q, k, v, d_out = (layer.read(x) for x in ("q", "k", "v", "do"))
            want_o, _, _ = R.attention_forward(q, k, v, layer.scale, True)
            assert T.hybrid_error(results["tm_launch_noalloc"]["o"], want_o) <= 2e-5
        finally:
            layer.free()


def test_noalloc_gemm_k_ranges_match_tm_launch_twice(device):
    """A GEMM with too few 64 x 64 tiles to fill the chip runs K ranges whose
    fp32 partials come from the static array: either entry point gives the
    same bits, two problems in a row with the second smaller."""
    lib = ops.library("bf16", 64, False)
    mm = lib.kernels["matmul_kernel"]
    for m, n, k in ((64, 2048, 8192), (16, 1000, 4096)):
        print(f"noalloc gemm K ranges m={m} n={n} k={k}", flush=True)
        rng = np.random.default_rng(m + k)
        a = DeviceBuffer.from_numpy(round_to(rng.standard_normal((m, k), dtype=np.float32), "bf16"),
                                    "bfloat16")
        b = DeviceBuffer.from_numpy(round_to(rng.standard_normal((k, n), dtype=np.float32), "bf16"),
                                    "bfloat16")
        c1, c2 = DeviceBuffer((m, n), "bfloat16"), DeviceBuffer((m, n), "bfloat16")
        try:
            for entry, c in (("tm_launch", c1), ("tm_launch_noalloc", c2)):
                c.write(np.full((m, n), 5.0, np.float32))
                grid, kinds, values = ops.matmul_args(a, b, c, m, n, k)
                assert _raw_launch(entry, mm, grid, kinds, values) == 0, _core.last_error()
                assert "K ranges" in _core.kernel_variant(mm), _core.kernel_variant(mm)
            got, want = c2.float32(), c1.float32()
            assert np.array_equal(got, want)
            ref = a.float32().astype(np.float64) @ b.float32().astype(np.float64)
            assert T.hybrid_error(got, ref) <= 2e-2
        finally:
            for x in (a, b, c1, c2):
                x.free()
