"""The opt-in backward in one call (kernel attn_bwd_fused, bwd=atomic): dK
and dV from the same arithmetic as attn_bwd_dkdv, dQ accumulated across key
blocks with fp32 atomics.

The reference chose the split backward for determinism and named the atomic
form as the unmeasured alternative (AttentionBackwardKernel.swift:27-41,
docs/COMPARISON.md:151-154); its backward tests set the bar used here
(AttentionBackwardTests.swift: hybrid error against an fp64 oracle).

Checks: parity with the fp64 oracle at small and ragged shapes, dK/dV
bit-identical to the split kernels (the same per-block arithmetic), dQ of two
runs within one rounding unit of each other, and, at the headline causal shape (B4 H32 S4096 D128) in
full, dK/dV identical to and dQ within the parity tolerance of the split
path."""

import math

import numpy as np
import pytest

from oracle import reference as R
from oracle import tolerance as T
from triton_metal import _core, ops
from triton_metal.buffer import DeviceBuffer, round_to

pytestmark = pytest.mark.gpu

DT = {"f16": "float16", "bf16": "bfloat16"}
B, I, F = _core.ARG_BUFFER, _core.ARG_I32, _core.ARG_F32


class _Run:
    """Q, K, V, dO uploaded once; forward, then the split and/or fused backward."""

    def __init__(self, heads, seq, dim, element, causal, seed=0, inputs=None, bwd="atomic"):
        self.heads, self.seq, self.dim = heads, seq, dim
        self.element, self.causal = element, causal
        if inputs is None:
            rng = np.random.default_rng(seed)
            inputs = [round_to(rng.standard_normal((heads, seq, dim), dtype=np.float32), element)
                      for _ in range(4)]
        self.inputs = inputs
        dtype = DT[element]
        self.bufs = {k: DeviceBuffer.from_numpy(x, dtype)
                     for k, x in zip(("q", "k", "v", "do"), inputs)}
        for k in ("o", "dq", "dk", "dv"):
            self.bufs[k] = DeviceBuffer((heads, seq, dim), dtype)
        self.bufs["lse"] = DeviceBuffer((heads, seq), "float32")
        self.bufs["delta"] = DeviceBuffer((heads, seq), "float32")
        self.scale = 1 / math.sqrt(dim)
        self.split = ops.library(element, dim, causal)
        self.fused_lib = ops.library(element, dim, causal, bwd=bwd)
        self.bwd = bwd
        sh, ss = seq * dim, dim
        self.tail = [_core.float_bits(self.scale), sh, ss, seq, seq]
        kern = self.split.kernels
        _core.launch(kern["attn_fwd"], (1, heads, 1), 128, [B, B, B, B, F, I, I, I, B, I],
                     [self.h("q"), self.h("k"), self.h("v"), self.h("o"),
                      _core.float_bits(self.scale), sh, ss, seq, self.h("lse"), seq])
        _core.launch(kern["attn_bwd_preprocess"], (1, heads, 1), 128, [B, B, B, I, I, I, I],
                     [self.h("o"), self.h("do"), self.h("delta"), sh, ss, seq, seq])

    def h(self, name):
        return self.bufs[name].tm_handle

    def grads(self):
        return {k: self.bufs[k].float32() for k in ("dq", "dk", "dv")}

    def run_split(self):
        kern = self.split.kernels
        _core.launch(kern["attn_bwd_dq"], (1, self.heads, 1), 128, [B] * 7 + [F, I, I, I, I],
                     [self.h(x) for x in ("q", "k", "v", "do", "dq", "lse", "delta")] + self.tail)
        _core.launch(kern["attn_bwd_dkdv"], (1, self.heads, 1), 128, [B] * 8 + [F, I, I, I, I],
                     [self.h(x) for x in ("q", "k", "v", "do", "dk", "dv", "lse", "delta")] +
                     self.tail)
        return self.grads()

    def run_fused(self):
        kern = self.fused_lib.kernels["attn_bwd_fused"]
        _core.launch(kern, (1, self.heads, 1), 128, [B] * 9 + [F, I, I, I, I],
                     [self.h(x) for x in ("q", "k", "v", "do", "dq", "dk", "dv", "lse", "delta")] +
                     self.tail)
        assert "tm_attn_fused_fast_" in _core.kernel_variant(kern)
        return self.grads()

    def free(self):
        for b in self.bufs.values():
            b.free()


BWD = ["atomic"]


@pytest.mark.parametrize("bwd", BWD)
@pytest.mark.parametrize("element", ["bf16", "f16"])
@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("seq", [1, 3, 65, 129, 300])
def test_fused_backward_matches_oracle(bwd, element, dim, causal, seq, device):
    run = _Run(2, seq, dim, element, causal, seed=seq, bwd=bwd)
    try:
        fused = run.run_fused()
        split = run.run_split()
    finally:
        run.free()
    q, k, v, d_out = run.inputs
    want = R.attention_backward(q, k, v, d_out, run.scale, causal)
    for name in ("dq", "dk", "dv"):
        assert T.hybrid_error(fused[name], want[name]) <= 2e-2, name
    # dK and dV: the fused kernel is the dK/dV kernel plus dQ work; its
    # per-block arithmetic and accumulation order are the same
    assert np.array_equal(fused["dk"], split["dk"])
    assert np.array_equal(fused["dv"], split["dv"])


@pytest.mark.parametrize("bwd", BWD)
def test_fused_backward_workspace_regrows_and_is_cleared(bwd, device):
    """One library, three problems in a row (small, larger, small): the
    library's workspace grows, and each launch starts from a clean state (a
    stale atomic sum would double dQ)."""
    for seq, heads in ((100, 1), (700, 3), (100, 1)):
        run = _Run(heads, seq, 128, "bf16", True, seed=seq + heads, bwd=bwd)
        try:
            fused = run.run_fused()
            again = run.run_fused()
        finally:
            run.free()
        q, k, v, d_out = run.inputs
        want = R.attention_backward(q, k, v, d_out, run.scale, True)
        assert T.hybrid_error(fused["dq"], want["dq"]) <= 2e-2
        # the second launch sums the same partials in another order: one
        # rounding unit of the element type apart at most, not twice the value
        assert T.hybrid_error(again["dq"], fused["dq"]) <= 2 * T.U_BF16
        assert np.array_equal(again["dk"], fused["dk"])


@pytest.mark.parametrize("bwd", BWD)
def test_fused_backward_config5_full_size_against_split(bwd, device):
    """B4 H32 S4096 D128, bf16, causal, at full size: dK and dV bit-identical
    to the split kernels, dQ within the parity tolerance of the split kernel's
    dQ, which the oracle-checked tests pin."""
    heads, seq, dim = 128, 4096, 128
    rng = np.random.default_rng(5)
    inputs = [round_to(rng.standard_normal((heads, seq, dim), dtype=np.float32), "bf16")
              for _ in range(4)]
    run = _Run(heads, seq, dim, "bf16", True, inputs=inputs, bwd=bwd)
    try:
        split = run.run_split()
        fused = run.run_fused()
    finally:
        run.free()
    assert np.array_equal(fused["dk"], split["dk"])
    assert np.array_equal(fused["dv"], split["dv"])
    assert np.all(np.isfinite(fused["dq"]))
    # the two dQ come from differently ordered MFMA sums of dS (itself
    # recomputed in the other orientation, so a rounded dS may differ by one
    # unit): the same hybrid metric the oracle tests use, against the split
    assert T.hybrid_error(fused["dq"], split["dq"]) <= 2e-2
