"""The oracle is pinned before anything is compared against it.

Each check is chosen so that a plausible mistake in the restatement (a dropped
term, a wrong sign or index, a transposed operand, a missing scale) fails it:
  - the reference's published training run (docs/USAGE.md:163-165);
  - exact GEMM known answers from the reference's matrix() inputs
    (DotTests.swift:32-34: every product and partial sum is a multiple of 1/16
    well inside f32/f64 range, so the exact answer is an integer multiple of
    1/16 computed here with integer arithmetic);
  - numpy restatement vs the independent C fp64 loop;
  - central finite differences of sum(O*dO) (AttentionBackwardTests.swift:397-482);
  - softmax invariants (rows of P sum to 1, O inside the range of V);
  - causal = non-causal attention applied to each query's key prefix.
"""

import math

import numpy as np
import pytest

from oracle import generators as G
from oracle import native as N
from oracle import reference as R
from oracle import tolerance as T


def test_published_training_run_is_reproduced():
    """attention_training.py:312-329 with the reference's inputs gives the
    published numbers (docs/USAGE.md:163-165)."""
    q, k, v, target = R.reference_training_inputs()
    scale = 1 / math.sqrt(64)

    def forward(q, k, v):
        return R.numpy_attention_f32(q, k, v, scale)[0]

    def grad(q, k, v, d_out):
        _, w = R.numpy_attention_f32(q, k, v, scale)
        return R.numpy_attention_backward_f32(q, k, v, w, d_out, scale)

    records, final = R.training_run(grad, forward, q, k, v, target, rate=0.5)
    assert records[0]["loss"] == pytest.approx(1541.733643, abs=5e-3)
    assert records[0]["dq"] == pytest.approx(1.4582, abs=5e-5)
    assert records[0]["dk"] == pytest.approx(1.4173, abs=5e-5)
    assert records[0]["dv"] == pytest.approx(8.3391, abs=5e-5)
    assert final == pytest.approx(1482.859741, abs=5e-3)


def test_fp64_oracle_reproduces_the_reference_float32_gradients():
    q, k, v, target = R.reference_training_inputs()
    scale = 1 / 8
    out, w = R.numpy_attention_f32(q, k, v, scale)
    d_out = (out - target).astype(np.float32)
    want = R.numpy_attention_backward_f32(q, k, v, w, d_out, scale)
    got = R.attention_backward(q, k, v, d_out, scale)
    for name, ref in zip(("dq", "dk", "dv"), want):
        assert T.relative_error(got[name], ref) < 2e-5, name


@pytest.mark.parametrize("m,n,k", [(16, 16, 16), (129, 257, 65), (37, 8, 96), (1, 1, 1)])
def test_gemm_known_answer_is_exact(m, n, k):
    a = G.matrix(m * k, 3).reshape(m, k)
    b = G.matrix(k * n, 11).reshape(k, n)
    # Exact integer arithmetic in units of 1/4: a = A/4, b = B/4, c = C/16.
    ai = (a * 4).astype(np.int64)
    bi = (b * 4).astype(np.int64)
    exact = (ai @ bi).astype(np.float64) / 16
    assert np.array_equal(R.gemm(a, b), exact)
    assert np.array_equal(N.gemm(a, b, m, n, k, k, 1, n, 1), exact)


def test_gemm_strided_c_oracle_matches_numpy():
    rng = np.random.default_rng(1)
    m, n, k, stride = 33, 40, 27, 3
    a = rng.standard_normal((m, k * stride)).astype(np.float32)
    b = rng.standard_normal((k, n * stride)).astype(np.float32)
    want = a[:, ::stride].astype(np.float64) @ b[:, ::stride].astype(np.float64)
    got = N.gemm(a, b, m, n, k, k * stride, stride, n * stride, stride)
    assert np.max(np.abs(got - want)) < 1e-12


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("heads,seq,dim", [(2, 33, 16), (1, 50, 20), (2, 64, 24)])
def test_numpy_and_c_oracles_agree(heads, seq, dim, causal):
    count = heads * seq * dim
    q, k, v, do = (G.tensor(count, s).reshape(heads, seq, dim) for s in (1, 5, 9, 13))
    scale = 1 / math.sqrt(dim)
    a = R.attention_backward(q, k, v, do, scale, causal)
    b = N.attention(q, k, v, do, scale, causal)
    for name in ("o", "lse", "delta", "dq", "dk", "dv"):
        assert np.max(np.abs(a[name] - b[name])) < 1e-12, name
    for name in ("dq", "dk", "dv"):
        assert a["amplification"][name] == pytest.approx(b["amplification"][name], rel=1e-12)


@pytest.mark.parametrize("causal", [False, True])
def test_oracle_gradients_match_finite_differences(causal):
    heads, seq, dim = 1, 48, 24
    count = heads * seq * dim
    q, k, v, do = (G.tensor(count, s).reshape(heads, seq, dim) for s in (1, 5, 9, 13))
    scale = 1 / math.sqrt(dim)
    ref = R.attention_backward(q, k, v, do, scale, causal)
    for which in ("dq", "dk", "dv"):
        for flat in range(0, count, count // 12):
            index = np.unravel_index(flat, q.shape)
            numeric = R.finite_difference(q, k, v, do, scale, which, index, causal=causal)
            assert abs(numeric - ref[which][index]) <= 1e-6 * max(1, abs(numeric)), (which, index)


def test_softmax_invariants_and_log2_lse():
    heads, seq, dim = 1, 100, 64
    count = heads * seq * dim
    q, k, v = (G.tensor(count, s, spread=12).reshape(heads, seq, dim) for s in (1, 5, 9))
    o, p, lse2 = R.attention_forward(q, k, v, 1.0)
    assert np.all(np.isfinite(o))
    assert np.allclose(p.sum(-1), 1.0, atol=1e-12)
    assert o.min() >= float(v.min()) - 1e-9 and o.max() <= float(v.max()) + 1e-9
    # L is log2 of the unshifted denominator: 2^L = sum_j exp(s_ij), checked on a
    # case small enough not to overflow.
    q2, k2, v2 = (x / 12 for x in (q, k, v))
    _, _, l_small = R.attention_forward(q2, k2, v2, 0.125)
    s = np.einsum("hid,hjd->hij", q2.astype(np.float64), k2.astype(np.float64)) * 0.125
    assert np.allclose(2.0 ** l_small, np.exp(s).sum(-1), rtol=1e-12)


def test_causal_is_the_noncausal_oracle_on_each_prefix():
    heads, seq, dim = 1, 20, 16
    count = heads * seq * dim
    q, k, v = (G.tensor(count, s).reshape(heads, seq, dim) for s in (2, 4, 6))
    scale = 0.25
    o_c, _, l_c = R.attention_forward(q, k, v, scale, causal=True)
    for i in range(seq):
        o_i, _, l_i = R.attention_forward(q[:, i:i + 1], k[:, :i + 1], v[:, :i + 1], scale)
        assert np.allclose(o_c[:, i], o_i[:, 0], atol=1e-13)
        assert np.allclose(l_c[:, i], l_i[:, 0], atol=1e-13)


def test_generators_match_the_reference_formulas():
    # DotTests.swift:32-34 at a few hand-evaluated points.
    m = G.matrix(20, 5)
    assert m[0] == ((0 * 7 + 5 * 13) % 17) * 0.25 - 2
    assert m[19] == ((19 * 7 + 5 * 13) % 17) * 0.25 - 2
    # AttentionTests.swift:56-62.
    t = G.tensor(30, 9, spread=2)
    assert t[29] == pytest.approx((((29 * 31 + 9 * 17) % 23) / 23 * 2 - 1) * 2, abs=1e-6)
    assert set(np.unique(G.tensor(1000, 1) * 23 / 2 + 23 / 2).round(4)).issubset(
        set(np.arange(23.0)))


def test_sae_generator_matches_hand_evaluated_values():
    # MLXTestSupport.swift:82-90 with offset 1, modulus 71: 13/71 - 1/2, 26/71 - 1/2,
    # ..., and at i = 5 the product 78 wraps to 7.
    x = G.synthetic([2, 3], offset=1, modulus=71)
    assert x.dtype == np.float32 and x.shape == (2, 3)
    want = np.array([13, 26, 39, 52, 65, 7], np.float32) / np.float32(71) - np.float32(0.5)
    assert np.array_equal(x.ravel(), want)
    assert G.synthetic([1], offset=0)[0] == np.float32(-0.5)  # default modulus, i = 0
    assert G.synthetic([3], offset=3, modulus=29)[2] == np.float32(65 % 29) / np.float32(29) - np.float32(0.5)


def test_sae_oracle_against_brute_force_and_relu_properties():
    # relu(x @ w + b) by explicit loops with exact summation, on a ragged shape.
    x = G.synthetic([7, 13], offset=1)
    w = G.synthetic([13, 5], offset=7, modulus=53)
    b = G.synthetic([5], offset=3, modulus=29)
    got = R.sae_encode(x, w, b)
    for i in range(7):
        for j in range(5):
            pre = math.fsum(float(x[i, k]) * float(w[k, j]) for k in range(13)) + float(b[j])
            assert got[i, j] == pytest.approx(max(pre, 0.0), abs=1e-15)
    # A -5 bias drives every unit of this input to exactly zero
    # (SAEEncoderTests.swift:70-82 uses the same bias).
    assert np.count_nonzero(R.sae_encode(x, w, np.full(5, -5.0))) == 0
    # With a zero-width contraction the output is relu(b) on every row.
    z = R.sae_encode(np.zeros((3, 0)), np.zeros((0, 5)), b)
    assert np.array_equal(z, np.tile(np.maximum(b.astype(np.float64), 0), (3, 1)))


@pytest.mark.parametrize("causal", [False, True])
def test_blas_head_restatement_matches_the_reference_numpy_and_fp64(causal):
    # The CPU baseline's BLAS form equals the reference's einsum form (non-causal)
    # and the fp64 oracle (both), at float32 accuracy.
    rng = np.random.default_rng(3)
    q, k, v, d_out = (rng.standard_normal((1, 40, 16), dtype=np.float32) for _ in range(4))
    scale = 0.25
    o, dq, dk, dv = R.attention_head_f32(q[0], k[0], v[0], d_out[0], scale, causal)
    if not causal:
        o_ref, w = R.numpy_attention_f32(q, k, v, np.float32(scale))
        dq_ref, dk_ref, dv_ref = R.numpy_attention_backward_f32(q, k, v, w, d_out, np.float32(scale))
        for got, want in ((o, o_ref), (dq, dq_ref), (dk, dk_ref), (dv, dv_ref)):
            assert np.allclose(got, want[0], rtol=1e-4, atol=1e-5)
    want = R.attention_backward(q, k, v, d_out, scale, causal)
    for got, name in ((o, "o"), (dq, "dq"), (dk, "dk"), (dv, "dv")):
        assert np.allclose(got, want[name][0], rtol=1e-4, atol=1e-5), name


@pytest.mark.parametrize("block", [1, 7, 16, 40, 64])
def test_blocked_causal_head_matches_the_masked_form_and_fp64(block):
    # The CPU baseline's row-blocked causal form visits only visible keys; it
    # must equal the masked full-square form (and the fp64 oracle) for every
    # block size, including ragged last blocks and blocks of one row.
    rng = np.random.default_rng(11)
    q, k, v, d_out = (rng.standard_normal((1, 40, 16), dtype=np.float32) for _ in range(4))
    scale = 0.25
    got = R.attention_head_causal_blocked_f32(q[0], k[0], v[0], d_out[0], scale, block=block)
    full = R.attention_head_f32(q[0], k[0], v[0], d_out[0], scale, causal=True)
    want = R.attention_backward(q, k, v, d_out, scale, causal=True)
    for g, f, name in zip(got, full, ("o", "dq", "dk", "dv")):
        assert np.allclose(g, f, rtol=1e-4, atol=1e-5), name
        assert np.allclose(g, want[name][0], rtol=1e-4, atol=1e-5), name


def test_tolerance_metrics():
    assert T.hybrid_error([1.0, 10.0], [1.0, 11.0]) == pytest.approx(1 / 11)
    assert T.hybrid_error([0.5], [0.0]) == pytest.approx(0.5)
    assert T.relative_error([1.0, 3.0], [1.0, 4.0]) == pytest.approx(0.25)
    assert T.hybrid_error([np.nan], [1.0]) == float("inf")
