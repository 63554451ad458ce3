"""FlashAttention-2 forward and backward on the device against the fp64 oracle.

Mirrors Tests/TritonMetalCoreTests/AttentionTests.swift:119-206 and
AttentionBackwardTests.swift:330-575, python/examples/attention_training.py
(benchmark config 2) and configs 4 and 5 at full size.  Tolerances:
the reference's own (2e-5 hybrid for f32 forward, 4e-3 for f16 forward, the
derived summation bound n*u*A for the backward) and the north star's 2e-2
absolute against an fp32-or-better reference for bf16.
"""

import math

import numpy as np
import pytest

from attn_util import Runner, inputs, normal_inputs
from oracle import reference as R
from oracle import tolerance as T

pytestmark = pytest.mark.gpu

LN2 = math.log(2.0)


def oracle(q, k, v, d_out, scale, causal=False):
    return R.attention_backward(q, k, v, d_out, scale, causal)


# --------------------------------------------------------------------------- #
# forward
# --------------------------------------------------------------------------- #

FWD_SHAPES = [(2, 127, 64), (1, 512, 64), (1, 96, 80), (3, 33, 64), (1, 64, 64)]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("heads,seq,dim", FWD_SHAPES)
def test_forward_f32_across_shapes(device, heads, seq, dim, causal):
    """AttentionTests.swift:119-135 at 2e-5 (and the causal extension)."""
    q, k, v, _ = inputs(heads, seq, dim)
    r = Runner(heads, seq, dim, "f32", causal)
    try:
        o, lse = r.forward(q, k, v)
    finally:
        r.free()
    want_o, _, want_l = R.attention_forward(q, k, v, r.scale, causal)
    assert T.hybrid_error(o, want_o) <= 2e-5
    assert T.hybrid_error(lse, want_l) <= 2e-5


@pytest.mark.parametrize("stats", [True, False])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("heads,seq,dim", [(1, 512, 64), (2, 300, 96), (1, 1000, 32), (3, 129, 128)])
def test_forward_f32_key_range_split(device, heads, seq, dim, causal, stats):
    """Grids too small to fill the chip split each workgroup's key blocks into
    ranges whose partials a second dispatch combines; same answers at 2e-5,
    including causal rows whose later ranges hold no visible key, and the
    8-argument form that writes no L."""
    q, k, v, _ = inputs(heads, seq, dim)
    r = Runner(heads, seq, dim, "f32", causal)
    try:
        r.layer.buffers["lse"].write(np.full((heads, seq), 7.0, np.float32))
        o, lse = r.forward(q, k, v, stats=stats)
    finally:
        r.free()
    assert "key ranges" in r.variant, r.variant
    want_o, _, want_l = R.attention_forward(q, k, v, r.scale, causal)
    assert T.hybrid_error(o, want_o) <= 2e-5
    if stats:
        assert T.hybrid_error(lse, want_l) <= 2e-5
    else:
        assert np.all(lse == 7.0)


@pytest.mark.parametrize("element,tol", [("f16", 4e-3), ("bf16", 2e-2)])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("heads,seq,dim", [(2, 127, 64), (1, 128, 64), (2, 200, 128),
                                           (1, 77, 128)])
def test_forward_half_precision(device, heads, seq, dim, causal, element, tol):
    """AttentionTests.swift:140-156: inputs pre-rounded so the reference measures
    the kernel, not the rounding."""
    q, k, v, _ = inputs(heads, seq, dim, element)
    r = Runner(heads, seq, dim, element, causal)
    try:
        o, lse = r.forward(q, k, v)
    finally:
        r.free()
    want_o, _, want_l = R.attention_forward(q, k, v, r.scale, causal)
    assert T.hybrid_error(o, want_o) <= tol
    assert T.max_abs_error(lse, want_l) <= T.lse_bound(element)


def test_forward_is_stable_on_scores_that_overflow_exp(device):
    """AttentionTests.swift:161-177: raw scores ~1100, output finite, 1e-4, in V's range."""
    heads, seq, dim = 1, 100, 64
    q, k, v, _ = inputs(heads, seq, dim, spread=12)
    r = Runner(heads, seq, dim, "f32", scale=1.0)
    try:
        o, _ = r.forward(q, k, v)
    finally:
        r.free()
    want, _, _ = R.attention_forward(q, k, v, 1.0)
    assert np.all(np.isfinite(o))
    assert T.hybrid_error(o, want) <= 1e-4
    assert o.max() <= 12 + 1e-3 and o.min() >= -12 - 1e-3


@pytest.mark.parametrize("threads", [32, 64, 128, 256])
def test_forward_at_every_requested_workgroup_size(device, threads):
    """AttentionTests.swift:181-206."""
    heads, seq, dim = 1, 65, 64
    q, k, v, _ = inputs(heads, seq, dim)
    r = Runner(heads, seq, dim, threads=threads)
    try:
        o, _ = r.forward(q, k, v, stats=False)
    finally:
        r.free()
    assert T.hybrid_error(o, R.attention_forward(q, k, v, r.scale)[0]) <= 2e-5


# --------------------------------------------------------------------------- #
# backward
# --------------------------------------------------------------------------- #

BWD_SHAPES = [
    (1, 64, 64, "f32"), (2, 127, 64, "f32"), (1, 96, 80, "f32"), (3, 33, 64, "f32"),
    (1, 50, 20, "f32"), (2, 128, 64, "f32"), (2, 127, 64, "f16"), (1, 128, 64, "f16"),
]


def _assert_within_bound(actual, expected, terms, u, amplification, label):
    bound = T.summation_bound(expected, terms, u, amplification)
    worst = T.max_abs_error(actual, expected)
    assert worst <= bound, f"{label}: worst {worst:.3e} > bound {bound:.3e}"


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("heads,seq,dim,element", BWD_SHAPES)
def test_gradients_match_the_analytic_reference(device, heads, seq, dim, element, causal):
    """AttentionBackwardTests.swift:330-385 with its derived bound n*u*A."""
    q, k, v, d_out = inputs(heads, seq, dim, element)
    r = Runner(heads, seq, dim, element, causal)
    want = oracle(q, k, v, d_out, r.scale, causal)
    try:
        delta, dq, dk, dv = r.backward(q, k, v, want["o"], want["lse"], d_out)
    finally:
        r.free()
    u = T.U_F16 if element == "f16" else T.U_F32
    terms = seq + dim + 2
    _assert_within_bound(delta, want["delta"], dim + 1, u, 1.0, "Delta")
    amp = want["amplification"]
    _assert_within_bound(dq, want["dq"], terms, u, amp["dq"], "dQ")
    _assert_within_bound(dk, want["dk"], terms, u, amp["dk"], "dK")
    _assert_within_bound(dv, want["dv"], terms, u, amp["dv"], "dV")


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("heads,seq,dim,element", [(1, 512, 64, "f32"), (2, 300, 96, "f32"),
                                                   (1, 1000, 32, "f32"), (3, 129, 128, "f32"),
                                                   (1, 300, 80, "bf16")])
def test_gradients_key_and_query_range_split(device, heads, seq, dim, element, causal):
    """Grids too small to fill the chip split dq's key blocks and dkdv's query
    blocks into ranges whose fp32 partials a second dispatch sums (with
    sm_scale and the output rounding): the same bound as the unsplit kernels,
    including causal ranges that hold no visible pair."""
    q, k, v, d_out = inputs(heads, seq, dim, element)
    r = Runner(heads, seq, dim, element, causal)
    want = oracle(q, k, v, d_out, r.scale, causal)
    try:
        delta, dq, dk, dv = r.backward(q, k, v, want["o"], want["lse"], d_out)
    finally:
        r.free()
    assert all("ranges" in v for v in r.variants[1:]), r.variants
    amp = want["amplification"]
    if element == "f32":
        terms = seq + dim + 2
        _assert_within_bound(dq, want["dq"], terms, T.U_F32, amp["dq"], "dQ")
        _assert_within_bound(dk, want["dk"], terms, T.U_F32, amp["dk"], "dK")
        _assert_within_bound(dv, want["dv"], terms, T.U_F32, amp["dv"], "dV")
    else:
        for name, got in (("dq", dq), ("dk", dk), ("dv", dv)):
            assert T.hybrid_error(got, want[name]) <= 2e-2, name


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("heads,seq,dim", [(2, 127, 64), (1, 200, 128), (2, 64, 32)])
def test_bf16_gradients(device, heads, seq, dim, causal):
    """bf16 backward (this build's extension): 2e-2 hybrid vs fp64 from rounded inputs."""
    q, k, v, d_out = inputs(heads, seq, dim, "bf16")
    r = Runner(heads, seq, dim, "bf16", causal)
    want = oracle(q, k, v, d_out, r.scale, causal)
    try:
        delta, dq, dk, dv = r.backward(q, k, v, want["o"], want["lse"], d_out)
    finally:
        r.free()
    assert T.hybrid_error(delta, want["delta"]) <= 2e-2
    for name, got in (("dq", dq), ("dk", dk), ("dv", dv)):
        assert T.hybrid_error(got, want[name]) <= 2e-2, name


@pytest.mark.parametrize("causal", [False, True])
def test_gradients_match_finite_differences(device, causal):
    """AttentionBackwardTests.swift:397-482: the check that owes nothing to the
    backward formulas."""
    heads, seq, dim = 1, 48, 24
    q, k, v, d_out = inputs(heads, seq, dim)
    r = Runner(heads, seq, dim, "f32", causal)
    want = oracle(q, k, v, d_out, r.scale, causal)
    try:
        _, dq, dk, dv = r.backward(q, k, v, want["o"], want["lse"], d_out)
    finally:
        r.free()
    count = heads * seq * dim
    terms = seq + dim + 2
    for name, gpu in (("dq", dq), ("dk", dk), ("dv", dv)):
        bound = T.summation_bound(want[name], terms, T.U_F32, want["amplification"][name])
        for flat in range(0, count, max(1, count // 12)):
            index = np.unravel_index(flat, q.shape)
            numeric = R.finite_difference(q, k, v, d_out, r.scale, name, index, causal=causal)
            assert abs(numeric - want[name][index]) <= 1e-6 * max(1, abs(numeric))
            assert abs(numeric - gpu[index]) <= bound, (name, index)


@pytest.mark.parametrize("element", ["f32", "bf16"])
@pytest.mark.parametrize("causal", [False, True])
def test_forward_statistics_feed_the_backward(device, element, causal):
    """AttentionBackwardTests.swift:490-535: the GPU forward's O and L feed the
    GPU backward; only the check is on the CPU."""
    heads, seq, dim = 2, 100, 64
    q, k, v, d_out = inputs(heads, seq, dim, element)
    r = Runner(heads, seq, dim, element, causal)
    try:
        _, lse = r.forward(q, k, v)
        r.layer.upload("do", d_out)
        delta, dq, dk, dv = r.backward_resident()
    finally:
        r.free()
    want = oracle(q, k, v, d_out, r.scale, causal)
    if element == "f32":
        _assert_within_bound(lse, want["lse"], seq + dim, T.U_F32, 1.0, "L")
        terms = seq + dim + 2
        for name, got in (("dq", dq), ("dk", dk), ("dv", dv)):
            _assert_within_bound(got, want[name], terms, T.U_F32,
                                 want["amplification"][name], name)
    else:
        assert T.max_abs_error(lse, want["lse"]) <= T.lse_bound(element)
        for name, got in (("dq", dq), ("dk", dk), ("dv", dv)):
            assert T.hybrid_error(got, want[name]) <= 2e-2, name


@pytest.mark.parametrize("threads", [32, 64, 128, 256])
def test_gradients_at_every_requested_workgroup_size(device, threads):
    """AttentionBackwardTests.swift:546-575."""
    heads, seq, dim = 1, 65, 64
    q, k, v, d_out = inputs(heads, seq, dim)
    r = Runner(heads, seq, dim, threads=threads)
    want = oracle(q, k, v, d_out, r.scale)
    try:
        _, dq, dk, dv = r.backward(q, k, v, want["o"], want["lse"], d_out)
    finally:
        r.free()
    terms = seq + dim + 2
    for name, got in (("dq", dq), ("dk", dk), ("dv", dv)):
        _assert_within_bound(got, want[name], terms, T.U_F32, want["amplification"][name], name)


# --------------------------------------------------------------------------- #
# Config 2: the attention training run
# --------------------------------------------------------------------------- #


def _gpu_training_run(q, k, v, target, rate, steps=8):
    heads, seq, dim = q.shape
    r = Runner(heads, seq, dim, "f32")

    def forward(q, k, v):
        return r.forward(q, k, v)[0]

    def grad(q, k, v, d_out):
        r.forward(q, k, v)
        r.layer.upload("do", d_out)
        _, dq, dk, dv = r.backward_resident()
        return dq, dk, dv

    try:
        return R.training_run(grad, forward, q, k, v, target, rate, steps)
    finally:
        r.free()


def test_published_training_run_on_the_device(device):
    """attention_training.py:312-329 on the device: the reference's published
    run (docs/USAGE.md:163-165) is 1541.733643 -> 1482.859741."""
    q, k, v, target = R.reference_training_inputs()
    records, final = _gpu_training_run(q, k, v, target, rate=0.5)
    assert records[0]["loss"] == pytest.approx(1541.733643, abs=1e-2)
    assert records[0]["dq"] == pytest.approx(1.4582, abs=2e-4)
    assert records[0]["dk"] == pytest.approx(1.4173, abs=2e-4)
    assert records[0]["dv"] == pytest.approx(8.3391, abs=2e-4)
    assert final == pytest.approx(1482.859741, abs=2e-2)
    assert final < records[0]["loss"]


def test_config2_training_steps_match_numpy_autograd(device):
    """Config 2: B1 H2 S96 D64 fp32, Q/K/V/W ~ N(0, 0.1), scale 1/8,
    forward + backward + 8 SGD steps at lr 1e-3 on the sum-of-squares loss
    0.5*||O - W||^2 (W read as the regression target), every step within 1e-5
    relative of the fp64 numpy autograd run from the same inputs."""
    rng = np.random.default_rng(2)
    q, k, v, w = (rng.standard_normal((2, 96, 64), dtype=np.float32) * np.float32(0.1)
                  for _ in range(4))
    scale = 1 / 8

    def forward64(q, k, v):
        return R.attention_forward(q, k, v, scale)[0]

    def grad64(q, k, v, d_out):
        g = R.attention_backward(q, k, v, d_out, scale)
        return g["dq"], g["dk"], g["dv"]

    want, want_final = R.training_run(grad64, forward64, q, k, v, w, rate=1e-3)
    got, got_final = _gpu_training_run(q, k, v, w, rate=1e-3)
    for g, e in zip(got, want):
        for key in ("loss", "dq", "dk", "dv"):
            assert abs(g[key] - e[key]) / max(1.0, abs(e[key])) <= 1e-5, key
    assert abs(got_final - want_final) / max(1.0, want_final) <= 1e-5


# --------------------------------------------------------------------------- #
# Configs 4 and 5 at full size
# --------------------------------------------------------------------------- #


def test_config4_bf16_forward_full_size(device):
    """B8 H16 S1024 D64 bf16, non-causal, N(0,1), scale 1/8: O and the natural-log
    logsumexp (L*ln2) of every head within 2e-2 absolute of an fp32 BLAS
    reference from the same bf16 inputs, and every head also against fp64."""
    bh, seq, dim = 128, 1024, 64
    q, k, v = normal_inputs(bh, seq, dim, "bf16", seed=4, count=3)
    r = Runner(bh, seq, dim, "bf16")
    try:
        o, lse = r.forward(q, k, v)
    finally:
        r.free()
    scale = 1 / 8
    s = np.matmul(q, k.transpose(0, 2, 1)) * np.float32(scale)
    peak = s.max(-1, keepdims=True)
    e = np.exp(s - peak)
    tot = e.sum(-1, keepdims=True)
    o32 = np.matmul(e / tot, v)
    lse_nat = (peak[..., 0] + np.log(tot[..., 0]))
    assert T.max_abs_error(o, o32) <= 2e-2
    assert T.max_abs_error(lse * LN2, lse_nat) <= 2e-2
    for h in range(bh):
        o64, _, l64 = R.attention_forward(q[h:h + 1], k[h:h + 1], v[h:h + 1], scale)
        assert T.max_abs_error(o[h:h + 1], o64) <= 2e-2
        assert T.max_abs_error(lse[h:h + 1] * LN2, l64 * LN2) <= 2e-2


def _head_backward64(q, k, v, d_out, scale):
    """fp64 causal attention forward+backward for one head, through BLAS."""
    q, k, v, d_out = (x.astype(np.float64) for x in (q, k, v, d_out))
    n = q.shape[0]
    s = (q @ k.T) * scale
    s[np.triu_indices(n, 1)] = -np.inf
    peak = s.max(-1, keepdims=True)
    e = np.exp(s - peak)
    tot = e.sum(-1, keepdims=True)
    p = e / tot
    o = p @ v
    lse_nat = peak[:, 0] + np.log(tot[:, 0])
    dv = p.T @ d_out
    dp = d_out @ v.T
    delta = np.sum(d_out * o, -1)
    ds = p * (dp - delta[:, None])
    return o, lse_nat, ds @ k * scale, ds.T @ q * scale, dv


@pytest.mark.parametrize("element", ["bf16", "f16"])
def test_config5_causal_forward_backward_full_size(device, element):
    """B4 H32 S4096 D128 causal in bf16 (the benchmark's element type) and f16
    (the reference's own attention element type), N(0,1), scale 1/sqrt(128): O,
    LSE, dQ, dK, dV.  Every head against fp64 (2e-2 absolute on O and LSE, 2e-2 hybrid on
    the gradients); every head through size-independent identities of causal
    attention: O[0] = V[0], dQ[0] = 0, sum_j dK_j = 0, sum_j dV_j = sum_i dO_i."""
    bh, seq, dim = 128, 4096, 128
    q, k, v, d_out = normal_inputs(bh, seq, dim, element, seed=5)
    r = Runner(bh, seq, dim, element, causal=True)
    try:
        o, lse = r.forward(q, k, v)
        r.layer.upload("do", d_out)
        delta, dq, dk, dv = r.backward_resident()
        variants = [r.variant] + r.variants
    finally:
        r.free()
    print("config5 variants:", variants)
    scale = 1 / math.sqrt(dim)
    worst = {"dq": 0.0, "dk": 0.0, "dv": 0.0}
    for h in range(bh):
        o64, l64, dq64, dk64, dv64 = _head_backward64(q[h], k[h], v[h], d_out[h], scale)
        assert T.max_abs_error(o[h], o64) <= 2e-2
        assert T.max_abs_error(lse[h] * LN2, l64) <= 2e-2
        for name, got, want in (("dq", dq[h], dq64), ("dk", dk[h], dk64), ("dv", dv[h], dv64)):
            err = T.hybrid_error(got, want)
            worst[name] = max(worst[name], err)
            assert err <= 2e-2, (h, name)
    print("config5 worst hybrid error over all heads:", {n: f"{e:.3e}" for n, e in worst.items()})
    assert np.all(np.isfinite(o)) and np.all(np.isfinite(dq))
    assert np.all(np.isfinite(dk)) and np.all(np.isfinite(dv))
    assert T.max_abs_error(o[:, 0], v[:, 0]) <= 1e-2
    assert np.max(np.abs(dq[:, 0])) <= 1e-2
    dk_sum = dk.astype(np.float64).sum(1)
    assert np.max(np.abs(dk_sum)) <= 2e-2 * max(1.0, np.abs(dk).max() * math.sqrt(seq))
    # sum_j dV_j = sum_i (sum_j P_ij) dO_i = sum_i dO_i; the bf16 output rounding
    # alone may move the left side by 2^-9 * sum_j |dV_j|, the bf16 P by about
    # as much again.
    dv_sum = dv.astype(np.float64).sum(1)
    do_sum = d_out.astype(np.float64).sum(1)
    bound = 2.0 ** -7 * np.abs(dv.astype(np.float64)).sum(1)
    assert np.max(np.abs(dv_sum - do_sum) / bound) <= 1.0
