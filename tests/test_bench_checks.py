"""bench.py's own checks, on any machine: the fp64 restatement it verifies its
timed outputs with agrees with the oracle, its verifier fails on a wrong
answer, and its error metrics are the oracle's."""

import math
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402
from oracle import reference as R  # noqa: E402
from oracle import tolerance as T  # noqa: E402


@pytest.mark.parametrize("causal", [False, True])
def test_bench_head_reference_matches_the_oracle(causal):
    rng = np.random.default_rng(21)
    q, k, v, d_out = (rng.standard_normal((1, 48, 16)) for _ in range(4))
    scale = 0.3
    got = bench._attention_head64(q[0], k[0], v[0], d_out[0], scale, causal)
    want = R.attention_backward(q, k, v, d_out, scale, causal)
    for name in ("o", "delta", "dq", "dk", "dv"):
        assert np.allclose(got[name], want[name][0], rtol=1e-12, atol=1e-12), name
    assert np.allclose(got["lse"], want["lse"][0] * math.log(2.0), rtol=1e-12, atol=1e-12)
    fwd = bench._attention_head64(q[0], k[0], v[0], None, scale, causal)
    assert set(fwd) == {"o", "lse"}


def test_bench_error_metrics_are_the_oracles():
    rng = np.random.default_rng(2)
    a, b = rng.standard_normal(50) * 3, rng.standard_normal(50) * 3
    assert bench._hybrid(a, b) == pytest.approx(T.hybrid_error(a, b))
    assert bench._abs(a, b) == pytest.approx(T.max_abs_error(a, b))
    assert bench._relative(a, b) == pytest.approx(T.relative_error(a, b))
    a[3] = np.nan
    assert bench._hybrid(a, b) == float("inf")


def test_verifier_records_and_fails():
    v = bench.Verifier()
    v.add("case", "dq", 1e-3, 2e-2)
    v.add("case", "dq", 5e-4, 2e-2)       # the worst error is kept
    assert v.record["case"]["dq"] == 1e-3 and not v.failures
    v.add("case", "dk", 3e-2, 2e-2)
    assert v.failures == ["case.dk: error 3.000e-02 > 0.02"]
    v.add("other", "o", float("inf"), 2e-2)
    assert len(v.failures) == 2


def test_operand_data_kinds():
    """The data study's operands: N(0,1) bf16 bits by default (the benchmark's
    data), the same values with the low 4 mantissa bits cleared, or zeros;
    the default is restored after a study."""
    base = bench.normal_bf16((64, 32), 5)
    assert base.dtype == np.uint16 and np.count_nonzero(base & 0xF) > 0
    try:
        bench._operand_data = "trunc4"
        t = bench.normal_bf16((64, 32), 5)
        assert np.array_equal(t, base & np.uint16(0xFFF0))
        bench._operand_data = "zeros"
        assert not np.any(bench.normal_bf16((64, 32), 5))
    finally:
        bench._operand_data = "normal"
    assert np.array_equal(bench.normal_bf16((64, 32), 5), base)
