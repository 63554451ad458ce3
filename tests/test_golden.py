"""Golden fixtures (tests/golden/fixtures.json, written by
tests/golden/make_fixtures.py): the seeded inputs of BASELINE's five
configurations, pinned by SHA-256, and the oracle's answers for configs 1 and 2.
A change of generator, seed, draw order or bf16 rounding, or of the oracle's
GEMM or training-step maths, fails here before it can shift a GPU comparison."""

import importlib.util
import json
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).with_name("golden")


@pytest.fixture(scope="module")
def fixtures():
    return json.loads((GOLDEN / "fixtures.json").read_text())


@pytest.fixture(scope="module")
def maker():
    spec = importlib.util.spec_from_file_location("make_fixtures", GOLDEN / "make_fixtures.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_inputs_match_their_checksums(fixtures, maker):
    ins, _, _ = maker.inputs()
    assert ins == fixtures["inputs"]


def test_config1_oracle_answer(fixtures, maker):
    _, (a, b), _ = maker.inputs()
    want = fixtures["answers"]["config1_c"]
    c = a.astype(np.float64) @ b.astype(np.float64)   # BLAS, a different summation order
    for i, j, v in want["picks"]:
        assert c[i, j] == pytest.approx(v, abs=want["tol"])
    assert c.sum() == pytest.approx(want["sum"], abs=1e-6)
    got = maker.answers((a, b), maker.inputs()[2])["config1_c"]
    assert got["picks"] == want["picks"]


def test_config2_training_answer(fixtures, maker):
    _, c1, c2 = maker.inputs()
    want = fixtures["answers"]["config2_training"]
    got = maker.answers(c1, c2)["config2_training"]
    tol = want["rel_tol"]
    for g, e in zip(got["records"], want["records"]):
        for key in ("loss", "dq", "dk", "dv"):
            assert g[key] == pytest.approx(e[key], rel=tol)
    assert got["final"] == pytest.approx(want["final"], rel=tol)
