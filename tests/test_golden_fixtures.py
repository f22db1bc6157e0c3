"""The committed fixture tests/golden/tiny_seed0.npz against the oracle.

The fixture is loaded without pickle.  Every integer / byte / bf16 array must
be reproduced bit for bit by the current oracle (an oracle change that moves a
result shows up here); fp32 golden values may differ by BLAS summation order
only.  The fixture's own stage-chain output meets the reference worker's gates
against its golden (worker.py:107-146)."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN_DIR = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN_DIR))

import make_golden  # noqa: E402

EXACT = ("x", "topk_ids", "w13_q", "w13_s", "w2_q", "w2_s", "q1", "s1", "sorted_ids", "expert_ids",
         "ntpp", "c13", "h", "q2", "s2", "D", "y", "topk_w")


@pytest.fixture(scope="module")
def fixture():
    with np.load(make_golden.FIXTURE) as f:
        return {k: f[k] for k in f.files}


def test_fixture_shapes(fixture):
    T, H, I, E, k, BM = fixture["shape"].tolist()
    S = T * k
    assert fixture["x"].shape == (T, H) and fixture["x"].dtype == np.uint16
    assert fixture["w13_q"].shape == (E, 2 * I, H) and fixture["w2_q"].shape == (E, H, I)
    assert fixture["c13"].shape == (S, 2 * I) and fixture["D"].shape == (S, H)
    assert fixture["y"].shape == (T, H) and fixture["golden"].shape == (T, H)


def test_oracle_reproduces_fixture(fixture):
    fresh = make_golden.build_fixture()
    for key in EXACT:
        assert np.array_equal(fresh[key], fixture[key]), key
    np.testing.assert_allclose(fresh["golden"], fixture["golden"], rtol=1e-5, atol=1e-7)
    for key in ("mag13", "mag2", "bound13", "bound2"):
        np.testing.assert_allclose(fresh[key], fixture[key], rtol=1e-6)
    np.testing.assert_allclose(fresh["atol"], fixture["atol"], rtol=1e-4)


def test_fixture_chain_meets_gates(fixture):
    y = oracle.bf16_to_f32(fixture["y"])
    rep = oracle.compare_outputs(y, fixture["golden"], atol=0.0, rtol=0.0, **oracle.DEFAULT_GATES)
    assert rep["pass"], rep
    assert rep["max_abs"] <= float(fixture["atol"][0])
