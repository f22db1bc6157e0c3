"""CPU: the A7 account (tests/moe_cases.py) catches what it is meant to catch.
Mistakes are planted in copies of the oracle chain's own outputs, on the CPU:
a code moved by several ULPs at a large |h|, and a code moved beyond the ULP
cap, must fail the bar; an untouched chain passes it."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from moe_cases import A7_GT1_MAX_REL_AMAX, A7_MFMA_MAX_ULP, a7_account, a7_assert, count_bar, make_case


@pytest.fixture(scope="module")
def chain():
    c = make_case(64, 256, 256, 2, 2, 16, seed=21)
    return oracle.moe_layer_stages(c.x, c.topk_ids, c.topk_w, c.w13_q, c.w13_s, c.w2_q, c.w2_s, c.BM)


def _account(st, codes, h):
    return a7_account(codes, st["s2"], h, None, st["q2"], st["s2"], st["h"], None)


def test_untouched_chain_passes(chain):
    rep = _account(chain, chain["q2"].copy(), chain["h"].copy())
    assert rep["frac"] == 0 and rep["max_ulp"] == 0
    a7_assert(rep, "untouched")


def _largest_code(st):
    """(row, col) of the largest |h| with a normal code below 448."""
    h = np.abs(oracle.bf16_to_f32(st["h"]))
    q = st["q2"] & 0x7F
    h = np.where((q < 0x70) & (q > 0x10), h, 0)
    return np.unravel_index(np.argmax(h), h.shape)


def test_multi_ulp_code_at_large_h_fails(chain):
    r, c = _largest_code(chain)
    codes, h = chain["q2"].copy(), chain["h"].copy()
    codes[r, c] = codes[r, c] + 2          # two ULPs at a value near its group's amax
    h[r, c] ^= 1                           # traced to a differing h, as a real flip would be
    rep = _account(chain, codes, h)
    assert rep["n_gt1"] == 1 and rep["gt1_max_rel_to_amax"] > A7_GT1_MAX_REL_AMAX
    with pytest.raises(AssertionError):
        a7_assert(rep, "planted 2-ulp code at a large |h|")


def test_code_beyond_the_ulp_cap_fails(chain):
    """A code near zero (|h| below A7_GT1_MAX_REL_AMAX of its group's amax,
    where multi-ULP moves are allowed) moved beyond the cap fails on the cap
    alone."""
    h32 = np.abs(oracle.bf16_to_f32(chain["h"])).astype(np.float64)
    amax = np.repeat(h32.reshape(h32.shape[0], -1, 128).max(axis=2), 128, axis=1)
    rel = np.where((chain["q2"] & 0x7F) > A7_MFMA_MAX_ULP + 1, h32 / np.maximum(amax, 1e-30), np.inf)
    r, c = np.unravel_index(np.argmin(rel), rel.shape)
    assert rel[r, c] <= A7_GT1_MAX_REL_AMAX
    codes, h = chain["q2"].copy(), chain["h"].copy()
    codes[r, c] = codes[r, c] - (A7_MFMA_MAX_ULP + 1)
    h[r, c] ^= 1
    rep = _account(chain, codes, h)
    assert rep["max_ulp"] == A7_MFMA_MAX_ULP + 1 and rep["gt1_max_rel_to_amax"] <= A7_GT1_MAX_REL_AMAX
    with pytest.raises(AssertionError, match="ulp cap"):
        a7_assert(rep, "planted code beyond the cap")


def test_count_bar_known_answers():
    """The Poisson bar for rare events: one event always allowed, about
    mean + 3 sigma for large samples."""
    assert count_bar(1e-3, 0) == 1.0
    assert abs(count_bar(1e-3, 10 ** 6) - (1000 + 3 * 1000 ** 0.5 + 1)) < 1e-9
    assert 5 < count_bar(1e-3, 1251) < 6
