"""CPU: the A7 account (tests/moe_cases.py) catches what it is meant to catch.
Mistakes are planted in copies of the oracle chain's own outputs, on the CPU:
a code moved by several ULPs at a large |h|, a code moved beyond the ULP cap,
and an h moved with its C13 inputs unchanged must fail the bar; an untouched
chain, and a one-step gate flip with h recomputed from it, pass it."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from moe_cases import (A7_GT1_MAX_REL_AMAX, A7_MFMA_MAX_ULP, a7_account, a7_assert, count_bar, h_propagation_ratio,
                       make_case)


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


@pytest.fixture(scope="module")
def chain_with_c13():
    c = make_case(64, 256, 256, 2, 2, 16, seed=22)
    return oracle.moe_layer_stages(c.x, c.topk_ids, c.topk_w, c.w13_q, c.w13_s, c.w2_q, c.w2_s, c.BM)


def _full_account(st, codes, h, c13):
    return a7_account(codes, st["s2"], h, c13, st["q2"], st["s2"], st["h"], st["c13"], st["c13_f32"],
                      st["bound13"])


def _mid_gate(st):
    """(row, col) of a gate value of middling size with a normal code."""
    I = st["h"].shape[1]
    g = np.abs(oracle.bf16_to_f32(st["c13"][:, :I]))
    q = st["q2"] & 0x7F
    score = np.where((q > 0x20) & (q < 0x70), -np.abs(g - np.median(g)), -np.inf)
    return np.unravel_index(np.argmax(score), score.shape)


def test_propagated_bound_covers_a_one_step_gate_flip(chain_with_c13):
    """A gate moved by one bf16 step (what an in-bound matrix-core error does
    near a rounding boundary), with h recomputed from it, is within the
    propagated bound."""
    st = chain_with_c13
    r, j = _mid_gate(st)
    c13 = st["c13"].copy()
    c13[r, j] += 1                                   # next bf16 value of the same sign
    h = oracle.silu_and_mul(c13)
    ratio = h_propagation_ratio(h, c13, st["h"], st["c13"], st["c13_f32"], st["bound13"])
    assert ratio[r, j] <= 1.0
    assert ratio[h != st["h"]].max() <= 1.0


def test_propagated_bound_catches_an_unexplained_h(chain_with_c13):
    """An h moved far with its C13 inputs unchanged (a planted SiLU*up or
    epilogue mistake) exceeds the propagated bound and fails the account."""
    st = chain_with_c13
    r, j = _mid_gate(st)
    h = st["h"].copy()
    h32 = oracle.bf16_to_f32(h)
    h32[r, j] *= 1.5
    h = oracle.f32_to_bf16(h32)
    codes = oracle.quant_group128(h)[0]
    rep = _full_account(st, codes, h, st["c13"].copy())
    assert rep["h_diff_need_max_bound"] > 1.0
    with pytest.raises(AssertionError, match="propagated"):
        a7_assert(rep, "planted h at 1.5x")
