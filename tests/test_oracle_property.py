"""Randomised pins of the oracle (CPU): many generated inputs against the
independent constructions of the other oracle tests.

* align (A3, the padded-cumsum layout of tdx/kernels/moe_utils.py:168-217):
  the Python brute force of test_oracle_align.py on random routings with
  empty experts, repeated experts and ids outside [0, E) (an expert map's -1);
* 1x128 quant (A1/A7, verify.py:108-117): the torch closed form of
  test_oracle_quant.py on random bf16 bit patterns (every finite value:
  subnormals, +-0, the largest magnitudes) and ragged widths.
Hypothesis runs derandomised, so the suite is the same on every run.
"""
from __future__ import annotations

import numpy as np
from hypothesis import given, settings
from hypothesis import strategies as st

import oracle
from test_oracle_align import brute_force_align
from test_oracle_quant import bf16_tensor, torch_group_quant


@st.composite
def routings(draw):
    E = draw(st.integers(1, 12))
    BM = draw(st.sampled_from([4, 8, 16, 32]))
    ids = draw(st.lists(st.integers(-1, E + 1), min_size=1, max_size=90))
    return np.asarray(ids, np.int32), E, BM


@settings(max_examples=300, deadline=None, derandomize=True)
@given(routings())
def test_align_matches_brute_force_on_random_routings(case):
    ids, E, BM = case
    mp = oracle.max_padded_size(ids.size, E, BM)
    got = oracle.moe_align(ids, E, BM, mp)
    ref = brute_force_align(ids.tolist(), E, BM, mp)
    assert got[2] == ref[2]
    assert got[0].tolist() == ref[0]
    assert got[1].tolist() == ref[1]


def _finite_bf16(bits: np.ndarray) -> np.ndarray:
    """Replaces the non-finite bf16 patterns (exponent all ones) by +-0."""
    bits = bits.astype(np.uint16)
    bits[(bits & 0x7F80) == 0x7F80] &= 0x8000
    return bits


@st.composite
def activations(draw):
    T = draw(st.integers(1, 4))
    H = draw(st.integers(1, 300))
    raw = draw(st.lists(st.integers(0, 0xFFFF), min_size=T * H, max_size=T * H))
    bits = _finite_bf16(np.asarray(raw, np.uint32).reshape(T, H))
    # also cover dense groups of ordinary values: scale a row to a common magnitude
    if draw(st.booleans()):
        bits[:, ::2] = (bits[:, ::2] & 0x807F) | 0x3F00  # exponents near 1.0
    return bits


@settings(max_examples=200, deadline=None, derandomize=True)
@given(activations())
def test_group128_quant_matches_closed_form_on_random_bits(bits):
    q, s = oracle.quant_group128(bits)
    rq, rs = torch_group_quant(bf16_tensor(bits))
    assert np.array_equal(s, rs)
    assert np.array_equal(q, rq)
