"""Pins the oracle's number-format conversions to torch's own casts.

The oracle's e4m3 and bf16 conversions (oracle/moe_oracle.c) are written from
the OCP e4m3fn / bfloat16 definitions; here they are checked against
``torch.Tensor.to(torch.float8_e4m3fn)`` / ``.to(torch.bfloat16)`` on the CPU,
the casts the reference itself performs (moe_bench/verify.py:116,
moe_bench/data/checkpoint.py:38), exhaustively over every bf16 input and on
dense fp32 samples around the rounding boundaries.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle


def torch_e4m3(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def torch_bf16(x: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def test_e4m3_encode_matches_torch_on_every_bf16_value():
    bits = np.arange(65536, dtype=np.uint32)
    x = (bits << 16).view(np.float32)
    finite = np.isfinite(x)
    got = oracle.f32_to_e4m3(x[finite])
    ref = torch_e4m3(x[finite])
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first x={x[finite][bad[:5]]} got={got[bad[:5]]} ref={ref[bad[:5]]}"


@pytest.mark.parametrize("seed", [0, 1])
def test_e4m3_encode_matches_torch_on_dense_fp32(seed):
    rng = np.random.default_rng(seed)
    # log-uniform magnitudes over the whole e4m3 range incl. subnormals and
    # the out-of-range band, plus exact midpoints between adjacent codes
    mag = np.exp2(rng.uniform(-12.0, 9.5, 400_000)).astype(np.float32)
    x = mag * rng.choice(np.array([-1.0, 1.0], np.float32), mag.size)
    lut = oracle.e4m3_lut()
    finite_codes = np.sort(lut[np.isfinite(lut) & (lut >= 0)])
    mids = ((finite_codes[1:] + finite_codes[:-1]) / 2).astype(np.float32)
    x = np.concatenate([x, mids, -mids, np.nextafter(mids, 0), np.nextafter(mids, 1000)])
    got = oracle.f32_to_e4m3(x)
    ref = torch_e4m3(x)
    assert np.array_equal(got, ref)


def test_e4m3_known_ties_round_to_even():
    # 1.0625 lies halfway between 1.0 (0x38) and 1.125 (0x39): even mantissa 0x38.
    # 1.1875 lies halfway between 1.125 (0x39) and 1.25 (0x3A): even is 0x3A.
    got = oracle.f32_to_e4m3(np.array([1.0625, 1.1875, 448.0, -448.0, 0.0, -0.0, 2.0 ** -9], np.float32))
    assert got.tolist() == [0x38, 0x3A, 0x7E, 0xFE, 0x00, 0x80, 0x01]


def test_e4m3_decode_matches_torch_for_every_code():
    lut = oracle.e4m3_lut()
    ref = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(lut), nan)
    assert np.array_equal(lut[~nan], ref[~nan])
    assert nan.sum() == 2  # 0x7F and 0xFF


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(500_000) * np.exp2(rng.uniform(-30, 30, 500_000))).astype(np.float32)
    # exact ties between adjacent bf16 values: low 16 bits 0x8000
    ties = ((rng.integers(0, 2 ** 31, 10_000, dtype=np.uint64) & 0xFFFF0000) | 0x8000).astype(np.uint32)
    x = np.concatenate([x, ties.view(np.float32)])
    x = x[np.isfinite(x)]
    assert np.array_equal(oracle.f32_to_bf16(x), torch_bf16(x))


def test_bf16_decode_is_exact_widening():
    b = np.arange(0, 65536, 257, dtype=np.uint16)
    ref = torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).float().numpy()
    got = oracle.bf16_to_f32(b)
    ok = ~np.isnan(ref)
    assert np.array_equal(got[ok].view(np.uint32), ref[ok].view(np.uint32))
