"""Pins the oracle's 1x128 activation quant (A1/A7) and 128x128 weight quant (A2).

Checks, none of which reuses the oracle's C code:
  * the reference's closed form (moe_bench/verify.py:108-117), evaluated with
    torch tensor ops and torch's float8 cast, over random and special inputs;
  * hand-computed known answers (all-zero group, single non-zero element,
    exact ties, subnormal codes, 128-aligned and ragged widths);
  * the reference's own tests, restated: the ragged 130x65 block-quant loop
    oracle (tests/test_quantize.py:9-36) and the group128 closeness bound
    (tests/test_golden.py:29-35).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

FP8_MAX = 448.0


def torch_group_quant(x: torch.Tensor) -> tuple[np.ndarray, np.ndarray]:
    """verify.py:108-117 with torch ops: pad to a multiple of 128, per-group
    amax/448 clamped at 1e-12, divide, clamp, cast."""
    T, H = x.shape
    pad = (-H) % 128
    xp = torch.nn.functional.pad(x.float(), (0, pad))
    g = xp.view(T, -1, 128)
    s = (g.abs().amax(dim=-1, keepdim=True) / FP8_MAX).clamp(min=1e-12)
    q = (g / s).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q.view(T, -1)[:, :H].view(torch.uint8).numpy(), s.squeeze(-1).numpy()


def bf16_tensor(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


@pytest.mark.parametrize("T,H,std,seed", [(7, 128, 1.0, 0), (33, 7168, 1.0, 1), (5, 384, 1e-3, 2),
                                          (9, 129, 1.0, 3), (4, 200, 30.0, 4)])
def test_group128_matches_reference_closed_form(T, H, std, seed):
    rng = np.random.default_rng(seed)
    x = oracle.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32) * np.float32(std))
    q, s = oracle.quant_group128(x)
    rq, rs = torch_group_quant(bf16_tensor(x))
    assert np.array_equal(s, rs)
    assert np.array_equal(q, rq)


def test_group128_known_answers():
    T, H = 4, 256
    x = np.zeros((T, H), np.float32)
    # row 0, group 0 all zero -> scale 1e-12, codes 0; group 1: single element 3.5
    x[0, 128 + 5] = 3.5
    # row 1: amax 448 -> scale exactly 1, codes are e4m3 of the values
    x[1, :4] = [448.0, 1.0625, 1.1875, -2.0]
    # row 2: amax 1.75 -> scale 1.75/448 = 2^-8 exactly; scaled values
    # 1.75*2^-4 (normal), 3.5*2^-9 and 2.5*2^-9 (subnormal ties -> even)
    x[2, 0] = 1.75
    x[2, 1] = 1.75 * 2.0 ** -12
    x[2, 2] = 1.75 * 2.0 ** -16
    x[2, 3] = 1.25 * 2.0 ** -16
    # row 3: negative tiny values that round to -0
    x[3, 0] = -1.0
    x[3, 1] = -1.0 / 448.0 * 2.0 ** -11
    bits = oracle.f32_to_bf16(x)
    q, s = oracle.quant_group128(bits)
    assert s[0, 0] == np.float32(1e-12) and np.all(q[0, :128] == 0)
    assert s[0, 1] == np.float32(3.5) / np.float32(448.0)
    assert q[0, 128 + 5] == 0x7E and np.all(np.delete(q[0, 128:], 5) == 0)
    assert s[1, 0] == 1.0
    assert q[1, :4].tolist() == [0x7E, 0x38, 0x3A, 0xC0]
    assert s[2, 0] == 2.0 ** -8
    assert q[2, 0] == 0x7E
    # 1.75 * 2^-4: exponent field -4 + 7 = 3, mantissa 0b110
    assert q[2, 1] == (3 << 3) | 0b110
    # subnormal step 2^-9: 3.5 steps -> 4 (0x04), 2.5 steps -> 2 (0x02)
    assert q[2, 2] == 0x04 and q[2, 3] == 0x02
    assert q[3, 0] == 0xFE and q[3, 1] == 0x80


def test_group128_qdq_close_for_small_values():
    # reference tests/test_golden.py:29-35
    x = (np.random.default_rng(6).standard_normal((3, 129)) * 0.01).astype(np.float32)
    qdq = oracle.group_quant_dequant(x)
    assert qdq.shape == x.shape
    assert np.abs(qdq - x).max() < 2e-3


def test_group_quant_dequant_equals_codes_times_scale():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((6, 256)).astype(np.float32)
    xb = oracle.bf16_to_f32(oracle.f32_to_bf16(x))
    q, s = oracle.quant_group128(oracle.f32_to_bf16(x))
    lut = oracle.e4m3_lut()
    assert np.array_equal(oracle.group_quant_dequant(xb), lut[q] * np.repeat(s, 128, axis=1))


def loop_quantize_block128(w: torch.Tensor):
    """Restatement of the reference's loop oracle (tests/test_quantize.py:9-24)."""
    E, N, K = w.shape
    nb, kb = (N + 127) // 128, (K + 127) // 128
    scale = torch.empty((E, nb, kb), dtype=torch.float32)
    fp8 = torch.empty_like(w, dtype=torch.float8_e4m3fn)
    for e in range(E):
        for ni in range(nb):
            for ki in range(kb):
                blk = w[e, ni * 128:(ni + 1) * 128, ki * 128:(ki + 1) * 128]
                sc = (blk.abs().amax() / FP8_MAX).clamp(min=1e-12)
                scale[e, ni, ki] = sc
                fp8[e, ni * 128:(ni + 1) * 128, ki * 128:(ki + 1) * 128] = \
                    (blk / sc).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return fp8.view(torch.uint8).numpy(), scale.numpy()


@pytest.mark.parametrize("shape,seed,std", [((2, 130, 65), 7, 0.01), ((3, 256, 384), 1, 0.02),
                                            ((1, 129, 257), 2, 5.0)])
def test_block128_matches_reference_loop_oracle(shape, seed, std):
    w = torch.randn(shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float32) * std
    q, s = oracle.quant_block128(w.numpy())
    rq, rs = loop_quantize_block128(w)
    assert s.shape == rs.shape
    assert np.array_equal(s, rs)
    assert np.array_equal(q, rq)


def test_block128_ragged_scale_shape_and_zero_block():
    w = np.zeros((1, 130, 65), np.float32)
    w[0, 129, 64] = -7.0
    q, s = oracle.quant_block128(w)
    assert s.shape == (1, 2, 1)
    assert s[0, 0, 0] == np.float32(1e-12)
    assert s[0, 1, 0] == np.float32(7.0) / np.float32(448.0)
    assert q[0, 129, 64] == 0xFE and np.count_nonzero(q) == 1


def test_dequant_block128_is_bf16_of_code_times_scale():
    # reference data/checkpoint.py:43-52 returns bf16 of fp8.float() * scale
    w = torch.randn((2, 130, 200), generator=torch.Generator().manual_seed(9)) * 0.03
    q, s = oracle.quant_block128(w.numpy())
    got = oracle.dequant_block128(q, s)
    qt = torch.from_numpy(q).view(torch.float8_e4m3fn).float()
    st = torch.from_numpy(s).repeat_interleave(128, 1).repeat_interleave(128, 2)[:, :130, :200]
    ref = (qt * st).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert got.shape == (2, 130, 200)
    assert np.array_equal(got, ref)
