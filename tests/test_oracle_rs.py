"""CPU: pinning the oracle's combine of the FP8-compressed reduce-scatter leg.

The reference dequantises and sums the FP8 chunks a rank receives with torch
(moe_bench/overlap/overlap_forward.py:932-944):

    fp8_f32 = fp8_3d.to(torch.float32)
    scale_expanded = scale_3d.repeat_interleave(128, dim=2)[:, :, :N]
    out = (fp8_f32 * scale_expanded).sum(dim=0).to(torch.bfloat16)

That expression is evaluated here by torch itself (its own float8 decode,
fp32 products, reduction and bf16 rounding) and compared with the C oracle,
and closed forms pin the scale indexing: a wrong 128-column group, a rank's
scale row taken from the wrong rank or row, or a dropped rank each fail one of
them."""
from __future__ import annotations

import numpy as np
import pytest

import oracle

torch = pytest.importorskip("torch")


def _codes(rng, shape):
    """Random e4m3 codes without the two NaN codes (the senders clamp to +-448)."""
    q = rng.integers(0, 256, size=shape, dtype=np.uint8)
    q[(q & 0x7F) == 0x7F] = 0x38
    return q


def _torch_reference(q, s3, N):
    fp8_f32 = torch.from_numpy(q).view(torch.float8_e4m3fn).to(torch.float32)
    scale_expanded = torch.from_numpy(s3).repeat_interleave(128, dim=2)[:, :, :N]
    out = (fp8_f32 * scale_expanded).sum(dim=0).to(torch.bfloat16)
    return out.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("R,M,N", [(1, 3, 16), (2, 5, 144), (4, 7, 256), (8, 9, 384), (12, 4, 272)])
def test_oracle_matches_the_reference_expression(R, M, N):
    rng = np.random.default_rng(R * 100 + N)
    q = _codes(rng, (R, M, N))
    G = (N + 127) // 128
    s3 = (rng.random((R, M, G), dtype=np.float32) * 0.05 + 1e-4).astype(np.float32)
    got = oracle.fp8_dequant_sum(q, s3.reshape(R * M, G))
    want = _torch_reference(q, s3, N)
    assert np.array_equal(got, want)


def test_scale_groups_ranks_and_rows_closed_form():
    # q = 1.0 everywhere; s[r, m, g] = 2^g * (r + 1) * (m + 1) / 64 (exact in
    # fp32 and bf16 for these sizes): out[m, n] = 2^(n//128) * (m+1) * R(R+1)/2 / 64.
    R, M, N = 3, 4, 384
    q = np.full((R, M, N), 0x38, np.uint8)  # e4m3 1.0
    s3 = np.empty((R, M, 3), np.float32)
    for r in range(R):
        for m in range(M):
            for g in range(3):
                s3[r, m, g] = 2.0 ** g * (r + 1) * (m + 1) / 64.0
    got = oracle.bf16_to_f32(oracle.fp8_dequant_sum(q, s3.reshape(R * M, 3)))
    n = np.arange(N)
    want = np.array([[2.0 ** (nn // 128) * (m + 1) * (R * (R + 1) / 2) / 64.0 for nn in n] for m in range(M)])
    assert np.array_equal(got, want.astype(np.float32))


def test_single_rank_is_one_rounding_of_each_product():
    # With one rank the sum is its product rounded once to bf16, except that a
    # -0 product comes out +0: a sum starts from +0, as torch's sum does
    # (torch.tensor([[-0.0]]).sum(dim=0) is +0).
    rng = np.random.default_rng(3)
    q = _codes(rng, (1, 6, 128))
    q[0, 0, :4] = 0x80  # -0
    s = (rng.random((6, 1), dtype=np.float32) + 0.5).astype(np.float32)
    got = oracle.fp8_dequant_sum(q, s)
    prod = torch.from_numpy(q[0]).view(torch.float8_e4m3fn).to(torch.float32) * torch.from_numpy(s)
    want = prod.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16).copy()
    want[want == 0x8000] = 0
    assert np.array_equal(got, want)
    assert not np.any(got == 0x8000)


def test_wider_scale_rows_and_output_rows():
    # scale rows wider than ceil(N/128) (the reference's padded scale buffers)
    # and an output row stride wider than N (a column slice of the concatenated
    # output): only the first ceil(N/128) scales and N columns take part.
    rng = np.random.default_rng(9)
    R, M, N = 2, 3, 144
    q = _codes(rng, (R, M, N))
    s_pad = rng.random((R * M, 5), dtype=np.float32)
    got = oracle.fp8_dequant_sum(q, s_pad, out_ld=160)
    want = oracle.fp8_dequant_sum(q, np.ascontiguousarray(s_pad[:, :2]))
    assert np.array_equal(got[:, :N], want)
    assert not got[:, N:].any()
