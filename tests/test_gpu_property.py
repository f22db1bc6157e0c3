"""GPU: randomised parity of align (A3) and the 1x128 quant (A1) against the
oracle, through the C ABI.

Hypothesis (derandomised, so every run sees the same cases) draws routings
with empty experts, skew and ids outside [0, E) for moe_align_block_size
(overlap_forward.py:165-169), and bf16 bit patterns covering every finite
value for per_token_group_quant_fp8 (verify.py:108-117).  Both must equal the
oracle bit for bit: sorted_token_ids and expert_ids up to ntpp, ntpp, codes
and scales.
"""
from __future__ import annotations

import numpy as np
import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

import oracle
from moe_cases import u8_bits

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@st.composite
def routings(draw):
    E = draw(st.integers(1, 64))
    k = draw(st.integers(1, 8))
    T = draw(st.integers(1, 300))
    BM = draw(st.sampled_from([16, 32, 64, 128]))
    hot = draw(st.integers(0, E - 1))
    skew = draw(st.floats(0.0, 0.9))
    seed = draw(st.integers(0, 2**31 - 1))
    rng = np.random.default_rng(seed)
    ids = rng.integers(-1, E + 1, size=(T, k)).astype(np.int32)
    ids[rng.random((T, k)) < skew] = hot  # a hot expert; duplicates within a token are allowed
    return ids, E, BM


@settings(max_examples=60, deadline=None, derandomize=True)
@given(routings())
def test_gpu_align_matches_oracle_on_random_routings(case):
    from td_benchmark_amd import ops
    ids, E, BM = case
    sorted_ids, eids, ntpp = ops.moe_align_block_size(torch.from_numpy(ids).cuda(), BM, E)
    torch.cuda.synchronize()
    r_sorted, r_eids, r_ntpp = oracle.moe_align(ids.ravel(), E, BM)
    n = int(ntpp.item())
    assert n == r_ntpp
    assert np.array_equal(sorted_ids.cpu().numpy()[:n], r_sorted[:n])
    assert np.array_equal(eids.cpu().numpy()[: n // BM], r_eids[: n // BM])


@st.composite
def activations(draw):
    T = draw(st.integers(1, 40))
    G = draw(st.integers(1, 6))
    seed = draw(st.integers(0, 2**31 - 1))
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 0x10000, size=(T, 128 * G), dtype=np.uint32).astype(np.uint16)
    bits[(bits & 0x7F80) == 0x7F80] &= 0x8000          # finite values only
    if draw(st.booleans()):
        bits[:, ::2] = (bits[:, ::2] & 0x807F) | 0x3F00  # dense groups near 1.0
    if draw(st.booleans()):
        bits[rng.integers(0, T), :] = 0                 # an all-zero row
    return bits


@settings(max_examples=60, deadline=None, derandomize=True)
@given(activations())
def test_gpu_quant_matches_oracle_on_random_bits(bits):
    from td_benchmark_amd import ops
    x = torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16)
    q, s = ops.per_token_group_quant_fp8(x)
    torch.cuda.synchronize()
    rq, rs = oracle.quant_group128(bits)
    assert np.array_equal(u8_bits(q), rq)
    assert np.array_equal(s.cpu().numpy(), rs)


@st.composite
def expert_rows(draw):
    T = draw(st.integers(1, 40))
    k = draw(st.integers(1, 32))
    H = 8 * draw(st.integers(1, 64))
    seed = draw(st.integers(0, 2**31 - 1))
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 0x10000, size=(T * k + T, H), dtype=np.uint32).astype(np.uint16)
    exp = (bits >> 7) & 0xFF
    bits = np.where(exp > 0xE3, (bits & 0x807F) | (0xE3 << 7), bits).astype(np.uint16)  # |v| < 2^101: no overflow
    return bits[: T * k], bits[T * k :], T, k, draw(st.booleans())


@settings(max_examples=60, deadline=None, derandomize=True)
@given(expert_rows())
def test_gpu_reduce_matches_oracle_on_random_rows(case):
    """moe_sum (overlap_forward.py:304-313), with and without the shared
    expert's addend (schemes/vllm_tp.py:62-63): bit-exact with the oracle."""
    from td_benchmark_amd import ops
    D, add, T, k, with_add = case
    dev = lambda b: torch.from_numpy(b.view(np.int16)).cuda().view(torch.bfloat16)  # noqa: E731
    y = torch.empty((T, D.shape[1]), dtype=torch.bfloat16, device="cuda")
    ops.moe_sum(dev(D), y, k, addend=dev(add) if with_add else None)
    torch.cuda.synchronize()
    want = oracle.moe_reduce(D, T, k)
    if with_add:
        want = oracle.f32_to_bf16(oracle.bf16_to_f32(want) + oracle.bf16_to_f32(add))
    assert np.array_equal(u8_bits(y).view(np.uint16), want)


@st.composite
def rs_chunks(draw):
    R = draw(st.integers(1, 64))
    M = draw(st.integers(1, 24))
    N = 16 * draw(st.integers(1, 40))
    G = (N + 127) // 128 + draw(st.integers(0, 2))        # scale rows may be wider
    ld = N + 8 * draw(st.integers(0, 4))                    # a column slice of a wider output
    seed = draw(st.integers(0, 2**31 - 1))
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 256, size=(R, M, N), dtype=np.uint8)
    q[(q & 0x7F) == 0x7F] = 0                               # the senders clamp to +-448: no NaN codes
    s = (rng.random((R * M, G), dtype=np.float32) * 0.05 + 1e-4).astype(np.float32)
    return q, s, ld


@settings(max_examples=40, deadline=None, derandomize=True)
@given(rs_chunks())
def test_gpu_fp8_combine_matches_oracle_on_random_chunks(case):
    """The combine after the FP8 reduce-scatter (overlap_forward.py:932-944)."""
    from td_benchmark_amd import ops
    q, s, ld = case
    R, M, N = q.shape
    full = torch.zeros((M, ld), dtype=torch.bfloat16, device="cuda")
    qd = torch.from_numpy(q).cuda().view(torch.float8_e4m3fn)
    ops.fp8_dequant_sum(qd, torch.from_numpy(s).cuda(), out=full[:, :N])
    torch.cuda.synchronize()
    assert np.array_equal(u8_bits(full[:, :N]).view(np.uint16), oracle.fp8_dequant_sum(q, s))
