"""GPU: hidden sizes that are not a multiple of 128, through the C ABI.

The reference's quant zero-pads a row to a multiple of 128 and slices the
result back (verify.py:108-117), and its weight quant zero-pads a ragged
128x128 block (data/checkpoint.py:28-40).  Here:
* moe_quant_group128 at ragged widths is bit-exact against the oracle (codes
  and scales, whose last group holds H mod 128 values), and
  moe_quant_group128_padded writes the same codes with the zero code in the
  padding columns;
* FusedExpertsRunner and SharedExpertRunner at a ragged H give, bit for bit,
  the first H columns of the same layer run at the padded width on inputs and
  weights that carry explicit zeros in the padding (the reference's padding
  made explicit), and the layer passes the reference worker's gates against
  the golden.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from moe_cases import bf16_bits, dequant_weights_f32, make_case, to_gpu, u8_bits

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.mark.parametrize("T,H", [(5, 1), (7, 100), (33, 129), (16, 200), (9, 300), (64, 7168 + 64)])
def test_quant_ragged_width_bit_exact(T, H):
    from td_benchmark_amd import ops
    from td_benchmark_amd._lib import check, lib
    print(f"case: ragged quant T={T} H={H}", flush=True)
    rng = np.random.default_rng(T * 1000 + H)
    x = oracle.f32_to_bf16(rng.standard_normal((T, H), dtype=np.float32))
    x[0, : min(H, 128)] = 0                # an all-zero group
    q_ref, s_ref = oracle.quant_group128(x)
    dx = torch.from_numpy(x.view(np.int16)).cuda().view(torch.bfloat16)
    q, s = ops.per_token_group_quant_fp8(dx)
    hp = (H + 127) // 128 * 128
    qp = torch.full((T, hp + 16), 0x55, dtype=torch.uint8, device="cuda")
    sp = torch.empty((T, hp // 128), dtype=torch.float32, device="cuda")
    check(lib().moe_quant_group128_padded(ops._ptr(dx), T, H, ops._ptr(qp), hp + 16, ops._ptr(sp), None), "padded")
    torch.cuda.synchronize()
    np.testing.assert_array_equal(u8_bits(q), q_ref)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    qp = qp.cpu().numpy()
    np.testing.assert_array_equal(qp[:, :H], q_ref)
    assert (qp[:, H:hp] == 0).all() and (qp[:, hp:] == 0x55).all()
    np.testing.assert_array_equal(sp.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))


def _padded_case(c, Hp):
    """The case with explicit zeros: x [T, Hp], W13 [E, 2I, Hp], W2 [E, Hp, I]
    (the weight scales keep their block counts)."""
    T, H = c.x.shape
    x = np.zeros((T, Hp), np.uint16)
    x[:, :H] = c.x
    w13 = np.zeros(c.w13_q.shape[:2] + (Hp,), np.uint8)
    w13[:, :, :H] = c.w13_q
    w2 = np.zeros((c.w2_q.shape[0], Hp, c.w2_q.shape[2]), np.uint8)
    w2[:, :H] = c.w2_q
    return x, w13, w2


@pytest.mark.parametrize("T,H,I,E,k,BM,routing", [
    (64, 200, 256, 8, 2, 64, "softmax"),
    (128, 300, 256, 16, 4, 32, "zipf"),
    (1024, 384 + 100, 256, 8, 2, 128, "sigmoid"),   # S >= 160 E: 256-row tiles, scales by position
])
def test_ragged_layer_equals_the_explicitly_padded_layer(T, H, I, E, k, BM, routing):
    from td_benchmark_amd import ops
    print(f"case: ragged layer T={T} H={H} I={I} E={E} k={k} BM={BM}", flush=True)
    c = make_case(T, H, I, E, k, BM, seed=T + H, routing=routing)
    g = to_gpu(c)
    Hp = (H + 127) // 128 * 128
    r = ops.FusedExpertsRunner(g["w13"], g["w13_s"], g["w2"], g["w2_s"], T, k, BM)
    y = bf16_bits(r.run(g["x"], g["topk_w"], g["topk_ids"]))
    xp, w13p, w2p = _padded_case(c, Hp)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    rp = ops.FusedExpertsRunner(dev(w13p).view(ops.FP8), g["w13_s"], dev(w2p).view(ops.FP8), g["w2_s"], T, k, BM)
    yp = bf16_bits(rp.run(dev(xp.view(np.int16)).view(torch.bfloat16), g["topk_w"], g["topk_ids"]))
    torch.cuda.synchronize()
    assert y.shape == (T, H)
    np.testing.assert_array_equal(y, yp[:, :H])
    assert (yp[:, H:] == 0).all()
    # and the layer meets the reference worker's gates against the golden
    x32 = oracle.bf16_to_f32(c.x)
    w1 = dequant_weights_f32(c.w13_q, c.w13_s)
    w2 = dequant_weights_f32(c.w2_q, c.w2_s)
    golden = oracle.golden_moe(x32, c.topk_ids, c.topk_w, w1, w2)
    rep = oracle.compare_outputs(oracle.bf16_to_f32(y), golden, atol=0.2, rtol=0.0, **oracle.DEFAULT_GATES)
    assert rep["pass"], rep
    atol = oracle.calibrated_atol(x32, c.topk_ids, c.topk_w, w1, w2)
    assert rep["max_abs"] <= atol, (rep, atol)


def test_ragged_shared_expert_equals_the_explicitly_padded_one():
    from td_benchmark_amd import ops
    print("case: ragged shared expert", flush=True)
    T, H, I = 96, 300, 256
    Hp = 384
    rng = np.random.default_rng(3)
    x = oracle.f32_to_bf16(rng.standard_normal((T, H), dtype=np.float32))
    w1q, w1s = oracle.quant_block128((rng.standard_normal((1, 2 * I, H)) * H ** -0.5).astype(np.float32))
    w2q, w2s = oracle.quant_block128((rng.standard_normal((1, H, I)) * I ** -0.5).astype(np.float32))
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    sh = ops.SharedExpertRunner(dev(w1q).view(ops.FP8), dev(w1s), dev(w2q).view(ops.FP8), dev(w2s), T)
    y = bf16_bits(sh(dev(x.view(np.int16)).view(torch.bfloat16)).contiguous())
    w1p = np.zeros((1, 2 * I, Hp), np.uint8)
    w1p[:, :, :H] = w1q
    w2p = np.zeros((1, Hp, I), np.uint8)
    w2p[:, :H] = w2q
    xp = np.zeros((T, Hp), np.uint16)
    xp[:, :H] = x
    shp = ops.SharedExpertRunner(dev(w1p).view(ops.FP8), dev(w1s), dev(w2p).view(ops.FP8), dev(w2s), T)
    yp = bf16_bits(shp(dev(xp.view(np.int16)).view(torch.bfloat16)))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y, yp[:, :H])


def test_split_runner_rejects_a_ragged_width():
    from td_benchmark_amd import ops
    c = make_case(16, 200, 128, 4, 2, 16, seed=1)
    g = to_gpu(c)
    with pytest.raises(ValueError, match="multiples of 128"):
        ops.SplitExpertsRunner(g["w13"], g["w13_s"], g["w2"], g["w2_s"], 16, 2, 2, 2, 16)
