"""GPU: the layer at the edges of its token count, through the C ABI.

* No tokens: every layer entry (``fused_experts``, the one-pass, token-chunk
  and K/N-split runners) returns a [0, H] output and launches nothing that
  reads an empty operand; the C entry points return before their pointer
  checks when there is nothing to compute (empty tensors have null pointers).
* One token with k = 8 of 64 experts: every align block then holds a single
  valid row, so every GEMM tile runs one 16-row subtile of which 15 rows are
  padding.  The output is held to the bars of the layer suite: the reference
  worker's three gates and the calibrated bound against the fp8-sim golden
  (moe_bench/verify.py:14-47, worker.py:107-110), and max-abs-rel 2e-2 against
  the fp32 reference on the dequantised operands the path consumed.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from moe_cases import bf16_bits, dequant_weights_f32, make_case, to_gpu, u8_bits

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

H, I, E, K = 512, 256, 64, 8


def _weights():
    c = make_case(1, H, I, E, K, 32, seed=11, routing="sigmoid")
    return c, to_gpu(c)


@pytest.mark.parametrize("entry", ["fused_experts", "one_pass_bm32", "one_pass_bm128", "chunked", "split"])
def test_no_tokens_gives_an_empty_output(entry):
    from td_benchmark_amd import ops

    print(f"case: no tokens, {entry}", flush=True)
    _, g = _weights()
    x = torch.empty((0, H), dtype=torch.bfloat16, device="cuda")
    w = torch.empty((0, K), dtype=torch.float32, device="cuda")
    ids = torch.empty((0, K), dtype=torch.int32, device="cuda")
    if entry == "fused_experts":
        y = ops.fused_experts(x, g["w13"], g["w2"], w, ids, E, w1_scale=g["w13_s"], w2_scale=g["w2_s"])
    elif entry.startswith("one_pass"):
        bm = int(entry[len("one_pass_bm"):])
        y = ops.FusedExpertsRunner(g["w13"], g["w13_s"], g["w2"], g["w2_s"], 0, K, bm).run(x, w.view(-1),
                                                                                             ids.view(-1))
    elif entry == "chunked":
        y = ops.ChunkedExpertsRunner(g["w13"], g["w13_s"], g["w2"], g["w2_s"], 0, K, 4, 2).run(x, w, ids)
    else:
        y = ops.SplitExpertsRunner(g["w13"], g["w13_s"], g["w2"], g["w2_s"], 0, K, 2, 2).run(x, w, ids)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (0, H) and y.dtype == torch.bfloat16


def _slot_intermediate(runner, S):
    """The runner's intermediate FP8 codes and scales, by slot."""
    ntpp = int(runner.align.ntpp.item())
    srt = runner.align.sorted_ids.cpu().numpy()[:ntpp]
    pos = np.nonzero(srt < S)[0]
    slots = srt[pos]
    assert np.array_equal(np.sort(slots), np.arange(S)), "every slot must be placed once"
    hq, hs = u8_bits(runner.hq), runner.hs.cpu().numpy()
    hq_slot = np.zeros((S, hq.shape[1]), np.uint8)
    hs_slot = np.zeros((S, hs.shape[1]), np.float32)
    hq_slot[slots] = hq[pos]
    hs_slot[slots] = hs[pos]
    return hq_slot, hs_slot


@pytest.mark.parametrize("bm", [16, 32, 128])
def test_one_token_meets_the_layer_bars(bm):
    from td_benchmark_amd import ops

    print(f"case: one token, k={K} of E={E}, BM={bm}", flush=True)
    c, g = _weights()
    runner = ops.FusedExpertsRunner(g["w13"], g["w13_s"], g["w2"], g["w2_s"], 1, K, bm)
    y = runner.run(g["x"], g["topk_w"].view(-1), g["topk_ids"].view(-1))
    torch.cuda.synchronize()
    assert int(runner.align.ntpp.item()) == K * bm, "one block per routed expert"
    y_np = oracle.bf16_to_f32(bf16_bits(y))
    x32 = oracle.bf16_to_f32(c.x)
    w1 = dequant_weights_f32(c.w13_q, c.w13_s)
    w2 = dequant_weights_f32(c.w2_q, c.w2_s)
    golden = oracle.golden_moe(x32, c.topk_ids, c.topk_w, w1, w2)
    rep = oracle.compare_outputs(y_np, golden, atol=0.2, rtol=0.0, **oracle.DEFAULT_GATES)
    assert rep["pass"], rep
    atol = oracle.calibrated_atol(x32, c.topk_ids, c.topk_w, w1, w2)
    assert rep["max_abs"] <= atol, (rep, atol)
    hq_slot, hs_slot = _slot_intermediate(runner, c.S)
    ref32 = oracle.dequant_reference(hq_slot, hs_slot, c.topk_ids, c.topk_w, c.w2_q, c.w2_s)
    rep32 = oracle.compare_outputs(y_np, ref32, atol=0.0, rtol=0.0)
    assert rep32["max_abs_rel"] <= oracle.MAX_ABS_REL, rep32


def test_one_token_split_runner_meets_the_golden_gates():
    from td_benchmark_amd import ops

    print("case: one token, split runner 2x2", flush=True)
    c, g = _weights()
    y = ops.SplitExpertsRunner(g["w13"], g["w13_s"], g["w2"], g["w2_s"], 1, K, 2, 2).run(
        g["x"], g["topk_w"], g["topk_ids"])
    torch.cuda.synchronize()
    x32 = oracle.bf16_to_f32(c.x)
    w1 = dequant_weights_f32(c.w13_q, c.w13_s)
    w2 = dequant_weights_f32(c.w2_q, c.w2_s)
    golden = oracle.golden_moe(x32, c.topk_ids, c.topk_w, w1, w2)
    rep = oracle.compare_outputs(oracle.bf16_to_f32(bf16_bits(y)), golden, atol=0.2, rtol=0.0,
                                 **oracle.DEFAULT_GATES)
    assert rep["pass"], rep
    assert rep["max_abs"] <= oracle.calibrated_atol(x32, c.topk_ids, c.topk_w, w1, w2), rep
