"""GPU: the prebuilt layer at the bench's full shapes: DeepSeek-V3 (T=8192,
H=7168, I=2048, E=256, top-8, 256-row GEMM tiles), Mixtral, Qwen3 (one pass)
and the skewed DSv3 decode batch, each with its benchmark seed.

The CPU oracle cannot run these layers whole (5.8 TFLOP at DSv3), so the checks are the
ones that hold at any size:
* align: the padded-cumsum closed form of ntpp and of every block's expert,
  every slot placed exactly once, padding = S (overlap/kernels.py:105-120);
* reduce: the layer output equals the oracle's top-k sum over the GPU's own
  D rows, bit for bit (overlap_forward.py:304-313);
* sampled tokens: y for a seeded sample of tokens through the three gates
  (worker.py:107-146) against the fp32 golden (verify.py:14-47) restricted to
  those tokens' experts, and within max-abs-rel 2e-2 of the fp32 reference
  on the dequantised FP8 operands the path consumed (the bound of the layer
  tests, which isolates the kernels' arithmetic from FP8 rounding-decision
  flips at the intermediate quant).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from moe_cases import bf16_bits

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", params=["dsv3", "mixtral", "qwen3", "dsv3_decode"])
def layer(request):
    from td_benchmark_amd import ops, workloads
    wl = workloads.CONFIGS[request.param]
    print(f"case: full-size {wl.name} layer", flush=True)
    d = workloads.generate(wl, "cuda")
    runner = ops.FusedExpertsRunner(d.w13, d.w13_s, d.w2, d.w2_s, wl.T, wl.top_k, wl.block_m)
    y = runner.run(d.x, d.topk_w, d.topk_ids)
    torch.cuda.synchronize()
    print(f"  gemm tile height {ops.gemm_tile_rows(runner.BM, runner.S, runner.E, runner.tile_m)}", flush=True)
    return wl, d, runner, y


def test_align_closed_form_at_full_size(layer):
    wl, d, runner, _ = layer
    ids = d.topk_ids.cpu().numpy().ravel()
    S, E, BM = ids.size, wl.E, wl.block_m
    counts = np.bincount(ids, minlength=E)
    padded = (counts + BM - 1) // BM * BM
    ntpp = int(runner.align.ntpp.item())
    assert ntpp == int(padded.sum())
    srt = runner.align.sorted_ids.cpu().numpy()[:ntpp]
    eids = runner.align.expert_ids.cpu().numpy()[: ntpp // BM]
    assert np.array_equal(eids, np.repeat(np.arange(E), padded // BM))
    valid = srt < S
    assert np.array_equal(np.sort(srt[valid]), np.arange(S))     # every slot exactly once
    assert np.all(srt[~valid] == S)                                # padding value
    assert np.all(ids[srt[valid]] == np.repeat(eids, BM)[valid])   # slot sits in its expert's blocks


def test_reduce_is_the_topk_sum_of_d(layer):
    wl, d, runner, y = layer
    D = bf16_bits(runner.D[: wl.S])
    assert np.array_equal(bf16_bits(y), oracle.moe_reduce(D, wl.T, wl.top_k))


def test_sampled_tokens_meet_the_golden_gates(layer):
    wl, d, runner, y = layer
    rng = np.random.default_rng(2024)
    tokens = np.sort(rng.choice(wl.T, size=4, replace=False))
    ids = d.topk_ids.cpu().numpy()[tokens]
    experts = np.unique(ids)
    print(f"  golden for tokens {tokens.tolist()} over {experts.size} experts", flush=True)

    def dequant(w, s):
        def get(e):
            q = w[e : e + 1].view(torch.uint8).cpu().numpy()
            return oracle.bf16_to_f32(oracle.dequant_block128(q, s[e : e + 1].cpu().numpy()))[0]
        return get

    x = oracle.bf16_to_f32(bf16_bits(d.x[torch.from_numpy(tokens).cuda()]))
    wts = d.topk_w.cpu().numpy()[tokens]
    golden = oracle.golden_moe(x, ids, wts, dequant(d.w13, d.w13_s), dequant(d.w2, d.w2_s), experts=experts)
    got = oracle.bf16_to_f32(bf16_bits(y)[tokens])
    rep = oracle.compare_outputs(got, golden, atol=0.0, rtol=0.0, **oracle.DEFAULT_GATES)
    print(f"  golden: {rep}", flush=True)
    assert rep["pass"], rep

    # the sampled slots' intermediate codes and scales, found by sorted position
    ntpp = int(runner.align.ntpp.item())
    srt = runner.align.sorted_ids.cpu().numpy()[:ntpp]
    pos_of = np.full(wl.S, -1, np.int64)
    valid = np.nonzero(srt < wl.S)[0]
    pos_of[srt[valid]] = valid
    slots = (tokens[:, None] * wl.top_k + np.arange(wl.top_k)).ravel()
    pos = torch.from_numpy(pos_of[slots]).cuda()
    hq = runner.hq[pos].view(torch.uint8).cpu().numpy()
    hs = runner.hs[pos].cpu().numpy()

    class PerExpert:  # w[e] fetched from the device when the reference asks for it
        def __init__(self, t):
            self.t, self.shape = t, tuple(t.shape)

        def __getitem__(self, e):
            t = self.t[e]
            return (t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t).cpu().numpy()

    ref = oracle.dequant_reference(hq, hs, ids, wts, PerExpert(d.w2), PerExpert(d.w2_s))
    rep = oracle.compare_outputs(got, ref, atol=0.0, rtol=0.0)
    print(f"  fp32 on the consumed operands: max-abs-rel {rep['max_abs_rel']:.4f}", flush=True)
    assert rep["max_abs_rel"] <= oracle.MAX_ABS_REL, rep


@pytest.mark.parametrize("layer", ["qwen3"], indirect=True)
def test_chunked_pipeline_equals_one_pass(layer):
    """Config 5 at its own size: the 4-chunk x 2-stream pipeline of the Qwen3
    layer (T=16384; every chunk's experts average 256 slots, so each chunk runs
    256-row tiles with the activation scales by sorted position) gives the
    one-pass runner's output bit for bit, on two runs in a row
    (overlap_forward.py:252-342: chunks on side streams, joined before return)."""
    wl, d, runner, y = layer
    assert wl.n_chunks > 1
    from td_benchmark_amd import ops
    ch = ops.ChunkedExpertsRunner(d.w13, d.w13_s, d.w2, d.w2_s, wl.T, wl.top_k, wl.n_chunks, wl.n_streams,
                                  wl.block_m)
    tm = [ops.gemm_tile_rows(r.BM, r.S, r.E, r.tile_m) for r in ch.runners]
    print(f"  chunks {ch.bounds}, tile heights {tm}, scales by position "
          f"{[r.scales_by_position for r in ch.runners]}", flush=True)
    assert all(t == 256 for t in tm) and all(r.scales_by_position for r in ch.runners)
    want = bf16_bits(y)
    for _ in range(2):
        got = ch.run(d.x, d.topk_w, d.topk_ids)
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(got), want)
