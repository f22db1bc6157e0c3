"""GPU: the prebuilt layer at the bench's full DeepSeek-V3 shape (T=8192,
H=7168, I=2048, E=256, top-8, block_size_m 128, 256-row GEMM tiles).

The CPU oracle cannot run this layer whole (5.8 TFLOP), so the checks are the
ones that hold at any size:
* align: the padded-cumsum closed form of ntpp and of every block's expert,
  every slot placed exactly once, padding = S (overlap/kernels.py:105-120);
* reduce: the layer output equals the oracle's top-k sum over the GPU's own
  D rows, bit for bit (overlap_forward.py:304-313);
* sampled tokens: y for a seeded sample of tokens against the fp32 golden
  (verify.py:14-47) restricted to those tokens' experts, through the three
  gates (worker.py:107-146) and max-abs-rel <= 2e-2 (the north-star bound
  from tests/calibrate_tolerance.py).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from moe_cases import bf16_bits

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def dsv3():
    from td_benchmark_amd import ops, workloads
    wl = workloads.CONFIGS["dsv3"]
    print("case: full-size dsv3 layer", flush=True)
    d = workloads.generate(wl, "cuda")
    runner = ops.FusedExpertsRunner(d.w13, d.w13_s, d.w2, d.w2_s, wl.T, wl.top_k, wl.block_m)
    y = runner.run(d.x, d.topk_w, d.topk_ids)
    torch.cuda.synchronize()
    print(f"  gemm tile height {ops.gemm_tile_rows(runner.BM, runner.S, runner.E, runner.tile_m)}", flush=True)
    return wl, d, runner, y


def test_align_closed_form_at_full_size(dsv3):
    wl, d, runner, _ = dsv3
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


def test_reduce_is_the_topk_sum_of_d(dsv3):
    wl, d, runner, y = dsv3
    D = bf16_bits(runner.D[: wl.S])
    assert np.array_equal(bf16_bits(y), oracle.moe_reduce(D, wl.T, wl.top_k))


def test_sampled_tokens_meet_the_golden_gates(dsv3):
    wl, d, runner, y = dsv3
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
    golden = oracle.golden_moe(x, ids, d.topk_w.cpu().numpy()[tokens], dequant(d.w13, d.w13_s),
                               dequant(d.w2, d.w2_s), experts=experts)
    got = oracle.bf16_to_f32(bf16_bits(y)[tokens])
    rep = oracle.compare_outputs(got, golden, atol=0.0, rtol=0.0, **oracle.DEFAULT_GATES)
    print(f"  {rep}", flush=True)
    assert rep["pass"], rep
    assert rep["max_abs_rel"] <= 2e-2, rep
