"""GPU: the reference pipeline's compute-stream structure (ops.SplitExpertsRunner;
overlap/overlap_forward.py:252-313 without the communication legs) against
the CPU oracle, stage by stage, on the runner's own intermediates:

* C13 from the K-split W13 chunks (bf16 accumulate, overlap/kernels.py:
  317-452) against the oracle's composition of per-chunk bf16 partials,
  C = bf16(C + bf16(partial)), within the FP8-MFMA accumulation bound;
* h = silu_and_mul(C13) on the GPU's C13, <= 1 bf16 ulp on <= 0.1 %
  (overlap_forward.py:277-279);
* hq, hs = 1x128 quant of the GPU's h, bit-exact (overlap_forward.py:282-284);
* D from the N-split W2 chunks with routed weights (rows by slot, top_k=1)
  against the oracle GEMM on the GPU's hq, hs, within the GEMM bound
  (overlap_forward.py:289-302);
* y = top-k sum of the GPU's D, bit-exact (overlap_forward.py:304-313);
* the layer output through the reference worker's three gates and the
  calibrated bound against the fp8-sim golden (verify.py:14-47).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from moe_cases import bf16_bits, dequant_weights_f32, make_case, to_gpu, u8_bits

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

# (T, H, I, E, k, BM, n_gateup, n_down): 32-row tiles; S >= 160*E (256-row tiles over 64-row blocks);
# and 256-row blocks whose experts' second tiles hold 90, 91, 47 and 92 valid rows (the 128-row and
# 64-row bodies of a 256-row launch, with the K-split accumulate epilogue)
CASES = {"short": (150, 512, 384, 6, 3, 32, 4, 2), "tall": (700, 512, 256, 4, 2, 64, 2, 4),
         "body128": (672, 512, 256, 4, 2, 256, 2, 4)}


@pytest.mark.parametrize("name", sorted(CASES))
def test_split_runner_matches_the_oracle_stage_by_stage(name):
    from td_benchmark_amd import ops

    T, H, I, E, k, BM, ng, nd = CASES[name]
    print(f"case: split runner {name} T={T} H={H} I={I} E={E} k={k} BM={BM} chunks {ng}x{nd}", flush=True)
    c = make_case(T, H, I, E, k, BM, seed=T + E)
    g = to_gpu(c)
    r = ops.SplitExpertsRunner(g["w13"], g["w13_s"], g["w2"], g["w2_s"], T, k, ng, nd, BM)
    assert len(r.k_bounds) == ng and len(r.n_bounds) == nd
    y = r.run(g["x"], g["topk_w"], g["topk_ids"])
    torch.cuda.synchronize()
    S = c.S
    srt = r.align.sorted_ids.cpu().numpy()
    eids = r.align.expert_ids.cpu().numpy()
    nt = int(r.align.ntpp.item())
    placed = srt[:nt][srt[:nt] < S]
    assert np.array_equal(np.sort(placed), np.arange(S))

    # 1) C13: oracle composition of the K chunks' bf16 partials
    q1, s1 = u8_bits(r.q1), r.s1.cpu().numpy()
    q_ref, s_ref = oracle.quant_group128(c.x)
    assert np.array_equal(q1, q_ref) and np.array_equal(s1.view(np.uint32), s_ref.view(np.uint32))
    ref = None
    bnd = np.zeros((S, 2 * I), np.float64)
    abs_parts = np.zeros((S, 2 * I), np.float64)
    for k0, k1 in r.k_bounds:
        part, m = oracle.grouped_gemm(q1[:, k0:k1], s1[:, k0 // 128:k1 // 128], c.w13_q[:, :, k0:k1],
                                      c.w13_s[:, :, k0 // 128:k1 // 128], srt, eids, nt, BM, S, k,
                                      with_bound=True)
        bnd += m
        abs_parts += np.abs(oracle.bf16_to_f32(part))
        ref = part if ref is None else oracle.f32_to_bf16(oracle.bf16_to_f32(ref) + oracle.bf16_to_f32(part))
    c13 = bf16_bits(r.C13[:S])
    g32, r32 = oracle.bf16_to_f32(c13).astype(np.float64), oracle.bf16_to_f32(ref).astype(np.float64)
    tol = 2.0 ** -7 * (np.abs(r32) + abs_parts) + bnd + 1e-30
    bad = np.abs(g32 - r32) > tol
    assert not bad.any(), f"C13: {int(bad.sum())} of {bad.size} outside the bound"

    # 2) h on the GPU's C13
    h = bf16_bits(r.h[:S])
    h_ref = oracle.silu_and_mul(c13)
    diff = h != h_ref
    assert diff.mean() <= 1e-3, diff.mean()
    ulps = np.abs(h.astype(np.int32) - h_ref.astype(np.int32))
    assert ulps[diff].max(initial=0) <= 1

    # 3) quant of the GPU's h, bit-exact
    hq_ref, hs_ref = oracle.quant_group128(h)
    assert np.array_equal(u8_bits(r.hq[:S]), hq_ref)
    assert np.array_equal(r.hs[:S].cpu().numpy().view(np.uint32), hs_ref.view(np.uint32))

    # 4) D: N-split W2 with routed weights on the GPU's hq, hs
    d_ref, d_bnd = oracle.grouped_gemm(hq_ref, hs_ref, c.w2_q, c.w2_s, srt, eids, nt, BM, S, 1,
                                       topk_w=c.topk_w, with_bound=True)
    D = bf16_bits(r.D[:S])
    bad = oracle.gemm_close(D, d_ref, d_bnd)
    assert not bad.any(), f"D: {int(bad.sum())} of {bad.size} outside the bound"

    # 5) y: top-k sum of the GPU's D, bit-exact
    assert np.array_equal(bf16_bits(y), oracle.moe_reduce(D, T, k))

    # 6) the layer through the gates against the golden
    x32 = oracle.bf16_to_f32(c.x)
    w1 = dequant_weights_f32(c.w13_q, c.w13_s)
    w2 = dequant_weights_f32(c.w2_q, c.w2_s)
    golden = oracle.golden_moe(x32, c.topk_ids, c.topk_w, w1, w2)
    rep = oracle.compare_outputs(oracle.bf16_to_f32(bf16_bits(y)), golden, atol=0.2, rtol=0.0,
                                 **oracle.DEFAULT_GATES)
    assert rep["pass"], rep
    atol = oracle.calibrated_atol(x32, c.topk_ids, c.topk_w, w1, w2)
    assert rep["max_abs"] <= atol, (rep, atol)


def test_split_runner_run_allocates_nothing():
    from td_benchmark_amd import ops

    c = make_case(150, 512, 384, 6, 3, 32, seed=5)
    g = to_gpu(c)
    r = ops.SplitExpertsRunner(g["w13"], g["w13_s"], g["w2"], g["w2_s"], c.T, c.k, 4, 4, c.BM)
    r.run(g["x"], g["topk_w"], g["topk_ids"])
    torch.cuda.synchronize()
    before = torch.cuda.memory_stats()["allocation.all.allocated"]
    for _ in range(3):
        r.run(g["x"], g["topk_w"], g["topk_ids"])
    torch.cuda.synchronize()
    assert torch.cuda.memory_stats()["allocation.all.allocated"] == before


def test_split_runner_adds_the_shared_expert():
    """With a shared expert the layer output is bf16(bf16(top-k sum) +
    shared(x)), the shared expert fed the layer's own FP8 input
    (overlap_forward.py:238-245, 315-320)."""
    from td_benchmark_amd import ops

    print("case: split runner with shared expert", flush=True)
    c = make_case(150, 512, 384, 6, 3, 32, seed=9)
    g = to_gpu(c)
    rng = np.random.default_rng(19)
    s1q, s1s = oracle.quant_block128((rng.standard_normal((1, 256, c.H)) * 0.02).astype(np.float32))
    s2q, s2s = oracle.quant_block128((rng.standard_normal((1, c.H, 128)) * 0.02).astype(np.float32))
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    shared = ops.SharedExpertRunner(dev(s1q).view(ops.FP8), dev(s1s), dev(s2q).view(ops.FP8), dev(s2s), c.T)
    r = ops.SplitExpertsRunner(g["w13"], g["w13_s"], g["w2"], g["w2_s"], c.T, c.k, 2, 3, c.BM, shared=shared)
    y = bf16_bits(r.run(g["x"], g["topk_w"], g["topk_ids"]))
    torch.cuda.synchronize()
    D = bf16_bits(r.D[: c.S])
    sh = bf16_bits(r.shared_out)
    sh_alone = bf16_bits(shared(g["x"]))
    torch.cuda.synchronize()
    assert np.array_equal(sh, sh_alone)
    ref = oracle.f32_to_bf16(oracle.bf16_to_f32(oracle.moe_reduce(D, c.T, c.k)) + oracle.bf16_to_f32(sh))
    assert np.array_equal(y, ref)
