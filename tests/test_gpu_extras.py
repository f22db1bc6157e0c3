"""GPU parity of the pieces around the core chain: the one-pass SiLU*up +
1x128 quant, the reduce with the shared expert's addend, the GEMM's tile
orders, the shared expert, the chunked multi-stream runner, the m1 scheme
plugin and the microbench drivers.  All calls go through the C ABI."""
from __future__ import annotations

import json
from types import SimpleNamespace

import numpy as np
import pytest

import oracle
from moe_cases import bf16_bits, dequant_weights_f32, e4m3_ulp_diff, make_case, to_gpu, u8_bits

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


@pytest.mark.parametrize("R,I,seed", [(7, 128, 0), (300, 768, 1), (64, 2048, 2)])
def test_silu_mul_quant_equals_two_pass_and_oracle(R, I, seed):
    torch = _torch()
    from td_benchmark_amd import ops

    print(f"case: silu_mul_quant R={R} I={I}", flush=True)
    rng = np.random.default_rng(seed)
    c = oracle.f32_to_bf16((rng.standard_normal((R, 2 * I)) * 3).astype(np.float32))
    ct = torch.from_numpy(c.view(np.int16)).cuda().view(torch.bfloat16)
    q1, s1 = ops.silu_mul_quant_group128(ct)
    h = torch.empty((R, I), dtype=torch.bfloat16, device="cuda")
    ops.silu_and_mul(h, ct)
    q2, s2 = ops.per_token_group_quant_fp8(h)
    torch.cuda.synchronize()
    assert np.array_equal(u8_bits(q1), u8_bits(q2))
    assert np.array_equal(s1.cpu().numpy(), s2.cpu().numpy())
    # against the oracle chain (silu may differ by one bf16 ulp on rare inputs)
    qo, so = oracle.quant_group128(oracle.silu_and_mul(c))
    ulp = e4m3_ulp_diff(u8_bits(q1), qo)
    assert ulp.max() <= 1 and np.mean(ulp > 0) <= 1e-3


def test_reduce_with_addend_matches_oracle():
    torch = _torch()
    from td_benchmark_amd import ops

    print("case: reduce_topk_add", flush=True)
    rng = np.random.default_rng(3)
    T, k, H = 37, 8, 1024
    D = oracle.f32_to_bf16(rng.standard_normal((T * k, H)).astype(np.float32))
    A = oracle.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    Dt = torch.from_numpy(D.view(np.int16)).cuda().view(torch.bfloat16)
    At = torch.from_numpy(A.view(np.int16)).cuda().view(torch.bfloat16)
    y = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    ops.moe_sum(Dt, y, k, addend=At)
    torch.cuda.synchronize()
    ref = oracle.f32_to_bf16(oracle.bf16_to_f32(oracle.moe_reduce(D, T, k)) + oracle.bf16_to_f32(A))
    assert np.array_equal(bf16_bits(y), ref)


@pytest.mark.parametrize("order", [1, 2])
def test_tile_orders_give_identical_results(order):
    torch = _torch()
    from td_benchmark_amd import ops

    print(f"case: tile order {order}", flush=True)
    c = make_case(T=200, H=512, I=384, E=16, k=4, BM=32, seed=5)
    g = to_gpu(c)
    q, s = ops.per_token_group_quant_fp8(g["x"])
    sorted_ids, eids, ntpp = ops.moe_align_block_size(g["topk_ids"].view(-1), c.BM, c.E)
    outs = []
    for o in (0, order):
        C = torch.zeros((c.S, 2 * c.I), dtype=torch.bfloat16, device="cuda")
        ops.dispatch_fused_moe_kernel(q, g["w13"], C, s, g["w13_s"], None, None, sorted_ids, eids, ntpp, False,
                                      c.k, {"BLOCK_SIZE_M": c.BM}, tile_order=o)
        outs.append(bf16_bits(C))
    torch.cuda.synchronize()
    assert np.array_equal(outs[0], outs[1])


def _shared_case(seed=8):
    c = make_case(T=96, H=256, I=256, E=4, k=2, BM=16, seed=seed)
    rng = np.random.default_rng(seed + 100)
    sw1 = (rng.standard_normal((1, 2 * 128, c.H)) * 0.02).astype(np.float32)
    sw2 = (rng.standard_normal((1, c.H, 128)) * 0.02).astype(np.float32)
    return c, oracle.quant_block128(sw1), oracle.quant_block128(sw2)


def test_shared_expert_runner_matches_oracle_chain():
    torch = _torch()
    from td_benchmark_amd import ops

    print("case: shared expert runner", flush=True)
    c, (s1q, s1s), (s2q, s2s) = _shared_case()
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    shared = ops.SharedExpertRunner(dev(s1q).view(ops.FP8), dev(s1s), dev(s2q).view(ops.FP8), dev(s2s), c.T)
    x = torch.from_numpy(c.x.view(np.int16)).cuda().view(torch.bfloat16)
    out_bf16 = bf16_bits(shared(x))
    q, s = ops.per_token_group_quant_fp8(x)
    out_fp8 = bf16_bits(shared(q, s))          # FP8 passthrough gives the same result
    torch.cuda.synchronize()
    assert np.array_equal(out_bf16, out_fp8)
    st = oracle.moe_layer_stages(c.x, np.zeros((c.T, 1), np.int32), np.ones((c.T, 1), np.float32),
                                 s1q, s1s, s2q, s2s, 16)
    # (the oracle chain's routed weight 1.0 equals no routed weight.)  The
    # GPU's h may flip an FP8 code against the oracle's, so compare through
    # the layer tolerance rather than the per-GEMM bound.
    rep = oracle.compare_outputs(oracle.bf16_to_f32(out_bf16), oracle.bf16_to_f32(st["y"]), atol=0.0, rtol=0.0)
    assert rep["max_abs_rel"] <= 2e-2 and rep["cos_sim"] > 0.999, rep


def test_layer_with_shared_expert_meets_golden_gates():
    torch = _torch()
    from td_benchmark_amd import ops

    print("case: layer + shared expert", flush=True)
    c, (s1q, s1s), (s2q, s2s) = _shared_case(9)
    g = to_gpu(c)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    shared = ops.SharedExpertRunner(dev(s1q).view(ops.FP8), dev(s1s), dev(s2q).view(ops.FP8), dev(s2s), c.T)
    runner = ops.FusedExpertsRunner(g["w13"], g["w13_s"], g["w2"], g["w2_s"], c.T, c.k, c.BM, shared=shared)
    y = runner.run(g["x"], g["topk_w"].view(-1), g["topk_ids"].view(-1))
    torch.cuda.synchronize()
    x = oracle.bf16_to_f32(c.x)
    w1, w2 = dequant_weights_f32(c.w13_q, c.w13_s), dequant_weights_f32(c.w2_q, c.w2_s)
    sw1, sw2 = dequant_weights_f32(s1q, s1s), dequant_weights_f32(s2q, s2s)
    golden = oracle.golden_moe(x, c.topk_ids, c.topk_w, w1, w2, sw1, sw2)
    rep = oracle.compare_outputs(oracle.bf16_to_f32(bf16_bits(y)), golden, atol=0.0, rtol=0.0,
                                 **oracle.DEFAULT_GATES)
    assert rep["pass"], rep
    # and the routed part alone is unchanged by the shared expert's presence
    plain = ops.FusedExpertsRunner(g["w13"], g["w13_s"], g["w2"], g["w2_s"], c.T, c.k, c.BM)
    y0 = plain.run(g["x"], g["topk_w"].view(-1), g["topk_ids"].view(-1))
    s_out = shared(runner.q1, runner.s1)
    y_ref = torch.empty_like(y0)
    ops.moe_sum(runner.D[: c.S], y_ref, c.k, addend=s_out)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(y), bf16_bits(y_ref))


# (T, E, k, BM): 32-row tiles per chunk; and chunks whose experts average
# >= 160 slots (S_chunk >= 160 E), so every chunk runs 256-row tiles over
# 64-row blocks with the activation scales by sorted position
CHUNK_SETUPS = {"short": (301, 8, 4, 32), "tall": (1600, 4, 2, 64)}


@pytest.mark.parametrize("setup", sorted(CHUNK_SETUPS))
@pytest.mark.parametrize("n_chunks,n_streams", [(4, 2), (3, 1), (2, 2)])
def test_chunked_runner_equals_single_pass(n_chunks, n_streams, setup):
    torch = _torch()
    from td_benchmark_amd import ops

    T, E, k, BM = CHUNK_SETUPS[setup]
    print(f"case: chunked runner {n_chunks}x{n_streams} {setup} T={T} E={E} k={k} BM={BM}", flush=True)
    c = make_case(T=T, H=256, I=256, E=E, k=k, BM=BM, seed=11)
    g = to_gpu(c)
    one = ops.FusedExpertsRunner(g["w13"], g["w13_s"], g["w2"], g["w2_s"], c.T, c.k, BM)
    y1 = bf16_bits(one.run(g["x"], g["topk_w"].view(-1), g["topk_ids"].view(-1)))
    ch = ops.ChunkedExpertsRunner(g["w13"], g["w13_s"], g["w2"], g["w2_s"], c.T, c.k, n_chunks, n_streams, BM)
    if setup == "tall" and n_chunks <= 4:
        assert all(ops.gemm_tile_rows(r.BM, r.S, r.E) == 256 and r.scales_by_position for r in ch.runners)
    for _ in range(2):
        y2 = ch.run(g["x"], g["topk_w"], g["topk_ids"])
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(y2), y1)


def _bundle(c, g, shared=None):
    torch = _torch()
    ckpt = SimpleNamespace(w1=SimpleNamespace(fp8=g["w13"], scale=g["w13_s"]),
                           w2=SimpleNamespace(fp8=g["w2"], scale=g["w2_s"]), shared_w1=None, shared_w2=None)
    if shared is not None:
        (s1q, s1s), (s2q, s2s) = shared
        dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
        ckpt.shared_w1 = SimpleNamespace(fp8=dev(s1q).view(torch.float8_e4m3fn), scale=dev(s1s))
        ckpt.shared_w2 = SimpleNamespace(fp8=dev(s2q).view(torch.float8_e4m3fn), scale=dev(s2s))
    routing = SimpleNamespace(topk_ids_full=g["topk_ids"], topk_weights_full=g["topk_w"],
                              topk_ids_local=g["topk_ids"], topk_weights_local=g["topk_w"])
    return SimpleNamespace(hidden_local=g["x"], ckpt=ckpt, routing=routing)


@pytest.mark.parametrize("tunables", [{}, {"n_chunks": 3, "n_streams": 2}, {"block_m": 64},
                                      {"n_chunks_gateup": 2, "n_chunks_down": 4}])
def test_scheme_m1_run_meets_golden_gates(tunables):
    torch = _torch()
    from td_benchmark_amd import schemes

    print(f"case: scheme m1 {tunables}", flush=True)
    c, s1, s2 = _shared_case(12)
    g = to_gpu(c)
    ctx = SimpleNamespace(rank=0, world_size=1, device=torch.device("cuda", 0))
    inst = schemes.build_scheme(None, ctx, _bundle(c, g, (s1, s2)), SimpleNamespace(code="m1", tunables=tunables))
    y = inst.run()
    torch.cuda.synchronize()
    assert tuple(y.shape) == (c.T, c.H) and y.dtype == torch.bfloat16
    x = oracle.bf16_to_f32(c.x)
    golden = oracle.golden_moe(x, c.topk_ids, c.topk_w, dequant_weights_f32(c.w13_q, c.w13_s),
                               dequant_weights_f32(c.w2_q, c.w2_s), dequant_weights_f32(*s1),
                               dequant_weights_f32(*s2))
    rep = oracle.compare_outputs(oracle.bf16_to_f32(bf16_bits(y)), golden, atol=0.0, rtol=0.0,
                                 **oracle.DEFAULT_GATES)
    assert rep["pass"], rep
    staged = inst.run_staged()
    assert np.array_equal(bf16_bits(staged.output), bf16_bits(y))
    if not tunables.get("n_chunks") and not tunables.get("n_chunks_gateup"):
        assert set(staged.stage_ms) == {"quant", "align", "scales", "w13", "w2", "shared", "reduce"}
    assert inst.diagnostics["scheme"] == "m1" and inst.diagnostics["shared_expert"] is True
    inst.close()
    with pytest.raises(RuntimeError, match="closed"):
        inst.run()


@pytest.mark.parametrize("tunables", [{}, {"n_chunks": 3, "n_streams": 2}, {"n_chunks_gateup": 2, "n_chunks_down": 4}])
def test_scheme_run_allocates_nothing(tunables):
    """The builder allocates every buffer; run() only launches kernels
    (schemes/base.py:45-93; the reference's own lesson on allocation inside the
    timed call, docs/exp/EXP-024-cgroup-perf-rootcause.md:6-9).  With a shared
    expert whose runner was built for a larger row count than a chunk holds,
    run() still allocates nothing: the align outputs for the chunk's rows are
    prepared at build time."""
    torch = _torch()
    from td_benchmark_amd import schemes

    print(f"case: scheme m1 allocation-free run {tunables}", flush=True)
    c, s1, s2 = _shared_case(12)
    g = to_gpu(c)
    ctx = SimpleNamespace(rank=0, world_size=1, device=torch.device("cuda", 0))
    inst = schemes.build_scheme(None, ctx, _bundle(c, g, (s1, s2)), SimpleNamespace(code="m1", tunables=tunables))
    inst.run()  # lazy instances build on the first call
    torch.cuda.synchronize()
    before = torch.cuda.memory_stats()["allocation.all.allocated"]
    for _ in range(3):
        inst.run()
    torch.cuda.synchronize()
    after = torch.cuda.memory_stats()["allocation.all.allocated"]
    assert after == before, f"run() allocated {after - before} blocks"
    inst.close()


def test_shared_expert_rejects_unprepared_row_counts():
    torch = _torch()
    from td_benchmark_amd import ops

    print("case: shared expert row counts", flush=True)
    c, s1, s2 = _shared_case(12)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    sh = ops.SharedExpertRunner(dev(s1[0]).view(ops.FP8), dev(s1[1]), dev(s2[0]).view(ops.FP8), dev(s2[1]), c.T,
                                row_counts=(c.T // 2,))
    x = to_gpu(c)["x"]
    y_half = sh(x[: c.T // 2].contiguous()).clone()
    y_full = sh(x)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(y_half), bf16_bits(y_full[: c.T // 2]))
    with pytest.raises(ValueError, match="no align outputs prepared"):
        sh(x[: c.T // 3].contiguous())
    with pytest.raises(ValueError, match="exceed max_tokens"):
        sh.prepare(c.T + 1)


@pytest.mark.parametrize("name", ["mb_moe_align", "mb_quant_kernels", "mb_group_gemm",
                                  "mb_tile_order_groupgemm", "mb_dispatch_prep", "mb_chunk_overlap"])
def test_microbench_writes_measured_rows(name, tmp_path):
    import importlib

    print(f"case: microbench {name}", flush=True)
    mod = importlib.import_module(f"td_benchmark_amd.microbench.{name}")
    out = tmp_path / "mb.jsonl"
    assert mod.main(["--output", str(out), "--warmup", "1", "--repeat", "2", "--max-cases", "2"]) == 0
    rows = [json.loads(line) for line in out.read_text().splitlines()]
    assert len(rows) == 2
    for r in rows:
        assert r["kind"] == "microbench" and r["script"] == f"{name}.py"
        assert r["status"] == "MEASURED"
        assert len(r["samples_ms"]) == 2
        assert r["metrics"]["latency_ms"] > 0


def test_layer_graph_replays_equal_eager_runs():
    torch = _torch()
    from td_benchmark_amd import ops

    print("case: layer graph replay", flush=True)
    c = make_case(T=120, H=256, I=256, E=8, k=2, BM=32, seed=44)
    c2 = make_case(T=120, H=256, I=256, E=8, k=2, BM=32, seed=45)
    g, g2 = to_gpu(c), to_gpu(c2)
    eager = ops.FusedExpertsRunner(g["w13"], g["w13_s"], g["w2"], g["w2_s"], c.T, c.k, 32)
    y_ref = bf16_bits(eager.run(g["x"], g["topk_w"].view(-1), g["topk_ids"].view(-1)))
    y_ref2 = bf16_bits(eager.run(g2["x"], g2["topk_w"].view(-1), g2["topk_ids"].view(-1)))
    runner = ops.FusedExpertsRunner(g["w13"], g["w13_s"], g["w2"], g["w2_s"], c.T, c.k, 32)
    x, w, ids = g["x"].clone(), g["topk_w"].view(-1).clone(), g["topk_ids"].view(-1).clone()
    graph = runner.capture(x, w, ids)
    for i in range(3):
        # unrelated eager work and a host synchronisation between replays
        junk = torch.randn(512, 512, device="cuda") @ torch.randn(512, 512, device="cuda")
        torch.cuda.synchronize()
        y = graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(y), y_ref), f"replay {i}"
        del junk
    # new inputs through the captured tensors
    x.copy_(g2["x"])
    w.copy_(g2["topk_w"].view(-1))
    ids.copy_(g2["topk_ids"].view(-1))
    y = graph.replay()
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(y), y_ref2)
