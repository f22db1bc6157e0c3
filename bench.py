#!/usr/bin/env python
"""Benchmark of the MI355X FP8 MoE expert path on one GPU.

A step is one pass of the whole rank-local MoE layer (1x128 quant -> align ->
W13 grouped GEMM with fused SiLU*up + quant -> W2 grouped GEMM with routed
weights -> top-k reduce) over one synthetic batch already resident in HBM.
Default workload: the DeepSeek-V3 expert layer (T=8192, H=7168, I=2048,
E=256, top-8, block_size_m=128), the shape the headline metric is quoted on.

Prints ONE JSON line.  ``value`` = algorithmic grouped-GEMM FLOP (6*S*H*I) per
second over the whole timed layer (quant/align/reduce included); per-stage
times come from HIP events recorded on the launch stream inside the timed
region.  ``roofline`` describes the dominant kernel (the W13 GEMM).
``cpu_baseline`` times the CPU restatement of the reference's torch golden
(oracle.golden_moe) on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "FP8 grouped-GEMM TFLOP/s (% MFMA peak) + MoE layer µs, DeepSeek-V3 shape, 1 GPU"
PEAK_FP8_TFLOPS = 5000.0     # MI355X dense FP8 MFMA
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E
STAGES = ("quant", "align", "scales", "w13", "w2", "reduce")


def stage_bytes(wl, ntpp: int, active: int, BM: int | None = None) -> dict[str, float]:
    """Algorithmic HBM bytes per launch of each stage (padding excluded)."""
    T, H, I, E, k = wl.T, wl.H, wl.I, wl.E, wl.top_k
    BM = BM or wl.block_m
    S = T * k
    w13 = active * (2 * I * H + 4 * (2 * I // 128) * (H // 128))
    w2 = active * (H * I + 4 * (H // 128) * (I // 128))
    return {
        "quant": 2 * T * H + T * H + 4 * T * H / 128,
        "align": 4 * S + 4 * ntpp + 4 * ntpp / BM + 4,
        # activation scales by sorted position: ids read, one scale row read and written per slot
        "scales": 4 * ntpp + 8 * S * H / 128,
        "w13": w13 + T * H + 4 * T * H / 128 + S * I + 4 * S * I / 128,
        "w2": w2 + S * I + 4 * S * I / 128 + 2 * S * H + 4 * S,
        "reduce": 2 * S * H + 2 * T * H,
    }


def measured_traffic(workload: str, kernel: str) -> tuple[float | None, str | None]:
    """HBM bytes per launch of ``kernel`` on ``workload`` as recorded by the
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes (scaled by the copy calibration)
    in profiles/*_hbm_traffic.md; (None, None) if no summary holds it."""
    pat = re.compile(r"traffic_bytes\[(\w+),\s*([^\]]+)\]\s*=\s*([0-9.eE+]+)")
    for path in sorted((ROOT / "profiles").glob("*_hbm_traffic.md")):
        for m in pat.finditer(path.read_text()):
            if m.group(1) == workload and m.group(2).replace(" ", "") == kernel.replace(" ", ""):
                return float(m.group(3)), path.name
    return None, None


def cpu_stage_times(data, wl, D_sample, block_m: int) -> dict:
    """The layer's quant, align and reduce stages on the host, single-threaded
    C restatements from the oracle: quant over all T tokens, align over all S
    slots, reduce over the first D_sample.shape[0] // k tokens' rows of the
    GPU's D (extrapolated to T)."""
    import numpy as np

    import oracle

    oracle.lib()  # load the library outside the timed calls
    out = {}
    x = data.x.view(__import__("torch").int16).cpu().numpy().view(np.uint16)
    ids = data.topk_ids.cpu().numpy()
    t0 = time.perf_counter()
    oracle.quant_group128(x)
    out["quant_us"] = (time.perf_counter() - t0) * 1e6
    t0 = time.perf_counter()
    oracle.moe_align(ids, wl.E, block_m)
    out["align_us"] = (time.perf_counter() - t0) * 1e6
    tr = D_sample.shape[0] // wl.top_k
    t0 = time.perf_counter()
    oracle.moe_reduce(D_sample[: tr * wl.top_k], tr, wl.top_k)
    out["reduce_us"] = (time.perf_counter() - t0) * 1e6 * wl.T / max(tr, 1)
    out["sample"] = (f"quant {wl.T}x{wl.H}, align {wl.S} slots, reduce {tr} of {wl.T} tokens "
                     "(scaled to T); one thread each")
    return out


def cpu_baseline(data, wl, budget_s: float) -> dict:
    """Time oracle.golden_moe (the reference's fp32 per-expert torch CPU path,
    restated in numpy) on whole experts of this workload until ``budget_s`` of
    compute has run; report its GEMM TFLOP/s and the extrapolated layer time."""
    import numpy as np

    import oracle

    try:
        from threadpoolctl import threadpool_info
        threads = max([int(i.get("num_threads", 1)) for i in threadpool_info()
                       if i.get("user_api") == "blas"] or [1])
    except Exception:
        threads = 1
    ids = data.topk_ids.cpu().numpy()
    wts = data.topk_w.cpu().numpy()
    x = data.x.float().cpu().numpy()
    counts = np.bincount(ids.ravel(), minlength=wl.E)
    order = np.random.default_rng(0).permutation(wl.E)
    t_total, slots, done = 0.0, 0, 0
    for e in order:
        if counts[e] == 0:
            continue
        w1 = oracle.bf16_to_f32(oracle.dequant_block128(
            data.w13[e:e + 1].contiguous().view(__import__("torch").uint8).cpu().numpy(),
            data.w13_s[e:e + 1].cpu().numpy()))[0]
        w2 = oracle.bf16_to_f32(oracle.dequant_block128(
            data.w2[e:e + 1].contiguous().view(__import__("torch").uint8).cpu().numpy(),
            data.w2_s[e:e + 1].cpu().numpy()))[0]
        t0 = time.perf_counter()
        oracle.golden_moe(x, ids, wts, lambda _e: w1, lambda _e: w2, experts=[e])
        t_total += time.perf_counter() - t0
        slots += int(counts[e])
        done += 1
        if t_total >= budget_s:
            break
    flop = 6.0 * slots * wl.H * wl.I
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": flop / t_total / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle.golden_moe (fp32 numpy/BLAS restatement of verify.py:14-47) on {done} of "
                   f"{int((counts > 0).sum())} active experts ({slots} of {wl.S} slots), {t_total:.1f} s"),
        "layer_us_extrapolated": t_total / max(slots, 1) * wl.S * 1e6,
        "cpu_model": model,
        "host_cpus": os.cpu_count(),
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="dsv3")
    ap.add_argument("--block-m", type=int, default=0, help="override the workload's block_size_m")
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU baseline compute")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the multi-GPU expert/tensor-parallel "
              "legs are out of scope); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    from td_benchmark_amd import ops, workloads

    wl = workloads.CONFIGS[args.workload]
    data = workloads.generate(wl, "cuda")
    bm = args.block_m or wl.block_m
    runner = ops.FusedExpertsRunner(data.w13, data.w13_s, data.w2, data.w2_s, wl.T, wl.top_k, bm)
    # Config 5 (n_chunks > 1): the headline time is the chunked pipeline over
    # n_streams HIP streams; per-stage times come from the single-pass runner.
    pipe = (ops.ChunkedExpertsRunner(data.w13, data.w13_s, data.w2, data.w2_s, wl.T, wl.top_k, wl.n_chunks,
                                     wl.n_streams, bm) if wl.n_chunks > 1 else None)

    def step(ev=None):
        if ev is not None:
            ev[0].record()
        runner.stage_quant(data.x)
        if ev is not None:
            ev[1].record()
        runner.stage_align(data.topk_ids)
        if ev is not None:
            ev[2].record()
        runner.stage_scales()
        if ev is not None:
            ev[3].record()
        runner.stage_w13()
        if ev is not None:
            ev[4].record()
        runner.stage_w2(data.topk_w)
        if ev is not None:
            ev[5].record()
        runner.stage_reduce()
        if ev is not None:
            ev[6].record()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(len(STAGES) + 1)] for _ in range(args.steps)]
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(args.steps):
        step(events[i])
    end.record()
    torch.cuda.synchronize()
    ms_per_step = start.elapsed_time(end) / args.steps
    ms_single = ms_per_step
    stage_ms = {name: sum(ev[j].elapsed_time(ev[j + 1]) for ev in events) / args.steps
                for j, name in enumerate(STAGES)}
    # The same layer replayed from a captured HIP graph (one launch per step);
    # shows the launch overhead that matters for the small configurations.
    ms_graph = None
    if pipe is None:
        graph = runner.capture(data.x, data.topk_w, data.topk_ids)
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
        start.record()
        for _ in range(args.steps):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        ms_graph = start.elapsed_time(end) / args.steps
    if pipe is not None:
        for _ in range(args.warmup):
            pipe.run(data.x, data.topk_w, data.topk_ids)
        torch.cuda.synchronize()
        start.record()
        for _ in range(args.steps):
            pipe.run(data.x, data.topk_w, data.topk_ids)
        end.record()
        torch.cuda.synchronize()
        ms_per_step = start.elapsed_time(end) / args.steps

    ntpp = int(runner.align.ntpp.item())
    counts = torch.bincount(data.topk_ids.view(-1).long(), minlength=wl.E)
    active = int((counts > 0).sum().item())
    sbytes = stage_bytes(wl, ntpp, active, bm)
    flop_w13 = 4.0 * wl.S * wl.H * wl.I
    flop_w2 = 2.0 * wl.S * wl.H * wl.I
    gemm_ms = stage_ms["w13"] + stage_ms["w2"]
    stages = {}
    for name in STAGES:
        sec = stage_ms[name] / 1e3
        row = {"us": stage_ms[name] * 1e3, "GB/s": sbytes[name] / sec / 1e9,
               "hbm_frac": sbytes[name] / sec / 1e9 / PEAK_HBM_GBS, "bytes": sbytes[name]}
        if name in ("w13", "w2"):
            fl = flop_w13 if name == "w13" else flop_w2
            row["TFLOP/s"] = fl / sec / 1e12
            row["mfma_frac"] = fl / sec / 1e12 / PEAK_FP8_TFLOPS
        stages[name] = row
    w13_sec = stage_ms["w13"] / 1e3
    w13_tflops = flop_w13 / w13_sec / 1e12
    w13_gbs = sbytes["w13"] / w13_sec / 1e9
    # The kernel's floor is the larger of its MFMA time and its HBM time.
    if sbytes["w13"] / (PEAK_HBM_GBS * 1e9) >= flop_w13 / (PEAK_FP8_TFLOPS * 1e12):
        roof = {"bound": "hbm", "achieved": w13_gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": w13_gbs / PEAK_HBM_GBS}
    else:
        roof = {"bound": "mfma", "achieved": w13_tflops, "peak": PEAK_FP8_TFLOPS, "unit": "TFLOP/s",
                "frac": w13_tflops / PEAK_FP8_TFLOPS}
    tm = ops.gemm_tile_rows(bm, wl.S, wl.E)
    traffic, traffic_src = measured_traffic(wl.name, f"grouped_gemm_kernel<{tm},true>")
    roof.update({"traffic": traffic, "traffic_source": traffic_src,
                 "kernel": f"grouped_gemm_kernel<{tm},true> (W13 + SiLU*up + 1x128 quant)",
                 "alg_bytes": sbytes["w13"], "alg_flop": flop_w13, "avg_us": stage_ms["w13"] * 1e3,
                 "mfma_frac": w13_tflops / PEAK_FP8_TFLOPS, "hbm_frac": w13_gbs / PEAK_HBM_GBS})
    result = {
        "metric": METRIC,
        "value": wl.gemm_flop / (ms_per_step / 1e3) / 1e12,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3fn (fp32 accumulate)",
        "data": "synthetic (N(0,1) activations, N(0,0.02) weights block-quantised 128x128, "
                f"{wl.routing} top-{wl.top_k} routing)",
        "config": {"workload": wl.name, "T": wl.T, "H": wl.H, "I": wl.I, "E": wl.E,
                   "top_k": wl.top_k, "block_size_m": bm, "gemm_tile_m": tm, "routing": wl.routing,
                   "n_chunks": wl.n_chunks, "n_streams": wl.n_streams,
                   "parallelism": "single GPU, all experts local"},
        "layer_us": ms_per_step * 1e3,
        "layer_us_single_pass": ms_single * 1e3,
        "layer_us_graph": None if ms_graph is None else ms_graph * 1e3,
        "gemm_tflops": wl.gemm_flop / (gemm_ms / 1e3) / 1e12,
        "gemm_mfma_frac": wl.gemm_flop / (gemm_ms / 1e3) / 1e12 / PEAK_FP8_TFLOPS,
        "stages": stages,
        "ntpp": ntpp,
        "active_experts": active,
        "roofline": roof,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(data, wl, args.cpu_budget)
        n_rows = min(wl.T, 1024) * wl.top_k
        D_sample = runner.D[:n_rows].view(torch.int16).cpu().numpy().view("uint16")
        result["cpu_baseline"]["stages"] = cpu_stage_times(data, wl, D_sample, bm)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
