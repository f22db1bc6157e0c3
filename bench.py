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
``layer_us_stats`` gives avg/min/med/p95/std over the per-step samples
(moe_bench/timing.py:23-34).  ``cpu_baseline`` times the reference's torch CPU
golden path (restated in oracle/golden_torch.py, all host cores) on a bounded
sample of the same workload.  ``shared_expert`` times the shared expert (one
E=1, top-1 expert of the same hidden and intermediate size) on the layer's own
FP8 input, outside the layer time.  ``power`` gives socket power, graphics
clock and energy per call of the layer, W13 and W2, each run back to back
for a few seconds (amd-smi; null where it is unavailable).  ``exact_dot``
times the layer with W13 in its opt-in exact-dot mode (the FP8 codes on the
bf16 matrix core); the headline numbers are the FP8 form.
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
PEAK_BF16_TFLOPS = 2500.0    # MI355X dense bf16 MFMA
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


def summarize_samples(samples_ms: list[float]) -> dict[str, float]:
    """avg/min/med/p95/std of per-step samples, the statistics of the
    reference's timing harness (moe_bench/timing.py:23-34)."""
    import statistics
    if not samples_ms:
        return {"avg": 0.0, "min": 0.0, "med": 0.0, "p95": 0.0, "std": 0.0, "n": 0}
    ordered = sorted(samples_ms)
    return {"avg": statistics.mean(samples_ms), "min": ordered[0], "med": statistics.median(samples_ms),
            "p95": ordered[min(len(ordered) - 1, int(0.95 * (len(ordered) - 1)))],
            "std": statistics.pstdev(samples_ms) if len(samples_ms) > 1 else 0.0, "n": len(samples_ms)}


def cpu_model_name() -> str:
    """The host CPU's model name as lscpu reports it, with its CPU family /
    model / stepping numbers (a virtualised host may report only a generic
    name); /proc/cpuinfo if lscpu is unavailable."""
    import subprocess
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        fields = {}
        for line in out.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                fields.setdefault(k.strip(), v.strip())
        if "Model name" in fields:
            ids = [f"{k.lower()} {fields[k]}" for k in ("CPU family", "Model", "Stepping") if fields.get(k)]
            return fields["Model name"] + (f" ({', '.join(ids)})" if ids else "")
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def shared_expert_leg(runner, wl, steps: int, warmup: int) -> dict:
    """The shared expert beside the routed layer: one expert (E = 1, top-1)
    of the layer's hidden size with intermediate size I (the reference's
    shared_intermediate default, config.py ShapeCfg), weights N(0, H^-0.5) and
    N(0, I^-0.5) block-quantised 128x128 (data/checkpoint.py:64-66), run on
    the layer's own FP8 input with its build-time align
    (schemes/shared_expert.py:81-148).  Each call is the fused W13 (SiLU*up +
    1x128 quant) and the W2 GEMM; the two are timed together with HIP events
    around every call."""
    import torch

    from td_benchmark_amd import ops, workloads

    T, H, I = wl.T, wl.H, wl.I
    gen = torch.Generator(device="cuda").manual_seed(wl.seed + 1)
    w1 = torch.randn((1, 2 * I, H), generator=gen, device="cuda") * H ** -0.5
    w2 = torch.randn((1, H, I), generator=gen, device="cuda") * I ** -0.5
    w1q, w1s = ops.quantize_block128(w1)
    w2q, w2s = ops.quantize_block128(w2)
    del w1, w2
    sh = ops.SharedExpertRunner(w1q, w1s, w2q, w2s, max_tokens=T)
    for _ in range(warmup):
        sh(runner.q1, runner.s1)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in ev:
        a.record()
        sh(runner.q1, runner.s1)
        b.record()
    torch.cuda.synchronize()
    stats = summarize_samples([a.elapsed_time(b) * 1e3 for a, b in ev])
    one = workloads.Workload("shared", T, H, I, 1, 1, sh.BM, "softmax")
    ntpp = int(sh._align_for(T).ntpp.item())
    by = stage_bytes(one, ntpp, 1, sh.BM)
    flop = 6.0 * T * H * I
    sec = stats["avg"] / 1e6
    bytes_ = by["w13"] + by["w2"]
    return {"us": stats["avg"], "us_stats": stats, "T": T, "H": H, "I": I, "block_size_m": sh.BM,
            "gemm_tile_m": ops.gemm_tile_rows(sh.BM, T, 1), "flop": flop, "bytes": bytes_,
            "TFLOP/s": flop / sec / 1e12, "mfma_frac": flop / sec / 1e12 / PEAK_FP8_TFLOPS,
            "GB/s": bytes_ / sec / 1e9, "hbm_frac": bytes_ / sec / 1e9 / PEAK_HBM_GBS,
            "bound": "mfma" if flop / (PEAK_FP8_TFLOPS * 1e12) >= bytes_ / (PEAK_HBM_GBS * 1e9) else "hbm",
            "input": "the routed layer's FP8 activations and 1x128 scales (no second quant)"}


def exact_dot_leg(runner, step, steps: int, warmup: int, flop_w13: float, power_seconds: float = 0.0) -> dict:
    """The layer with the W13 stage in exact-dot mode (every 128-element dot
    as four bf16 MFMAs on the codes converted exactly to bf16): W13 and
    layer time per call, timed with events like the headline layer, and,
    with ``power_seconds``, the exact W13's socket power and clock as in the
    power leg.  The headline numbers are the FP8 form; this is the cost of
    the opt-in mode."""
    import torch
    runner.exact_dot = True
    try:
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        for a, b in ev:
            a.record()
            runner.stage_w13()
            b.record()
        lev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        for a, b in lev:
            a.record()
            step()
            b.record()
        torch.cuda.synchronize()
        power = power_leg(runner.stage_w13, power_seconds) if power_seconds > 0 else None
    finally:
        runner.exact_dot = False
    step()  # leave the runner's buffers as the FP8 form writes them
    torch.cuda.synchronize()
    w13 = summarize_samples([a.elapsed_time(b) * 1e3 for a, b in ev])
    tflops = flop_w13 / (w13["avg"] / 1e6) / 1e12
    return {"w13_us_stats": w13, "layer_us_stats": summarize_samples([a.elapsed_time(b) * 1e3 for a, b in lev]),
            "w13_TFLOP/s": tflops, "w13_bf16_mfma_frac": tflops / PEAK_BF16_TFLOPS, "w13_power": power,
            "form": "FP8 codes converted to bf16, four v_mfma_f32_16x16x32_bf16 per 128-element dot"}


def _amd_smi_sample() -> tuple[float, float] | None:
    """(socket power W, mean graphics clock MHz over the XCDs) of GPU 0 from
    `amd-smi metric -p -c --json -g 0`; None when amd-smi is unavailable."""
    import subprocess
    try:
        out = subprocess.run(["amd-smi", "metric", "-p", "-c", "--json", "-g", "0"], capture_output=True,
                             text=True, timeout=10).stdout
        doc, _ = json.JSONDecoder().raw_decode(out[out.index("{"):])
        gpu = doc["gpu_data"][0] if "gpu_data" in doc else doc
        power = float(gpu["power"]["socket_power"]["value"])
        clks = [float(v["clk"]["value"]) for k, v in gpu["clock"].items()
                if k.startswith("gfx_") and isinstance(v, dict) and isinstance(v.get("clk"), dict)]
        return power, sum(clks) / len(clks)
    except (OSError, ValueError, KeyError, TypeError, IndexError, ZeroDivisionError,
            subprocess.SubprocessError):
        return None


def power_leg(fn, seconds: float) -> dict | None:
    """Runs ``fn`` back to back for about ``seconds`` while a thread samples
    socket power and the graphics clock with amd-smi; returns the averages of
    the samples taken after the first half second, the calls' mean time and
    the energy per call (power x time).  None without amd-smi."""
    import threading
    import torch
    if _amd_smi_sample() is None:
        return None
    samples, stop = [], threading.Event()

    def sampler():
        t0 = time.perf_counter()
        while not stop.is_set():
            smp = _amd_smi_sample()
            if smp is not None and time.perf_counter() - t0 > 0.5:
                samples.append(smp)
            stop.wait(0.2)

    fn()
    torch.cuda.synchronize()
    th = threading.Thread(target=sampler, daemon=True)
    th.start()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_end = time.perf_counter() + seconds
    calls = 0
    start.record()
    while time.perf_counter() < t_end:
        for _ in range(20):
            fn()
        calls += 20
        torch.cuda.synchronize()
    end.record()
    torch.cuda.synchronize()
    stop.set()
    th.join()
    if not samples:
        return None
    us = start.elapsed_time(end) * 1e3 / calls
    power = sum(p for p, _ in samples) / len(samples)
    return {"us_per_call": us, "socket_power_W": power, "gfx_clock_MHz": sum(c for _, c in samples) / len(samples),
            "energy_J_per_call": power * us * 1e-6, "samples": len(samples), "calls": calls}


def _time_cpu(fn, warmup: int, repeat: int) -> dict:
    """bench_cpu semantics (moe_bench/timing.py:37-45): warmup calls, then
    ``repeat`` timed calls with time.perf_counter."""
    for _ in range(warmup):
        fn()
    samples = []
    for _ in range(repeat):
        t0 = time.perf_counter()
        fn()
        samples.append((time.perf_counter() - t0) * 1e3)
    return summarize_samples(samples)


def cpu_stage_times(data, wl, D_sample, block_m: int) -> dict:
    """The layer's quant, align and reduce stages as the reference's torch CPU
    ops (oracle/golden_torch.py), warmup 1 and repeat 3: quant over all T
    tokens, align over all S slots, reduce over the first D_sample rows'
    tokens (extrapolated to T)."""
    import torch

    from oracle.golden_torch import align_torch, quant_group128_torch, reduce_torch

    x = data.x.cpu()
    ids = data.topk_ids.cpu()
    tr = D_sample.shape[0] // wl.top_k
    D = D_sample[: tr * wl.top_k]
    q = _time_cpu(lambda: quant_group128_torch(x), 1, 3)
    a = _time_cpu(lambda: align_torch(ids, wl.E, block_m), 1, 3)
    r = _time_cpu(lambda: reduce_torch(D, tr, wl.top_k), 1, 3)
    return {"quant_us": q["med"] * 1e3, "align_us": a["med"] * 1e3,
            "reduce_us": r["med"] * 1e3 * wl.T / max(tr, 1),
            "threads": torch.get_num_threads(),
            "sample": (f"torch CPU ops, median of 3 after 1 warmup: quant {wl.T}x{wl.H}, align {wl.S} slots, "
                       f"reduce {tr} of {wl.T} tokens (scaled to T)")}


def cpu_baseline(data, wl, budget_s: float) -> dict:
    """The reference's torch CPU golden path (moe_bench/verify.py:14-47,
    restated in oracle/golden_torch.py) with torch.set_num_threads(os.cpu_count()):
    weights dequantised one expert at a time outside the timed calls, one
    expert's fp32 chain warmed up, then whole experts timed until ``budget_s``
    of compute has run.  Reports its GEMM TFLOP/s and the layer time
    extrapolated to every slot."""
    import torch

    from oracle.golden_torch import dequant_expert_torch, golden_moe_torch

    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    ids = data.topk_ids.cpu()
    wts = data.topk_w.cpu()
    x = data.x.float().cpu()
    counts = torch.bincount(ids.view(-1).long(), minlength=wl.E)
    order = [int(e) for e in torch.randperm(wl.E, generator=torch.Generator().manual_seed(0)) if counts[e] > 0]

    def weights(e):
        w1 = dequant_expert_torch(data.w13[e].cpu(), data.w13_s[e].cpu())
        w2 = dequant_expert_torch(data.w2[e].cpu(), data.w2_s[e].cpu())
        return w1, w2

    out = torch.zeros((wl.T, wl.H), dtype=torch.float32)
    w1, w2 = weights(order[0])
    golden_moe_torch(x, ids, wts, lambda _e: w1, lambda _e: w2, experts=[order[0]], out=out)  # warmup
    t_total, slots, done = 0.0, 0, 0
    for e in order:
        w1, w2 = weights(e)
        t0 = time.perf_counter()
        golden_moe_torch(x, ids, wts, lambda _e: w1, lambda _e: w2, experts=[e], out=out)
        t_total += time.perf_counter() - t0
        slots += int(counts[e])
        done += 1
        if t_total >= budget_s:
            break
    flop = 6.0 * slots * wl.H * wl.I
    return {
        "value": flop / t_total / 1e12,
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"torch CPU restatement of verify.py:14-47 (oracle/golden_torch.py), "
                   f"torch.set_num_threads({cores}), on {done} of {len(order)} active experts "
                   f"({slots} of {wl.S} slots), {t_total:.1f} s after one warmup expert"),
        "layer_us_extrapolated": t_total / max(slots, 1) * wl.S * 1e6,
        "cpu_model": cpu_model_name(),
        "host_cpus": cores,
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
    ap.add_argument("--no-shared", action="store_true",
                    help="skip the shared-expert leg (one E=1, top-1 expert on the layer's FP8 input)")
    ap.add_argument("--no-exact", action="store_true",
                    help="skip the exact-dot leg (the layer with W13 in its exact-dot mode)")
    ap.add_argument("--power-seconds", type=float, default=2.0,
                    help="seconds of back-to-back layer, W13 and W2 runs sampled for socket power and clock "
                         "(0 to skip)")
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
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # The layer as a caller runs it: K steps, one event pair around each for the
    # per-step samples and nothing between its launches.
    sev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    start.record()
    for i in range(args.steps):
        sev[i][0].record()
        step()
        sev[i][1].record()
    end.record()
    torch.cuda.synchronize()
    ms_per_step = start.elapsed_time(end) / args.steps
    ms_single = ms_per_step
    single_stats = summarize_samples([a.elapsed_time(b) * 1e3 for a, b in sev])
    # Per-stage times from K more steps with an event between every two
    # launches (on launch-bound layers those records add host time, which is
    # why the layer time above is taken without them).
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(len(STAGES) + 1)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    for i in range(args.steps):
        step(events[i])
    torch.cuda.synchronize()
    stage_ms = {name: sum(ev[j].elapsed_time(ev[j + 1]) for ev in events) / args.steps
                for j, name in enumerate(STAGES)}
    stage_stats = {name: summarize_samples([ev[j].elapsed_time(ev[j + 1]) * 1e3 for ev in events])
                   for j, name in enumerate(STAGES) if name in ("w13", "w2")}
    step_stats = single_stats
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
        pev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(args.steps)]
        start.record()
        for i in range(args.steps):
            pev[i][0].record()
            pipe.run(data.x, data.topk_w, data.topk_ids)
            pev[i][1].record()
        end.record()
        torch.cuda.synchronize()
        ms_per_step = start.elapsed_time(end) / args.steps
        step_stats = summarize_samples([a.elapsed_time(b) * 1e3 for a, b in pev])
    # Config 5 also in the reference pipeline's own compute-stream structure
    # (W13 K-split into a bf16 C13, SiLU*up, quant, W2 N-split; no comm legs),
    # reported beside the token-chunk pipeline and the single pass.
    kn_stats = None
    if pipe is not None:
        split = ops.SplitExpertsRunner(data.w13, data.w13_s, data.w2, data.w2_s, wl.T, wl.top_k, wl.n_chunks,
                                       wl.n_chunks, bm)
        for _ in range(args.warmup):
            split.run(data.x, data.topk_w, data.topk_ids)
        torch.cuda.synchronize()
        kev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(args.steps)]
        for i in range(args.steps):
            kev[i][0].record()
            split.run(data.x, data.topk_w, data.topk_ids)
            kev[i][1].record()
        torch.cuda.synchronize()
        kn_stats = summarize_samples([a.elapsed_time(b) * 1e3 for a, b in kev])
        del split
        torch.cuda.empty_cache()

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
        "layer_us_stats": step_stats,
        "layer_us_single_pass": ms_single * 1e3,
        "layer_us_single_pass_stats": single_stats,
        "gemm_us_stats": stage_stats,
        "layer_us_graph": None if ms_graph is None else ms_graph * 1e3,
        "layer_us_kn_split_stats": kn_stats,
        "gemm_tflops": wl.gemm_flop / (gemm_ms / 1e3) / 1e12,
        "gemm_mfma_frac": wl.gemm_flop / (gemm_ms / 1e3) / 1e12 / PEAK_FP8_TFLOPS,
        "stages": stages,
        "ntpp": ntpp,
        "active_experts": active,
        "roofline": roof,
    }
    if args.power_seconds > 0 and pipe is None:
        result["power"] = {"layer": power_leg(lambda: step(), args.power_seconds),
                           "w13": power_leg(runner.stage_w13, args.power_seconds),
                           "w2": power_leg(lambda: runner.stage_w2(data.topk_w), args.power_seconds),
                           "source": "amd-smi metric -p -c (socket power, mean gfx clock of the XCDs), "
                                     "sampled every ~0.2 s while the stage runs back to back"}
    if not args.no_shared:
        result["shared_expert"] = shared_expert_leg(runner, wl, args.steps, args.warmup)
    if not args.no_exact:
        result["exact_dot"] = exact_dot_leg(runner, step, args.steps, args.warmup, flop_w13,
                                            args.power_seconds if pipe is None else 0.0)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(data, wl, args.cpu_budget)
        n_rows = min(wl.T, 1024) * wl.top_k
        D_sample = runner.D[:n_rows].cpu()
        result["cpu_baseline"]["stages"] = cpu_stage_times(data, wl, D_sample, bm)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
