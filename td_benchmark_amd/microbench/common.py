"""Shared driver of the microbench counterparts.

Contract of the reference's microbench harness (microbench/common.py:12-91,
tests/test_microbench_dry_run.py:7-30): ``--dry-run`` prints one JSON plan
with keys kind, script, exp_id, purpose, sweep, metrics, warmup, repeat,
output, result_schema{kind, metric, unit, aggregation}, recommended_command,
server_verify, server_verify_detail; otherwise every case of the sweep's
cartesian product (up to ``--max-cases``) is measured and written as one JSONL
row {kind, script, exp_id, case_index, case, status, warmup, repeat,
samples_ms, metrics{latency_ms, ...}}.  Unlike the reference's placeholder
probe, each case here runs this library's HIP kernels on the local GPU and
times them with HIP events on the launch stream; ``status`` is "MEASURED",
or "UNSUPPORTED" with a reason for a case outside what the kernels implement.
"""
from __future__ import annotations

import argparse
import json
import statistics
from itertools import islice, product
from pathlib import Path
from typing import Any, Callable

RESULT_SCHEMA = {
    "kind": "microbench",
    "metric": "name of the measured quantity, for example latency_ms or bandwidth_gbps",
    "unit": "unit associated with metric",
    "aggregation": "median over repeat samples (HIP events on the launch stream)",
}
PEAK_HBM_GBS = 8000.0
PEAK_FP8_TFLOPS = 5000.0


class UnsupportedCase(Exception):
    """The case asks for something the kernels do not implement."""


def iter_cases(sweep: dict[str, list[Any]], max_cases: int):
    keys = list(sweep)
    combos = (dict(zip(keys, vals)) for vals in product(*(sweep[k] for k in keys)))
    return islice(combos, max_cases) if max_cases > 0 else combos


def time_gpu(fn: Callable[[], Any], warmup: int, repeat: int) -> list[float]:
    """Per-call milliseconds of `fn` (which only enqueues GPU work)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(repeat)]
    for a, b in ev:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in ev]


def run_microbench(script: str, exp_id: str, purpose: str, sweep: dict[str, list[Any]],
                   metrics: list[str], detail: str,
                   case_fn: Callable[[dict[str, Any], argparse.Namespace], tuple[list[float], dict[str, Any]]],
                   argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=purpose)
    ap.add_argument("--dry-run", action="store_true")
    ap.add_argument("--output", default=f"results/microbench_{Path(script).stem[3:]}.jsonl")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--repeat", type=int, default=50)
    ap.add_argument("--max-cases", type=int, default=0)
    args = ap.parse_args(argv)
    name = Path(script).name
    module = f"td_benchmark_amd.microbench.{Path(script).stem}"
    plan = {
        "kind": "microbench",
        "script": name,
        "exp_id": exp_id,
        "purpose": purpose,
        "sweep": sweep,
        "metrics": metrics,
        "warmup": args.warmup,
        "repeat": args.repeat,
        "output": args.output,
        "result_schema": RESULT_SCHEMA,
        "recommended_command": ["torchrun", "--nproc_per_node=1", "--module", module, "--output", args.output,
                                "--warmup", str(args.warmup), "--repeat", str(args.repeat)],
        "server_verify": True,
        "server_verify_detail": detail,
    }
    if args.dry_run:
        print(json.dumps(plan, sort_keys=True))
        return 0
    out = Path(args.output)
    out.parent.mkdir(parents=True, exist_ok=True)
    n = 0
    with out.open("w", encoding="utf-8") as fh:
        for index, case in enumerate(iter_cases(sweep, args.max_cases)):
            print(f"{name} case {index}: {json.dumps(case, sort_keys=True)}", flush=True)
            row = {"kind": "microbench", "script": name, "exp_id": exp_id, "case_index": index, "case": case,
                   "warmup": args.warmup, "repeat": args.repeat}
            try:
                samples, extra = case_fn(case, args)
                row.update(status="MEASURED", samples_ms=samples,
                           metrics={"latency_ms": statistics.median(samples), **extra})
            except UnsupportedCase as exc:
                row.update(status="UNSUPPORTED", detail=str(exc), samples_ms=[], metrics={})
            fh.write(json.dumps(row, sort_keys=True) + "\n")
            n += 1
    print(json.dumps({"output": str(out), "rows": n}, sort_keys=True))
    return 0


def routed_ids(M: int, E: int, top_k: int, distribution: str, seed: int = 42):
    """Token -> expert draws on the GPU: top_k distinct experts per token from
    a uniform, Zipf(1.2) or hotspot (4 experts carry 60 % of the mass) law,
    with softmax(N(0,1)) weights -- the distributions of the reference's
    GroupGEMM sweep (REWORK-B.md:818-836)."""
    import torch

    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(seed)
    if distribution == "uniform":
        probs = torch.ones(E, device=dev)
    elif distribution == "zipf":
        probs = torch.arange(1, E + 1, device=dev, dtype=torch.float32).pow(-1.2)
    elif distribution == "hotspot":
        probs = torch.ones(E, device=dev)
        probs[:4] = 1.5 * (E - 4) / 4
    else:
        raise UnsupportedCase(f"distribution {distribution!r}")
    probs = probs / probs.sum()
    ids = torch.multinomial(probs.expand(M, E).contiguous(), top_k, replacement=False, generator=gen)
    w = torch.softmax(torch.randn(M, top_k, generator=gen, device=dev), dim=-1)
    return ids.to(torch.int32).contiguous(), w.float().contiguous()


_WEIGHTS: dict[tuple, tuple] = {}


def fp8_weights(E: int, H: int, I: int, seed: int = 42):
    """Block-quantised random W13 [E, 2I, H] and W2 [E, H, I] (N(0, 0.02)),
    cached per shape; quantised by this library's own 128x128 kernel."""
    import torch

    from td_benchmark_amd import ops

    key = (E, H, I)
    if key not in _WEIGHTS:
        dev = torch.device("cuda", 0)
        gen = torch.Generator(device=dev).manual_seed(seed)
        out = []
        for shape in ((E, 2 * I, H), (E, H, I)):
            q = torch.empty(shape, dtype=ops.FP8, device=dev)
            s = torch.empty((E, (shape[1] + 127) // 128, (shape[2] + 127) // 128), dtype=torch.float32, device=dev)
            for e0 in range(0, E, 8):
                e1 = min(E, e0 + 8)
                w = torch.randn((e1 - e0, *shape[1:]), generator=gen, device=dev) * 0.02
                ops.quantize_block128(w, q[e0:e1], s[e0:e1])
                del w
            out += [q, s]
        _WEIGHTS.clear()
        _WEIGHTS[key] = tuple(out)
    return _WEIGHTS[key]
