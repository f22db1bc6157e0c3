"""EXP-012 counterpart: workgroup -> tile order versus expert locality in the
FP8 grouped GEMM (reference microbench/mb_tile_order_groupgemm.py:13; orders
of REWORK-C.md:524-533: expert-sorted, shuffled arrival, half-phase
interleave).  The W13 GEMM of the reference's UND shape (H=2048,
2I=1536, E=128, top-8, uniform routing) at M tokens; outputs are identical
for every order, only the schedule changes.

l2_hit_rate comes from hardware counters: with ``--l2-counters`` every case is
also run once more in a child process under ``rocprofv3 --pmc TCC_HIT_sum
TCC_MISS_sum`` (restricted to the grouped GEMM kernel) and the row carries
sum(TCC_HIT) / (sum(TCC_HIT) + sum(TCC_MISS)) over that child's GEMM
dispatches; without it (or when rocprofv3 is absent) the field is null."""
from __future__ import annotations

import csv
import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parents[2]))

from td_benchmark_amd.microbench.common import fp8_weights, routed_ids, run_microbench, time_gpu  # noqa: E402

SWEEP = {"order": ["expert_major", "phase_major", "half_phase"], "M": [2048, 4096, 6647]}
# "phase_major" is the reference sweep's name for arrival (shuffled) order
ORDER_CODE = {"expert_major": 0, "phase_major": 1, "shuffled": 1, "half_phase": 2}
SHAPE = dict(H=2048, I=768, E=128, top_k=8)


def case_fn(case, args):
    import torch

    from td_benchmark_amd import ops

    H, I, E, k = (SHAPE[x] for x in ("H", "I", "E", "top_k"))
    M = case["M"]
    w13, w13s, _, _ = fp8_weights(E, H, I)
    ids, _ = routed_ids(M, E, k, "uniform")
    dev = torch.device("cuda", 0)
    x = torch.randn((M, H), generator=torch.Generator(device=dev).manual_seed(7), device=dev).to(torch.bfloat16)
    q, s = ops.per_token_group_quant_fp8(x)
    bm = ops.get_moe_config(M, E, k)["BLOCK_SIZE_M"]
    sorted_ids, eids, ntpp = ops.moe_align_block_size(ids.view(-1), bm, E)
    C = torch.empty((M * k, 2 * I), dtype=torch.bfloat16, device=dev)
    order = ORDER_CODE[case["order"]]

    def call():
        ops.dispatch_fused_moe_kernel(q, w13, C, s, w13s, None, None, sorted_ids, eids, ntpp, False, k,
                                      {"BLOCK_SIZE_M": bm}, tile_order=order)

    samples = time_gpu(call, args.warmup, args.repeat)
    lat = sorted(samples)[len(samples) // 2]
    return samples, {"tflops": 2.0 * M * k * 2 * I * H / (lat / 1e3) / 1e12, "l2_hit_rate": None,
                     "block_size_m": bm, "tile_order_code": order, "shape": SHAPE}


def l2_hit_rate_from_csv(paths, kernel_substr: str = "grouped_gemm_kernel"):
    """sum(TCC_HIT) / (sum(TCC_HIT) + sum(TCC_MISS)) over the dispatches of
    kernels whose name contains ``kernel_substr`` in rocprofv3 counter CSVs
    (one row per dispatch and counter); None if there are none."""
    hit = miss = 0.0
    for path in paths:
        with open(path, newline="", encoding="utf-8") as fh:
            for row in csv.DictReader(fh):
                if kernel_substr not in row["Kernel_Name"]:
                    continue
                name = row["Counter_Name"]
                if name.startswith("TCC_HIT"):
                    hit += float(row["Counter_Value"])
                elif name.startswith("TCC_MISS"):
                    miss += float(row["Counter_Value"])
    return hit / (hit + miss) if hit + miss > 0 else None


def measure_l2_hit_rate(case, timeout_s: int = 180):
    """Runs this script on one case in a child process under rocprofv3 with
    the TCC hit/miss counters and returns the GEMM's L2 hit rate (None when
    rocprofv3 is not installed)."""
    exe = shutil.which("rocprofv3") or ("/opt/rocm/bin/rocprofv3" if os.path.exists("/opt/rocm/bin/rocprofv3") else None)
    if exe is None:
        return None
    with tempfile.TemporaryDirectory(dir=os.environ.get("TMPDIR")) as tmp:
        cmd = ["timeout", "-s", "KILL", str(timeout_s), exe, "--pmc", "TCC_HIT_sum", "TCC_MISS_sum",
               "--kernel-include-regex", "grouped_gemm_kernel", "-d", tmp, "-o", "l2", "--output-format", "csv",
               "--", sys.executable, str(Path(__file__).resolve()), "--one-case", f"{case['order']}:{case['M']}",
               "--warmup", "1", "--repeat", "3", "--output", os.path.join(tmp, "rows.jsonl")]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"rocprofv3 child failed ({proc.returncode}): {proc.stderr[-2000:]}")
        return l2_hit_rate_from_csv(sorted(Path(tmp).rglob("*counter_collection.csv")))


def main(argv=None) -> int:
    import argparse

    pre = argparse.ArgumentParser(add_help=False)
    pre.add_argument("--l2-counters", action="store_true")
    pre.add_argument("--one-case", default=None, help="order:M -- run only this case (the counter child)")
    opts, rest = pre.parse_known_args(argv)
    sweep = SWEEP
    fn = case_fn
    if opts.one_case:
        order, m = opts.one_case.split(":")
        sweep = {"order": [order], "M": [int(m)]}
    elif opts.l2_counters:
        def fn(case, args):
            samples, extra = case_fn(case, args)
            extra["l2_hit_rate"] = measure_l2_hit_rate(case)
            return samples, extra
    return run_microbench(__file__, "EXP-012", "tile order and expert locality effects on FP8 GroupGEMM", sweep,
                          ["latency_ms", "tflops", "l2_hit_rate"],
                          "runs the ordered FP8 grouped GEMM (HIP) on the local MI355X", fn, rest)


if __name__ == "__main__":
    raise SystemExit(main())
