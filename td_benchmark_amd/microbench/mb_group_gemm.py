"""EXP-014 counterpart: FP8 grouped-GEMM efficiency versus the token ->
expert distribution (reference microbench/mb_group_gemm.py:11; shape of its
real design REWORK-B.md:795-903: H=4096, E=64, top-8, I=768, at the token
counts of its recorded results, M in {1024, 5120},
docs/exp/EXP-014-group-gemm-dist.md:11-19).  One call is the whole
fused_experts layer at block_size_m = tile;
tflops counts the algorithmic 6*S*H*I of both GEMMs; tile_utilization is
valid rows / padded rows (S / num_tokens_post_padded)."""
from __future__ import annotations

import sys
from pathlib import Path

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parents[2]))

from td_benchmark_amd.microbench.common import (UnsupportedCase, fp8_weights, routed_ids,  # noqa: E402
                                                run_microbench, time_gpu)

SWEEP = {"dtype": ["fp8"], "M": [1024, 5120], "distribution": ["uniform", "zipf", "hotspot"], "tile": [64, 128, 256]}
SHAPE = dict(H=4096, E=64, top_k=8, I=768)


def case_fn(case, args):
    import torch

    from td_benchmark_amd import ops

    if case["dtype"] != "fp8":
        raise UnsupportedCase("only fp8 weights are implemented")
    if case["tile"] not in ops.SUPPORTED_BLOCK_M:
        raise UnsupportedCase(f"block_size_m {case['tile']} not implemented (supported {ops.SUPPORTED_BLOCK_M})")
    M = case["M"]
    H, E, k, I = (SHAPE[x] for x in ("H", "E", "top_k", "I"))
    w13, w13s, w2, w2s = fp8_weights(E, H, I)
    ids, w = routed_ids(M, E, k, case["distribution"])
    dev = torch.device("cuda", 0)
    x = torch.randn((M, H), generator=torch.Generator(device=dev).manual_seed(7), device=dev).to(torch.bfloat16)
    runner = ops.FusedExpertsRunner(w13, w13s, w2, w2s, M, k, case["tile"])
    idv, wv = ids.view(-1), w.view(-1)
    samples = time_gpu(lambda: runner.run(x, wv, idv), args.warmup, args.repeat)
    lat = sorted(samples)[len(samples) // 2]
    ntpp = int(runner.align.ntpp.item())
    counts = torch.bincount(idv.long(), minlength=E).float()
    return samples, {"tflops": 6.0 * M * k * H * I / (lat / 1e3) / 1e12, "tile_utilization": M * k / ntpp,
                     "imbalance_max_over_mean": float(counts.max() / counts.mean()), "shape": dict(SHAPE, M=M)}


def main(argv=None) -> int:
    return run_microbench(__file__, "EXP-014", "FP8 GroupGEMM efficiency versus token distribution", SWEEP,
                          ["latency_ms", "tflops", "tile_utilization"],
                          "runs the FP8 grouped-GEMM layer (HIP) on the local MI355X", case_fn, argv)


if __name__ == "__main__":
    raise SystemExit(main())
