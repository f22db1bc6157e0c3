"""EXP-015 counterpart: bandwidth of the 1x128 FP8 quant kernels (reference
microbench/mb_quant_kernels.py:11).  group128: x [M, K] bf16 -> codes +
scales; swiglu_group128: c [M, 2K] bf16 (gate | up) -> quant of
bf16(silu(gate)*up) [M, K].  Bytes moved per call are the algorithmic ones:
group128 3MK + 4MK/128, swiglu_group128 5MK + 4MK/128."""
from __future__ import annotations

import sys
from pathlib import Path

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parents[2]))

from td_benchmark_amd.microbench.common import PEAK_HBM_GBS, run_microbench, time_gpu  # noqa: E402

SWEEP = {"kernel": ["group128", "swiglu_group128"], "M": [1024, 4096, 6647], "K": [2048, 3200, 4096]}


def case_fn(case, args):
    import torch

    from td_benchmark_amd import ops

    M, K, kern = case["M"], case["K"], case["kernel"]
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(42)
    q = torch.empty((M, K), dtype=ops.FP8, device=dev)
    s = torch.empty((M, K // 128), dtype=torch.float32, device=dev)
    if kern == "group128":
        x = torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16)
        fn = lambda: ops.per_token_group_quant_fp8(x, out_q=q, out_s=s)  # noqa: E731
        nbytes = 3 * M * K + 4 * M * K / 128
    else:
        x = torch.randn((M, 2 * K), generator=gen, device=dev).to(torch.bfloat16)
        fn = lambda: ops.silu_mul_quant_group128(x, out_q=q, out_s=s)  # noqa: E731
        nbytes = 5 * M * K + 4 * M * K / 128
    samples = time_gpu(fn, args.warmup, args.repeat)
    lat = sorted(samples)[len(samples) // 2]
    gbps = nbytes / (lat / 1e3) / 1e9
    return samples, {"bandwidth_gbps": gbps, "bandwidth_utilization": gbps / PEAK_HBM_GBS, "bytes": nbytes}


def main(argv=None) -> int:
    return run_microbench(__file__, "EXP-015", "group128 token quantization and SwiGLU+group128 kernel bandwidth",
                          SWEEP, ["latency_ms", "bandwidth_gbps", "bandwidth_utilization"],
                          "runs the group128 quant kernels (HIP) on the local MI355X", case_fn, argv)


if __name__ == "__main__":
    raise SystemExit(main())
