"""EXP-011 counterpart: cost of the preprocessing ahead of the expert GEMMs
(reference microbench/mb_dispatch_prep.py:11, REWORK-B.md:701-793).  On this
path the preparation is the 1x128 quant of the tokens plus moe_align (no host
readback: num_tokens_post_padded stays on the device and the GEMM reads it);
percent_of_e2e relates it to the whole layer (H=4096, I=768, uniform routing)."""
from __future__ import annotations

import sys
from pathlib import Path

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parents[2]))

from td_benchmark_amd.microbench.common import fp8_weights, routed_ids, run_microbench, time_gpu  # noqa: E402

SWEEP = {"M": [1024, 2048, 4096, 6647], "E": [64, 128], "top_k": [8, 16]}
SHAPE = dict(H=4096, I=768)


def case_fn(case, args):
    import torch

    from td_benchmark_amd import ops

    M, E, k = case["M"], case["E"], case["top_k"]
    H, I = SHAPE["H"], SHAPE["I"]
    w13, w13s, w2, w2s = fp8_weights(E, H, I)
    ids, w = routed_ids(M, E, k, "uniform")
    dev = torch.device("cuda", 0)
    x = torch.randn((M, H), generator=torch.Generator(device=dev).manual_seed(7), device=dev).to(torch.bfloat16)
    runner = ops.FusedExpertsRunner(w13, w13s, w2, w2s, M, k)
    idv, wv = ids.view(-1), w.view(-1)

    def prep():
        runner.stage_quant(x)
        runner.stage_align(idv)

    samples = time_gpu(prep, args.warmup, args.repeat)
    e2e = time_gpu(lambda: runner.run(x, wv, idv), max(1, args.warmup // 4), max(3, args.repeat // 4))
    lat = sorted(samples)[len(samples) // 2]
    e2e_ms = sorted(e2e)[len(e2e) // 2]
    return samples, {"percent_of_e2e": 100.0 * lat / e2e_ms, "tokens_per_s": M / (lat / 1e3), "e2e_ms": e2e_ms,
                     "host_sync_ms": 0.0, "block_size_m": runner.BM, "shape": SHAPE}


def main(argv=None) -> int:
    return run_microbench(__file__, "EXP-011", "dispatch preprocessing (quant + align) cost", SWEEP,
                          ["latency_ms", "percent_of_e2e", "tokens_per_s"],
                          "runs quant + moe_align (HIP) and the layer on the local MI355X", case_fn, argv)


if __name__ == "__main__":
    raise SystemExit(main())
