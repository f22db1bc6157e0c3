"""EXP-010 counterpart: cost of moe_align_block_size (sort + pad by expert)
versus tokens M, experts E and top_k (reference microbench/mb_moe_align.py:11;
the reference times torch argsort/bincount/cumsum, REWORK-B.md:622-697).
Here the whole align (three kernels) runs per call on uniform random ids."""
from __future__ import annotations

import sys
from pathlib import Path

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parents[2]))

from td_benchmark_amd.microbench.common import run_microbench, time_gpu  # noqa: E402

SWEEP = {"M": [1024, 2048, 4096, 6647], "E": [64, 128], "top_k": [8, 16]}


def case_fn(case, args):
    import torch

    from td_benchmark_amd import ops

    M, E, k = case["M"], case["E"], case["top_k"]
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(42)
    ids = torch.randint(0, E, (M * k,), generator=gen, device=dev, dtype=torch.int32)
    bm = ops.get_moe_config(M, E, k)["BLOCK_SIZE_M"]
    bufs = ops.AlignBuffers(M * k, E, bm, dev)
    samples = time_gpu(lambda: bufs.run(ids), args.warmup, args.repeat)
    ntpp = int(bufs.ntpp.item())
    lat = sorted(samples)[len(samples) // 2]
    return samples, {"pad_overhead_ratio": (ntpp - M * k) / (M * k), "effective_tokens_per_s": M / (lat / 1e3),
                     "block_size_m": bm, "num_tokens_post_padded": ntpp}


def main(argv=None) -> int:
    return run_microbench(__file__, "EXP-010", "dispatch pre-sort, align, and pad cost", SWEEP,
                          ["latency_ms", "pad_overhead_ratio", "effective_tokens_per_s"],
                          "runs moe_align_block_size (HIP) on the local MI355X", case_fn, argv)


if __name__ == "__main__":
    raise SystemExit(main())
