"""EXP-016 counterpart, one-GPU half: chunk count versus the cost of the
b-group pipelines' compute stream (reference microbench/mb_chunk_overlap.py:
sweep {"n_chunks": [1, 2, 4, 8, 16], "scheme": ["b1", "b2", "b3"]}; real design
REWORK-B.md:905-1011, eta = (T_a1 - T_b) / T_comm at M in {1024, 5120}, K = 4096).

The b schemes split W13 over K chunks (each chunk's all-gathered hidden slice
quantised and accumulated into a bf16 C13) and W2 over N chunks (each chunk
reduce-scattered), overlap/overlap_forward.py:252-321.  On one GPU there is
no all-gather or reduce-scatter, so the communication estimate, eta and the
exposed communication are not measurable here and the rows carry null for
them.  What one GPU does measure is the compute stream those schemes run:
ops.SplitExpertsRunner with n_chunks K chunks and n_chunks N chunks
(latency_ms), against the single-pass layer ops.FusedExpertsRunner (the a1
baseline, a1_latency_ms); chunk_overhead_ms is their difference, the cost of
chunking that any communication overlap must pay back.  The three b schemes
differ only in the dtype of their communication legs (b1 bf16 AG + bf16 RS,
b2 FP8 AG, b3 FP8 AG + FP8 RS), so their compute streams are the same; the
scheme is kept in the case for the row format.  Shape: the reference's v1
preset (moe_bench/config.py:16-24, configs/run_v1.yaml) at one rank, so the
full expert set: K = H = 4096, E = 64, top-8, n_gateup = 2I = 6144, n_down =
I = 3072, uniform routing; the routed experts only, on both sides."""
from __future__ import annotations

import sys
from pathlib import Path

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parents[2]))

from td_benchmark_amd.microbench.common import (UnsupportedCase, fp8_weights, routed_ids,  # noqa: E402
                                                run_microbench, time_gpu)

SWEEP = {"M": [1024, 5120], "scheme": ["b1", "b2", "b3"], "n_chunks": [1, 2, 4, 8, 16]}
SHAPE = dict(H=4096, E=64, top_k=8, I=3072)
_A1: dict[int, float] = {}


def case_fn(case, args):
    import torch

    from td_benchmark_amd import ops

    if case["scheme"] not in ("b1", "b2", "b3"):
        raise UnsupportedCase(f"scheme {case['scheme']!r}")
    M, n = case["M"], case["n_chunks"]
    H, E, k, I = (SHAPE[x] for x in ("H", "E", "top_k", "I"))
    if n > H // 128:
        raise UnsupportedCase(f"{n} chunks of whole 128-column blocks do not fit H = {H}")
    w13, w13s, w2, w2s = fp8_weights(E, H, I)
    ids, w = routed_ids(M, E, k, "uniform")
    dev = torch.device("cuda", 0)
    x = torch.randn((M, H), generator=torch.Generator(device=dev).manual_seed(7), device=dev).to(torch.bfloat16)
    bm = ops.get_moe_config(M, E, k)["BLOCK_SIZE_M"]
    idv, wv = ids.view(-1), w.view(-1)
    if M not in _A1:
        one = ops.FusedExpertsRunner(w13, w13s, w2, w2s, M, k, bm)
        a1 = time_gpu(lambda: one.run(x, wv, idv), args.warmup, args.repeat)
        _A1[M] = sorted(a1)[len(a1) // 2]
        del one
    split = ops.SplitExpertsRunner(w13, w13s, w2, w2s, M, k, n, n, bm)
    samples = time_gpu(lambda: split.run(x, wv, idv), args.warmup, args.repeat)
    lat = sorted(samples)[len(samples) // 2]
    return samples, {"a1_latency_ms": _A1[M], "chunk_overhead_ms": lat - _A1[M],
                     "overlap_efficiency_eta": None, "exposed_comm_ms": None, "comm_est_ms": None,
                     "chunks_gateup": [list(b) for b in split.k_bounds],
                     "chunks_down": [list(b) for b in split.n_bounds], "block_size_m": bm,
                     "shape": dict(SHAPE, M=M)}


def main(argv=None) -> int:
    return run_microbench(__file__, "EXP-016", "b-group chunk count versus overlap efficiency eta", SWEEP,
                          ["latency_ms", "overlap_efficiency_eta", "exposed_comm_ms"],
                          "runs the b-scheme compute stream (K-split W13, N-split W2; HIP) on the local MI355X; "
                          "the communication legs need more than one GPU", case_fn, argv)


if __name__ == "__main__":
    raise SystemExit(main())
