"""EXP-012 counterpart: workgroup -> tile order versus expert locality in the
FP8 grouped GEMM (reference microbench/mb_tile_order_groupgemm.py:13; orders
of REWORK-C.md:524-533: expert-sorted, shuffled arrival, half-phase
interleave).  The W13 GEMM of the reference's UND shape (H=2048,
2I=1536, E=128, top-8, uniform routing) at M tokens; outputs are identical
for every order, only the schedule changes.  l2_hit_rate needs hardware
counters: collect TCC_HIT_sum / TCC_MISS_sum with rocprofv3 --pmc around this
script; the row carries null."""
from __future__ import annotations

import sys
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


def main(argv=None) -> int:
    return run_microbench(__file__, "EXP-012", "tile order and expert locality effects on FP8 GroupGEMM", SWEEP,
                          ["latency_ms", "tflops", "l2_hit_rate"],
                          "runs the ordered FP8 grouped GEMM (HIP) on the local MI355X", case_fn, argv)


if __name__ == "__main__":
    raise SystemExit(main())
