"""Writes the committed golden fixture tests/golden/tiny_seed0.npz.

Inputs: a tiny MoE layer (T=32, H=256, I=128, E=4, top-2, block_size_m=16,
softmax routing, seed 0; activations N(0,1) rounded to bf16, weights
N(0, 0.02) quantised 128x128).  Expected outputs: every intermediate of the
stage chain computed by the CPU oracle with the reference's rounding points
(quant codes/scales, align outputs, C13, h, intermediate codes/scales, D, y),
the fp32 golden of verify.py:14-47, the calibrated absolute tolerance of
tests/calibrate_tolerance.py, and the oracle's L1 magnitudes and matrix-core
bounds for the two GEMMs (the GPU parity tests' accumulation bound).

The reference itself cannot be imported here (it needs vLLM and a GPU
runtime for its MoE path), so the fixture freezes this build's pinned oracle:
tests/test_golden_fixtures.py re-derives it on every CPU run to catch drift,
and the GPU tests compare the HIP path against it.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(HERE.parent))

import oracle  # noqa: E402
from moe_cases import dequant_weights_f32, make_case  # noqa: E402

FIXTURE = HERE / "tiny_seed0.npz"
SHAPE = dict(T=32, H=256, I=128, E=4, k=2, BM=16)


def build_fixture() -> dict[str, np.ndarray]:
    c = make_case(**SHAPE, seed=0, routing="softmax")
    st = oracle.moe_layer_stages(c.x, c.topk_ids, c.topk_w, c.w13_q, c.w13_s, c.w2_q, c.w2_s, c.BM)
    _, mag13, bound13 = oracle.grouped_gemm(st["q1"], st["s1"], c.w13_q, c.w13_s, st["sorted_ids"],
                                            st["expert_ids"], st["ntpp"], c.BM, c.S, c.k, with_magnitude=True,
                                            with_bound=True)
    _, mag2, bound2 = oracle.grouped_gemm(st["q2"], st["s2"], c.w2_q, c.w2_s, st["sorted_ids"],
                                          st["expert_ids"], st["ntpp"], c.BM, c.S, 1,
                                          topk_w=c.topk_w.ravel(), with_magnitude=True, with_bound=True)
    w1 = dequant_weights_f32(c.w13_q, c.w13_s)
    w2 = dequant_weights_f32(c.w2_q, c.w2_s)
    x = oracle.bf16_to_f32(c.x)
    golden = oracle.golden_moe(x, c.topk_ids, c.topk_w, w1, w2)
    atol = oracle.calibrated_atol(x, c.topk_ids, c.topk_w, w1, w2)
    return {
        "shape": np.array([SHAPE[k] for k in ("T", "H", "I", "E", "k", "BM")], np.int64),
        "x": c.x, "topk_ids": c.topk_ids, "topk_w": c.topk_w,
        "w13_q": c.w13_q, "w13_s": c.w13_s, "w2_q": c.w2_q, "w2_s": c.w2_s,
        "q1": st["q1"], "s1": st["s1"],
        "sorted_ids": st["sorted_ids"], "expert_ids": st["expert_ids"],
        "ntpp": np.array([st["ntpp"]], np.int32),
        "c13": st["c13"], "mag13": mag13, "bound13": bound13, "h": st["h"], "q2": st["q2"], "s2": st["s2"],
        "D": st["D"], "mag2": mag2, "bound2": bound2, "y": st["y"],
        "golden": golden, "atol": np.array([atol], np.float64),
    }


if __name__ == "__main__":
    fx = build_fixture()
    np.savez_compressed(FIXTURE, **fx)
    print(f"wrote {FIXTURE} ({FIXTURE.stat().st_size} bytes)")
