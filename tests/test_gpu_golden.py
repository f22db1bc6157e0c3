"""The HIP path on the committed fixture tests/golden/tiny_seed0.npz.

Each stage runs on the GPU through the C ABI on the fixture's own inputs
(or on the fixture's previous-stage outputs, so that stages are checked in
isolation) and is compared with the fixture's expected outputs:
quant codes/scales and align outputs bit-exact; GEMM outputs within the
FP8 matrix core's accumulation bound (|d| <= 2^-7|ref| + the oracle's per-output
bound, fixture arrays bound13 / bound2);
silu*up within one bf16 ulp on at most 0.1% of elements; the reduce bit-exact;
the full layer through the reference worker's gates and the calibrated
tolerance against the fixture's fp32 golden."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

import oracle
from moe_cases import a7_account, a7_assert, bf16_bits, u8_bits

pytestmark = pytest.mark.gpu

FIXTURE = Path(__file__).resolve().parent / "golden" / "tiny_seed0.npz"


@pytest.fixture(scope="module")
def fx():
    with np.load(FIXTURE) as f:
        return {k: f[k] for k in f.files}


@pytest.fixture(scope="module")
def dev(fx):
    import torch

    d = torch.device("cuda", 0)

    def u8(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(d).view(torch.float8_e4m3fn)

    def bf16(a):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(d).view(torch.bfloat16)

    def f32(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(d)

    def i32(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(d)

    return dict(u8=u8, bf16=bf16, f32=f32, i32=i32, device=d)


def shape(fx):
    return fx["shape"].tolist()


def test_quant_and_align_bit_exact(fx, dev):
    import torch

    from td_benchmark_amd import ops

    print("case: golden tiny_seed0 quant+align", flush=True)
    T, H, I, E, k, BM = shape(fx)
    q, s = ops.per_token_group_quant_fp8(dev["bf16"](fx["x"]))
    torch.cuda.synchronize()
    assert np.array_equal(u8_bits(q), fx["q1"])
    assert np.array_equal(s.cpu().numpy(), fx["s1"])
    sorted_ids, eids, ntpp = ops.moe_align_block_size(dev["i32"](fx["topk_ids"].ravel()), BM, E)
    torch.cuda.synchronize()
    assert int(ntpp.item()) == int(fx["ntpp"][0])
    assert np.array_equal(sorted_ids.cpu().numpy(), fx["sorted_ids"])
    assert np.array_equal(eids.cpu().numpy(), fx["expert_ids"])


def test_w13_gemm_and_silu(fx, dev):
    import torch

    from td_benchmark_amd import ops

    print("case: golden tiny_seed0 W13 + silu", flush=True)
    T, H, I, E, k, BM = shape(fx)
    S = T * k
    c13 = torch.zeros((S, 2 * I), dtype=torch.bfloat16, device=dev["device"])
    ops.dispatch_fused_moe_kernel(dev["u8"](fx["q1"]), dev["u8"](fx["w13_q"]), c13, dev["f32"](fx["s1"]),
                                  dev["f32"](fx["w13_s"]), None, None, dev["i32"](fx["sorted_ids"]),
                                  dev["i32"](fx["expert_ids"]), dev["i32"](fx["ntpp"]), False, k,
                                  {"BLOCK_SIZE_M": BM})
    torch.cuda.synchronize()
    bad = oracle.gemm_close(bf16_bits(c13), fx["c13"], fx["bound13"])
    assert not bad.any(), f"{bad.sum()} W13 outputs outside the accumulation bound"
    h = torch.empty((S, I), dtype=torch.bfloat16, device=dev["device"])
    ops.silu_and_mul(h, dev["bf16"](fx["c13"]))
    torch.cuda.synchronize()
    d = np.abs(bf16_bits(h).astype(np.int32) - fx["h"].astype(np.int32))
    assert d.max() <= 1 and np.mean(d > 0) <= 1e-3


def test_fused_w13_codes(fx, dev):
    import torch

    from td_benchmark_amd import ops

    print("case: golden tiny_seed0 fused W13+silu+quant", flush=True)
    T, H, I, E, k, BM = shape(fx)
    S = T * k
    hq, hs = ops.gemm_w13_silu_quant(dev["u8"](fx["q1"]), dev["f32"](fx["s1"]), dev["u8"](fx["w13_q"]),
                                     dev["f32"](fx["w13_s"]), dev["i32"](fx["sorted_ids"]),
                                     dev["i32"](fx["expert_ids"]), dev["i32"](fx["ntpp"]), S, k, BM)
    torch.cuda.synchronize()
    # the GPU's own C13 and h (unfused chain, same kernels) to trace differences
    c13 = torch.zeros((S, 2 * I), dtype=torch.bfloat16, device=dev["device"])
    ops.dispatch_fused_moe_kernel(dev["u8"](fx["q1"]), dev["u8"](fx["w13_q"]), c13, dev["f32"](fx["s1"]),
                                  dev["f32"](fx["w13_s"]), None, None, dev["i32"](fx["sorted_ids"]),
                                  dev["i32"](fx["expert_ids"]), dev["i32"](fx["ntpp"]), False, k,
                                  {"BLOCK_SIZE_M": BM})
    h = torch.empty((S, I), dtype=torch.bfloat16, device=dev["device"])
    ops.silu_and_mul(h, c13)
    torch.cuda.synchronize()
    codes, scales = u8_bits(hq), hs.cpu().numpy()
    pos = np.nonzero(fx["sorted_ids"][: int(fx["ntpp"][0])] < S)[0]
    slots = fx["sorted_ids"][pos]
    # codes follow the GPU's own C13, which may differ from the oracle's by the
    # MFMA accumulation bound: each differing code traced to a differing h or
    # scale, each differing h to a C13 flip inside that bound; scales
    # bit-exact wherever the group's h matches
    _, c13_f32 = oracle.grouped_gemm(fx["q1"], fx["s1"], fx["w13_q"], fx["w13_s"], fx["sorted_ids"],
                                     fx["expert_ids"], int(fx["ntpp"][0]), BM, S, k, with_f32=True)
    rep = a7_account(codes[pos], scales[pos], bf16_bits(h)[slots], bf16_bits(c13)[slots], fx["q2"][slots],
                     fx["s2"][slots], fx["h"][slots], fx["c13"][slots], c13_f32[slots], fx["bound13"][slots])
    a7_assert(rep, "golden tiny_seed0 fused W13")


def test_w2_gemm_and_reduce(fx, dev):
    import torch

    from td_benchmark_amd import ops

    print("case: golden tiny_seed0 W2 + reduce", flush=True)
    T, H, I, E, k, BM = shape(fx)
    S = T * k
    D = torch.zeros((S, H), dtype=torch.bfloat16, device=dev["device"])
    ops.dispatch_fused_moe_kernel(dev["u8"](fx["q2"]), dev["u8"](fx["w2_q"]), D, dev["f32"](fx["s2"]),
                                  dev["f32"](fx["w2_s"]), None, dev["f32"](fx["topk_w"]),
                                  dev["i32"](fx["sorted_ids"]), dev["i32"](fx["expert_ids"]),
                                  dev["i32"](fx["ntpp"]), True, 1, {"BLOCK_SIZE_M": BM})
    torch.cuda.synchronize()
    bad = oracle.gemm_close(bf16_bits(D), fx["D"], fx["bound2"])
    assert not bad.any(), f"{bad.sum()} W2 outputs outside the accumulation bound"
    y = torch.empty((T, H), dtype=torch.bfloat16, device=dev["device"])
    ops.moe_sum(dev["bf16"](fx["D"]), y, k)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(y), fx["y"])


def test_full_layer_meets_golden_gates(fx, dev):
    import torch

    from td_benchmark_amd import ops

    print("case: golden tiny_seed0 full layer", flush=True)
    T, H, I, E, k, BM = shape(fx)
    runner = ops.FusedExpertsRunner(dev["u8"](fx["w13_q"]), dev["f32"](fx["w13_s"]), dev["u8"](fx["w2_q"]),
                                    dev["f32"](fx["w2_s"]), T, k, BM)
    y = runner.run(dev["bf16"](fx["x"]), dev["f32"](fx["topk_w"].ravel()), dev["i32"](fx["topk_ids"].ravel()))
    torch.cuda.synchronize()
    yf = oracle.bf16_to_f32(bf16_bits(y))
    rep = oracle.compare_outputs(yf, fx["golden"], atol=0.0, rtol=0.0, **oracle.DEFAULT_GATES)
    assert rep["pass"], rep
    assert rep["max_abs"] <= float(fx["atol"][0]), (rep["max_abs"], float(fx["atol"][0]))
