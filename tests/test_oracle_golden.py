"""Pins the end-to-end golden (verify.py:14-47 restated in numpy), the
three-gate comparator (verify.py:50-105) and the oracle's stage chain.

Restates the reference's own tests as known-answer checks:
tests/test_golden.py:9-26 (E=1, top-1 golden equals a direct FFN),
tests/test_golden.py:38-45 (report keys), tests/test_verify_gate.py:8-45
(all-zero output fails, near-identical passes, legacy atol-only call,
uniformly scaled output fails with the scale reported).  The stage chain
(quant -> align -> W13 -> silu*up -> quant -> W2 -> reduce) is held to the
golden through the reference worker's gates (worker.py:107-146) and to an
fp32 evaluation on its own dequantised intermediates through the 2e-2 bound.
The two checkers the GPU layer tests use are pinned on their own:
dequant_reference by a closed form (a scaled-permutation W2), and
calibrated_atol by the torch restatement of the golden run in both of its
activation modes (tests/calibrate_tolerance.py:17-25's rule).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from moe_cases import dequant_weights_f32, make_case


def silu(x):
    return x / (1.0 + np.exp(-x))


def test_golden_e1_top1_matches_direct_ffn():
    rng = np.random.default_rng(3)
    hidden = oracle.bf16_to_f32(oracle.f32_to_bf16(rng.standard_normal((5, 3)).astype(np.float32)))
    w1 = oracle.bf16_to_f32(oracle.f32_to_bf16(rng.standard_normal((1, 4, 3)).astype(np.float32)))
    w2 = oracle.bf16_to_f32(oracle.f32_to_bf16(rng.standard_normal((1, 3, 2)).astype(np.float32)))
    ids = np.zeros((5, 1), np.int32)
    wts = np.ones((5, 1), np.float32)
    golden = oracle.golden_moe(hidden, ids, wts, w1, w2, act_quant="none")
    gu = hidden.astype(np.float64) @ w1[0].T.astype(np.float64)
    direct = (silu(gu[:, :2]) * gu[:, 2:]) @ w2[0].T.astype(np.float64)
    np.testing.assert_allclose(golden, direct, rtol=1e-5, atol=1e-6)


def test_golden_weights_slots_and_shared_expert():
    rng = np.random.default_rng(4)
    T, H, I, E, k = 6, 4, 3, 3, 2
    hidden = rng.standard_normal((T, H)).astype(np.float32)
    w1 = rng.standard_normal((E, 2 * I, H)).astype(np.float32)
    w2 = rng.standard_normal((E, H, I)).astype(np.float32)
    sw1 = rng.standard_normal((1, 2 * I, H)).astype(np.float32)
    sw2 = rng.standard_normal((1, H, I)).astype(np.float32)
    ids = np.array([[0, 2], [1, 0], [2, 1], [0, 1], [2, 0], [1, 2]], np.int32)
    wts = rng.uniform(0, 1, (T, k)).astype(np.float32)

    def ffn(x, a, b):
        gu = x.astype(np.float64) @ a.T
        return (silu(gu[:, :I]) * gu[:, I:]) @ b.T

    ref = np.zeros((T, H))
    for t in range(T):
        for i in range(k):
            ref[t] += wts[t, i] * ffn(hidden[t:t + 1], w1[ids[t, i]], w2[ids[t, i]])[0]
    ref += ffn(hidden, sw1[0], sw2[0])
    got = oracle.golden_moe(hidden, ids, wts, w1, w2, sw1, sw2, act_quant="none")
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)


def test_compare_outputs_report_keys():
    rep = oracle.compare_outputs(np.array([[1.01, 1.99]]), np.array([[1.0, 2.0]]), atol=0.02, rtol=0.0)
    assert rep["pass"] is True
    assert {"max_abs", "max_rel", "cos_sim", "pass", "rel_p99", "scale"} <= set(rep)


def test_gate_rejects_all_zero_output():
    g = np.random.default_rng(0).standard_normal((256, 64)).astype(np.float32)
    rep = oracle.compare_outputs(np.zeros_like(g), g, atol=0.2, rtol=0.0, cos_threshold=0.99,
                                 rel_p99_threshold=0.05)
    assert rep["pass"] is False


def test_gate_accepts_near_identical():
    g = np.random.default_rng(0).standard_normal((256, 64)).astype(np.float32)
    rep = oracle.compare_outputs(g * 1.0001, g, atol=0.2, rtol=0.0, cos_threshold=0.999,
                                 rel_p99_threshold=0.05)
    assert rep["pass"] is True


def test_gate_legacy_atol_only_call():
    g = np.ones((8, 8), np.float32)
    rep = oracle.compare_outputs(g * 1.01, g, atol=0.2, rtol=0.0)
    assert rep["pass"] is True and "rel_p99" in rep and "scale" in rep


def test_gate_rejects_uniformly_scaled_output():
    g = np.random.default_rng(0).standard_normal((256, 64)).astype(np.float32)
    rep = oracle.compare_outputs(g * 0.5, g, atol=0.2, rtol=0.0, cos_threshold=0.99,
                                 rel_p99_threshold=5.0, scale_tolerance=0.05)
    assert rep["pass"] is False
    assert abs(rep["scale"] - 0.5) < 0.01


@pytest.mark.parametrize("routing", ["softmax", "sigmoid"])
def test_stage_chain_meets_golden_gates(routing):
    c = make_case(T=48, H=256, I=256, E=4, k=2, BM=16, seed=11, routing=routing)
    st = oracle.moe_layer_stages(c.x, c.topk_ids, c.topk_w, c.w13_q, c.w13_s, c.w2_q, c.w2_s, c.BM)
    y = oracle.bf16_to_f32(st["y"])
    w1 = dequant_weights_f32(c.w13_q, c.w13_s)
    w2 = dequant_weights_f32(c.w2_q, c.w2_s)
    x = oracle.bf16_to_f32(c.x)
    golden = oracle.golden_moe(x, c.topk_ids, c.topk_w, w1, w2)
    rep = oracle.compare_outputs(y, golden, atol=0.0, rtol=0.0, **oracle.DEFAULT_GATES)
    assert rep["pass"], rep
    atol = oracle.calibrated_atol(x, c.topk_ids, c.topk_w, w1, w2)
    assert rep["max_abs"] <= atol, (rep["max_abs"], atol)
    # the chain against fp32 arithmetic on its own dequantised operands
    ref = oracle.dequant_reference(st["q2"], st["s2"], c.topk_ids, c.topk_w, c.w2_q, c.w2_s)
    rep2 = oracle.compare_outputs(y, ref, atol=0.0, rtol=0.0)
    assert rep2["max_abs_rel"] <= oracle.MAX_ABS_REL, rep2
    # a dropped routed weight fails the gates
    bad = oracle.moe_layer_stages(c.x, c.topk_ids, np.ones_like(c.topk_w), c.w13_q, c.w13_s,
                                  c.w2_q, c.w2_s, c.BM)
    rep3 = oracle.compare_outputs(oracle.bf16_to_f32(bad["y"]), golden, atol=0.0, rtol=0.0,
                                  **oracle.DEFAULT_GATES)
    assert rep3["pass"] is False


def test_dequant_reference_closed_form():
    """dequant_reference on a W2 that is a scaled permutation: every expert's
    dequantised W2 maps intermediate column perm[n] to output column n, so
    y[t, n] = sum_i w[t,i] * s_w2(e) * deq(h[t*k+i, perm_e[n]]) exactly.  A
    transposed weight, a dropped routed weight, a wrong scale axis or a slot
    paired with the wrong expert moves whole entries."""
    rng = np.random.default_rng(21)
    T, k, H, I, E = 6, 2, 256, 256, 3
    lut = oracle.e4m3_lut().astype(np.float64)
    one = int(np.where(lut == 1.0)[0][0])
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    w = rng.random((T, k), dtype=np.float32) + np.float32(0.25)
    hq = rng.integers(0, 0x7E, size=(T * k, I), dtype=np.uint8)
    hs = (rng.random((T * k, I // 128)) + 0.5).astype(np.float32)
    w2q = np.zeros((E, H, I), np.uint8)
    perms = [rng.permutation(I)[:H] for _ in range(E)]
    for e in range(E):
        w2q[e, np.arange(H), perms[e]] = one
    w2s = np.stack([np.full((H // 128, I // 128), 2.0 ** (e - 1), np.float32) for e in range(E)])
    got = oracle.dequant_reference(hq, hs, ids, w, w2q, w2s).astype(np.float64)
    h = lut[hq] * np.repeat(hs.astype(np.float64), 128, axis=1)
    want = np.zeros((T, H))
    for t in range(T):
        for i in range(k):
            e = ids[t, i]
            want[t] += float(w[t, i]) * 2.0 ** (e - 1) * h[t * k + i, perms[e]]
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=0)


def test_calibrated_atol_against_the_torch_golden():
    """calibrated_atol is tests/calibrate_tolerance.py:17-25's rule, 1.5 x the
    largest |golden(group128) - golden(no quant)|; held to the torch
    restatement of the golden (oracle/golden_torch.py, pinned to the C oracle
    separately) evaluated in both modes."""
    import torch

    from oracle.golden_torch import golden_moe_torch
    c = make_case(T=40, H=256, I=256, E=4, k=2, BM=16, seed=13, routing="softmax")
    w1 = dequant_weights_f32(c.w13_q, c.w13_s)
    w2 = dequant_weights_f32(c.w2_q, c.w2_s)
    x = oracle.bf16_to_f32(c.x)
    args = (torch.from_numpy(np.asarray(x, np.float32)), torch.from_numpy(c.topk_ids).long(),
            torch.from_numpy(c.topk_w), lambda e: torch.from_numpy(w1[e]), lambda e: torch.from_numpy(w2[e]))
    fp8 = golden_moe_torch(*args, act_quant="group128").numpy()
    none = golden_moe_torch(*args, act_quant="none").numpy()
    want = 1.5 * float(np.abs(fp8 - none).max())
    got = oracle.calibrated_atol(x, c.topk_ids, c.topk_w, w1, w2)
    assert want > 0 and abs(got - want) <= 1e-5 * want + 1e-7, (got, want)
    # a tolerance of another shape (the p99, or 1x the max) would differ
    assert abs(got - 1.5 * float(np.quantile(np.abs(fp8 - none), 0.99))) > 1e-3 * want
    assert abs(got - float(np.abs(fp8 - none).max())) > 0.3 * want
