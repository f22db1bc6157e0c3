"""Seeded synthetic MoE cases shared by the CPU and GPU tests.

Inputs follow the shapes and distributions of the build's benchmark configs:
activations ~N(0,1) rounded to bf16, router logits ~N(0,1) with softmax or
sigmoid top-k and renormalised weights (reference moe_bench/data/routing.py:
49-74), or Zipf expert draws without replacement; weights ~N(0, std) block
quantised 128x128 with the CPU oracle (reference data/checkpoint.py:28-40).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

import oracle


@dataclass
class MoeCase:
    T: int
    H: int
    I: int
    E: int
    k: int
    BM: int
    x: np.ndarray          # bf16 bits [T, H]
    topk_ids: np.ndarray   # int32 [T, k]
    topk_w: np.ndarray     # fp32 [T, k]
    w13_q: np.ndarray      # uint8 [E, 2I, H]
    w13_s: np.ndarray      # fp32 [E, 2I/128, H/128]
    w2_q: np.ndarray       # uint8 [E, H, I]
    w2_s: np.ndarray       # fp32 [E, H/128, I/128]

    @property
    def S(self) -> int:
        return self.T * self.k


def route(logits: np.ndarray, k: int, kind: str, rng: np.random.Generator,
          zipf_alpha: float = 1.2) -> tuple[np.ndarray, np.ndarray]:
    T, E = logits.shape
    if kind == "softmax":
        z = logits - logits.max(axis=1, keepdims=True)
        p = np.exp(z)
        p /= p.sum(axis=1, keepdims=True)
    elif kind == "sigmoid":
        p = 1.0 / (1.0 + np.exp(-logits))
    elif kind == "zipf":
        perm = rng.permutation(E)
        probs = np.empty(E)
        probs[perm] = np.arange(1, E + 1, dtype=np.float64) ** (-zipf_alpha)
        probs /= probs.sum()
        ids = np.stack([rng.choice(E, size=k, replace=False, p=probs) for _ in range(T)])
        w = rng.standard_normal((T, k))
        w = np.exp(w - w.max(axis=1, keepdims=True))
        w /= w.sum(axis=1, keepdims=True)
        return ids.astype(np.int32), w.astype(np.float32)
    elif kind == "one_expert":
        ids = np.zeros((T, k), np.int32)
        ids[:, :] = np.arange(k, dtype=np.int32)[None, :] % E
        w = np.full((T, k), 1.0 / k, np.float32)
        return ids, w
    else:
        raise ValueError(kind)
    ids = np.argsort(-p, axis=1, kind="stable")[:, :k]
    w = np.take_along_axis(p, ids, axis=1)
    w = w / w.sum(axis=1, keepdims=True)
    return ids.astype(np.int32), w.astype(np.float32)


def make_case(T: int, H: int, I: int, E: int, k: int, BM: int, seed: int = 0,
              routing: str = "softmax", weight_std: float = 0.02, x_std: float = 1.0) -> MoeCase:
    rng = np.random.default_rng(seed)
    x = oracle.f32_to_bf16(rng.standard_normal((T, H), dtype=np.float32) * np.float32(x_std))
    logits = rng.standard_normal((T, E), dtype=np.float32)
    ids, w = route(logits, k, routing, rng)
    w13 = rng.standard_normal((E, 2 * I, H), dtype=np.float32) * np.float32(weight_std)
    w2 = rng.standard_normal((E, H, I), dtype=np.float32) * np.float32(weight_std)
    w13_q, w13_s = oracle.quant_block128(w13)
    w2_q, w2_s = oracle.quant_block128(w2)
    return MoeCase(T, H, I, E, k, BM, x, ids, w, w13_q, w13_s, w2_q, w2_s)


def dequant_weights_f32(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    """bf16-dequantised weights as fp32 (the golden's ckpt.w*.bf16 view)."""
    return oracle.bf16_to_f32(oracle.dequant_block128(q, s))


# ---------------------------------------------------------------- torch glue

def to_gpu(case: MoeCase):
    import torch

    dev = torch.device("cuda", 0)

    def u8(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev).view(torch.float8_e4m3fn)

    def bf16(a):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev).view(torch.bfloat16)

    def f32(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)

    def i32(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)

    return dict(x=bf16(case.x), topk_ids=i32(case.topk_ids), topk_w=f32(case.topk_w),
                w13=u8(case.w13_q), w13_s=f32(case.w13_s), w2=u8(case.w2_q), w2_s=f32(case.w2_s))


def bf16_bits(t) -> np.ndarray:
    return t.detach().contiguous().cpu().view(dtype=__import__("torch").int16).numpy().view(np.uint16)


def u8_bits(t) -> np.ndarray:
    import torch
    return t.detach().contiguous().cpu().view(torch.uint8).numpy()


def e4m3_ulp_diff(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """|code difference| in e4m3 ULPs for same-sign codes (codes are monotone
    in magnitude within a sign), 255 where the signs differ and both are non-zero."""
    a = a.astype(np.int16)
    b = b.astype(np.int16)
    sa, sb = a >> 7, b >> 7
    ma, mb = a & 0x7F, b & 0x7F
    d = np.abs(ma - mb)
    opposite = (sa != sb) & ~((ma == 0) & (mb == 0))
    # crossing zero: +m vs -n differ by m+n ulps
    d = np.where(opposite, ma + mb, d)
    return d
