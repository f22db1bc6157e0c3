"""Synthetic MoE-layer workloads (the five benchmark configurations), generated
directly on the GPU.

Distributions follow the reference's data builders: activations ~N(0,1) in
bf16 (moe_bench/data/bundle.py:43-50), 128x128 block-quantised FP8 weights
(data/checkpoint.py:55-68; the weight std is N(0, 0.02) as the benchmark
configurations state), and router top-k with renormalised fp32 weights / int32
ids (data/routing.py:49-74): softmax or sigmoid scores over N(0,1) logits, or
k distinct experts per token drawn from a Zipf law over a seeded expert
permutation (routing.py:32-38).  Generation happens outside any timed region.
"""
from __future__ import annotations

from dataclasses import asdict, dataclass

import torch

from . import ops


@dataclass(frozen=True)
class Workload:
    name: str
    T: int            # tokens (reference shape.M)
    H: int            # hidden (reference shape.K)
    I: int            # per-expert intermediate (reference shape.n_down)
    E: int            # experts
    top_k: int
    block_m: int      # moe_align block size
    routing: str      # softmax | sigmoid | zipf
    zipf_alpha: float = 1.2
    weight_std: float = 0.02
    n_chunks: int = 1
    n_streams: int = 1
    seed: int = 0

    @property
    def S(self) -> int:
        return self.T * self.top_k

    @property
    def gemm_flop(self) -> int:
        """Algorithmic FLOP of both grouped GEMMs (padding excluded): 6*S*H*I."""
        return 6 * self.S * self.H * self.I

    def describe(self) -> dict:
        return asdict(self)


CONFIGS: dict[str, Workload] = {
    "tiny": Workload("tiny", 64, 256, 512, 8, 2, 64, "softmax"),
    "mixtral": Workload("mixtral", 4096, 4096, 14336, 8, 2, 128, "softmax"),
    "dsv3": Workload("dsv3", 8192, 7168, 2048, 256, 8, 128, "sigmoid"),
    "dsv3_decode": Workload("dsv3_decode", 128, 7168, 2048, 256, 8, 32, "zipf"),  # BM from {16, 32, 64}: 32 is fastest
    # the config names no block size: 256 is fastest for both the 4-chunk pipeline and one pass
    "qwen3": Workload("qwen3", 16384, 2048, 768, 128, 8, 256, "softmax", n_chunks=4, n_streams=2),
}


@dataclass
class LayerData:
    x: torch.Tensor          # [T, H] bf16
    topk_ids: torch.Tensor   # [T, k] int32
    topk_w: torch.Tensor     # [T, k] fp32
    w13: torch.Tensor        # [E, 2I, H] e4m3fn
    w13_s: torch.Tensor      # [E, 2I/128, H/128] fp32
    w2: torch.Tensor         # [E, H, I] e4m3fn
    w2_s: torch.Tensor       # [E, H/128, I/128] fp32


def route(logits: torch.Tensor, wl: Workload, gen: torch.Generator) -> tuple[torch.Tensor, torch.Tensor]:
    k = wl.top_k
    if wl.routing == "softmax":
        scores = torch.softmax(logits, dim=-1)
    elif wl.routing == "sigmoid":
        scores = torch.sigmoid(logits)
    elif wl.routing == "zipf":
        perm = torch.randperm(wl.E, generator=gen, device=logits.device)
        probs = torch.empty(wl.E, dtype=torch.float32, device=logits.device)
        probs[perm] = torch.arange(1, wl.E + 1, dtype=torch.float32, device=logits.device).pow(-wl.zipf_alpha)
        probs = probs / probs.sum()
        ids = torch.multinomial(probs.expand(wl.T, wl.E), k, replacement=False, generator=gen)
        w = torch.softmax(torch.randn((wl.T, k), generator=gen, device=logits.device), dim=-1)
        return ids.to(torch.int32).contiguous(), w.float().contiguous()
    else:
        raise ValueError(f"unknown routing {wl.routing}")
    w, ids = torch.topk(scores, k, dim=-1)
    w = w / w.sum(dim=-1, keepdim=True)
    return ids.to(torch.int32).contiguous(), w.float().contiguous()


def generate(wl: Workload, device: str | torch.device = "cuda", expert_chunk: int = 8) -> LayerData:
    dev = torch.device(device)
    gen = torch.Generator(device=dev).manual_seed(wl.seed)
    x = torch.randn((wl.T, wl.H), generator=gen, device=dev).to(torch.bfloat16)
    logits = torch.randn((wl.T, wl.E), generator=gen, device=dev)
    ids, w = route(logits, wl, gen)
    fp8 = ops.FP8
    w13 = torch.empty((wl.E, 2 * wl.I, wl.H), dtype=fp8, device=dev)
    w13_s = torch.empty((wl.E, 2 * wl.I // 128, wl.H // 128), dtype=torch.float32, device=dev)
    w2 = torch.empty((wl.E, wl.H, wl.I), dtype=fp8, device=dev)
    w2_s = torch.empty((wl.E, wl.H // 128, wl.I // 128), dtype=torch.float32, device=dev)
    for e0 in range(0, wl.E, expert_chunk):
        e1 = min(wl.E, e0 + expert_chunk)
        src = torch.randn((e1 - e0, 2 * wl.I, wl.H), generator=gen, device=dev) * wl.weight_std
        ops.quantize_block128(src, w13[e0:e1], w13_s[e0:e1])
        del src
        src = torch.randn((e1 - e0, wl.H, wl.I), generator=gen, device=dev) * wl.weight_std
        ops.quantize_block128(src, w2[e0:e1], w2_s[e0:e1])
        del src
    torch.cuda.synchronize(dev)
    return LayerData(x, ids, w, w13, w13_s, w2, w2_s)
