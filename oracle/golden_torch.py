"""Torch CPU restatement of the reference's golden MoE path -- the CPU
baseline that bench.py times beside the GPU.  TEST INFRASTRUCTURE: only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it; the
product path (td_benchmark_amd) never imports anything under oracle/.

Each function restates the reference's torch code on the CPU:
* ``golden_moe_torch``: moe_bench/verify.py:14-47 (per-expert fp32 loop:
  1x128 quant-dequant of the routed rows, x @ W13^T, silu(gate) * up, a
  second quant-dequant, @ W2^T, routed-weight index_add_), with the weights
  dequantised one expert at a time (data/checkpoint.py:43-52) so that the
  DeepSeek-V3 layer fits in host memory;
* ``group_quant_dequant_torch``: verify.py:108-117;
* ``dequant_expert_torch``: data/checkpoint.py:43-52, then bf16;
* ``quant_group128_torch``: the codes and scales of the same quant
  (scale = max(amax/448, 1e-12), e4m3(clamp(x/scale, +-448)));
* ``align_torch``: moe_align_block_size's outputs by the torch ops the
  reference's dispatch pre-chain uses (docs/exp/EXP-010-moe-align.md: stable
  argsort + bincount + cumsum), padded to the block size
  (tdx/kernels/moe_utils.py:168-217);
* ``reduce_torch``: torch.sum(C_down.view(T, k, H), dim=1)
  (overlap/overlap_forward.py:304-313).

Pinned by tests/test_oracle_torch.py against the C oracle (bit-exact for the
quant, align and reduce; the golden within fp32 matmul reordering of the numpy
restatement, which is itself pinned by the reference's known answers)."""
from __future__ import annotations

from typing import Callable

import torch
import torch.nn.functional as F


def group_quant_dequant_torch(x: torch.Tensor, block: int = 128) -> torch.Tensor:
    """1x128 quant-dequant of the last dimension (zero-padded to the block)."""
    n = x.shape[-1]
    pad = (n + block - 1) // block * block
    xp = F.pad(x.float(), (0, pad - n))
    blocks = xp.view(*xp.shape[:-1], pad // block, block)
    scale = (blocks.abs().amax(dim=-1, keepdim=True) / 448.0).clamp(min=1e-12)
    q = (blocks / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).float() * scale
    return q.view(*xp.shape)[..., :n].contiguous()


def quant_group128_torch(x_bf16: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """x [T, H] bf16 (H % 128 == 0) -> (codes [T, H] e4m3fn, scales [T, H/128] fp32)."""
    T, H = x_bf16.shape
    blocks = x_bf16.float().view(T, H // 128, 128)
    scale = (blocks.abs().amax(dim=-1, keepdim=True) / 448.0).clamp(min=1e-12)
    q = (blocks / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q.view(T, H), scale.view(T, H // 128)


def align_torch(topk_ids: torch.Tensor, num_experts: int, block_size: int):
    """(sorted_token_ids, expert_ids, num_tokens_post_padded) with slots in
    ascending order within each expert and pad value S; ids outside
    [0, num_experts) are dropped."""
    flat = topk_ids.reshape(-1).long()
    S = flat.numel()
    valid = (flat >= 0) & (flat < num_experts)
    key = torch.where(valid, flat, torch.full_like(flat, num_experts))
    order = torch.argsort(key, stable=True)
    counts = torch.bincount(key, minlength=num_experts + 1)[:num_experts]
    padded = (counts + block_size - 1) // block_size * block_size
    ntpp = int(padded.sum())
    starts = torch.cumsum(padded, 0) - padded
    cstarts = torch.cumsum(counts, 0) - counts
    sorted_ids = torch.full((ntpp,), S, dtype=torch.int32)
    n_valid = int(counts.sum())
    e_of = key[order[:n_valid]]
    rank = torch.arange(n_valid) - cstarts[e_of]
    sorted_ids[starts[e_of] + rank] = order[:n_valid].to(torch.int32)
    expert_ids = torch.repeat_interleave(torch.arange(num_experts, dtype=torch.int32), padded // block_size)
    return sorted_ids, expert_ids, ntpp


def reduce_torch(D_bf16: torch.Tensor, T: int, k: int) -> torch.Tensor:
    """y [T, H] = sum over the k rows of each token, fp32 accumulate, bf16 out."""
    return D_bf16.view(T, k, -1).float().sum(dim=1).to(torch.bfloat16)


def dequant_expert_torch(q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """One expert's FP8 [N, K] weights with 128x128 block scales -> the
    bf16-dequantised values as fp32 (data/checkpoint.py:43-52; the golden
    consumes ckpt.w*.bf16)."""
    N, K = q.shape
    sc = s.float().repeat_interleave(128, 0).repeat_interleave(128, 1)[:N, :K]
    return (q.float() * sc).to(torch.bfloat16).float()


def golden_moe_torch(hidden: torch.Tensor, topk_ids: torch.Tensor, topk_w: torch.Tensor,
                     w1: Callable[[int], torch.Tensor], w2: Callable[[int], torch.Tensor],
                     experts=None, act_quant: str = "group128", out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 [T, H] golden over ``experts`` (all experts with routed slots when
    None); ``w1(e)`` / ``w2(e)`` return expert e's fp32 [2I, H] / [H, I].
    With ``out`` the contributions are added into it (the reference allocates
    its output once for the whole expert loop)."""
    hidden = hidden.float()
    qdq = group_quant_dequant_torch if act_quant == "group128" else (lambda v: v.float())
    ids = topk_ids
    if experts is None:
        experts = torch.unique(ids[(ids >= 0)]).tolist()
    for e in experts:
        m = (ids == e).nonzero(as_tuple=False)
        if m.numel() == 0:
            continue
        rows, slots = m[:, 0], m[:, 1]
        x = qdq(hidden[rows])
        gate, up = (x @ w1(e).float().T).chunk(2, dim=-1)
        inter = qdq(F.silu(gate) * up)
        contrib = inter @ w2(e).float().T
        if out is None:
            out = torch.zeros((hidden.shape[0], contrib.shape[1]), dtype=torch.float32)
        out.index_add_(0, rows, contrib * topk_w[rows, slots].float().unsqueeze(-1))
    return out
