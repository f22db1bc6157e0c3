"""Torch-facing operators of the MI355X MoE expert path.

Each function mirrors the vLLM operator the reference calls at that point of
its ``fused_experts`` decomposition (moe_bench/overlap/overlap_forward.py:
153-313), with the same argument meaning, and launches the hand-written HIP
kernels of ``libmoe_mi355x.so`` through the C ABI (include/moe_mi355x.h) on the
current torch stream.  PyTorch only provides device memory and the stream;
there is no torch compute and no fallback on the path.
"""
from __future__ import annotations

import ctypes
from typing import Any

import torch

from ._lib import check, lib

FP8 = torch.float8_e4m3fn
BLOCK_SHAPE = [128, 128]
SUPPORTED_BLOCK_M = (16, 32, 64, 128, 256)
# workgroup -> tile orders of the grouped GEMM (include/moe_mi355x.h)
TILE_ORDERS = {"expert_major": 0, "shuffled": 1, "half_phase": 2}


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


# The current stream's raw handle straight from torch's C++ side (the accessor
# torch's own code generator uses); torch.cuda.current_stream() builds a Stream
# object through a device-index lookup and costs about 2.7 us a call, which a
# launch-bound layer of seven kernels pays on every op.
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_CUR_DEVICE = getattr(torch._C, "_cuda_getDevice", None)


def _stream(stream: torch.cuda.Stream | None = None) -> ctypes.c_void_p:
    if stream is None:
        if _RAW_STREAM is not None and _CUR_DEVICE is not None:
            return ctypes.c_void_p(_RAW_STREAM(_CUR_DEVICE()))
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _need(t: torch.Tensor, name: str, dtype: torch.dtype | None = None,
          shape: tuple | None = None) -> None:
    """Checks of a tensor handed to the C ABI, which receives only pointers and
    sizes: a buffer smaller than the sizes say would be read or written out of
    bounds on the device, so dtype and shape are checked here, before the
    contiguity and device checks."""
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")


def _blocks128(n: int) -> int:
    return (n + 127) // 128


def _need_weights(w: torch.Tensor, w_scale: torch.Tensor, name: str) -> tuple[int, int, int]:
    """FP8 expert weights [E, N, K] and their 128x128 block scales
    [E, N/128, K/128] -> (E, N, K)."""
    if w.dim() != 3:
        raise ValueError(f"{name} must be [E, N, K], got {tuple(w.shape)}")
    E, N, K = w.shape
    _need(w, name, FP8)
    _need(w_scale, f"{name}_scale", torch.float32, (E, _blocks128(N), _blocks128(K)))
    return E, N, K


def _pad_fp8(w: torch.Tensor, dim: int, size: int) -> torch.Tensor:
    """FP8 weights [E, N, K] with dimension ``dim`` (1 or 2) zero-padded to
    ``size``: the zero code, as the reference's 128x128 block quant pads a
    ragged block (data/checkpoint.py:28-40), so the padded rows or columns
    contribute nothing to a GEMM."""
    if w.shape[dim] == size:
        return w
    shape = list(w.shape)
    shape[dim] = size
    out = torch.zeros(shape, dtype=torch.uint8, device=w.device)
    if dim == 1:
        out[:, : w.shape[1]] = w.view(torch.uint8)
    else:
        out[:, :, : w.shape[2]] = w.view(torch.uint8)
    return out.view(FP8)


def _need_routing(sorted_token_ids: torch.Tensor, expert_ids: torch.Tensor,
                  num_tokens_post_padded: torch.Tensor, block_m: int) -> None:
    """moe_align_block_size outputs: one expert id per block of sorted positions."""
    _need(sorted_token_ids, "sorted_token_ids", torch.int32)
    _need(expert_ids, "expert_ids", torch.int32)
    _need(num_tokens_post_padded, "num_tokens_post_padded", torch.int32)
    if num_tokens_post_padded.numel() < 1:
        raise ValueError("num_tokens_post_padded must hold one element")
    if expert_ids.numel() * block_m < sorted_token_ids.numel():
        raise ValueError(f"expert_ids has {expert_ids.numel()} blocks, fewer than the "
                         f"{sorted_token_ids.numel()} sorted positions need at block size {block_m}")


def _need_activations(A: torch.Tensor, A_scale: torch.Tensor, rows: int, cols: int | None = None) -> None:
    """FP8 activations [>= rows, cols] and their 1x128 group scales."""
    if A.dim() != 2:
        raise ValueError(f"A must be 2-D, got {tuple(A.shape)}")
    if cols is not None and A.shape[1] != cols:
        raise ValueError(f"A has {A.shape[1]} columns, expected {cols}")
    if A.shape[0] < rows:
        raise ValueError(f"A has {A.shape[0]} rows, the routing reads {rows}")
    _need(A, "A", FP8)
    _need(A_scale, "A_scale", torch.float32, (A.shape[0], _blocks128(A.shape[1])))


def _check_grouped_gemm(A, A_scale, B, B_scale, C, weights, sorted_token_ids, expert_ids,
                        num_tokens_post_padded, top_k: int, a_by_pos: bool, block_m: int,
                        row_width: int) -> int:
    """Operands of the grouped GEMM entry points -> S, the slots (rows of C)."""
    _need_weights(B, B_scale, "B")
    _need_routing(sorted_token_ids, expert_ids, num_tokens_post_padded, block_m)
    if top_k < 1:
        raise ValueError("top_k must be >= 1")
    if C.numel() % row_width:
        raise ValueError(f"C ({C.numel()} elements) is not a whole number of {row_width}-wide rows")
    S = C.numel() // row_width
    _need(C, "C", torch.bfloat16)
    rows = sorted_token_ids.numel() if a_by_pos else (S + top_k - 1) // top_k
    _need_activations(A, A_scale, rows)
    if weights is not None:
        _need(weights, "topk_weights", torch.float32)
        if weights.numel() < S:
            raise ValueError(f"topk_weights has {weights.numel()} entries for {S} slots")
    return S


# ---------------------------------------------------------------------------
# A1 / A7 -- 1x128 activation quant
# ---------------------------------------------------------------------------

def per_token_group_quant_fp8(x: torch.Tensor, group_size: int = 128,
                              out_q: torch.Tensor | None = None,
                              out_s: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """x [T,H] bf16 -> (q [T,H] e4m3fn, scales [T,ceil(H/128)] fp32).

    Arithmetic of moe_bench/verify.py:108-117 (scale = max(amax/448, 1e-12),
    q = e4m3(clamp(x/scale, +-448)); a last group of H mod 128 columns is
    quantised as the reference's zero padding leaves it); output form of
    vLLM's per_token_group_quant_fp8 as consumed by the grouped GEMM."""
    if group_size != 128:
        raise NotImplementedError("only 1x128 activation groups are implemented")
    if x.dim() != 2:
        raise ValueError(f"x must be [T, H], got {tuple(x.shape)}")
    _need(x, "x", torch.bfloat16)
    T, H = x.shape
    q = torch.empty((T, H), dtype=FP8, device=x.device) if out_q is None else out_q
    s = torch.empty((T, _blocks128(H)), dtype=torch.float32, device=x.device) if out_s is None else out_s
    _need(q, "out_q", FP8, (T, H))
    _need(s, "out_s", torch.float32, (T, _blocks128(H)))
    check(lib().moe_quant_group128(_ptr(x), T, H, _ptr(q), _ptr(s), _stream()), "moe_quant_group128")
    return q, s


def moe_kernel_quantize_input(A: torch.Tensor, A_scale: torch.Tensor | None, quant_dtype: Any,
                              per_act_token_quant: bool, block_shape: list[int] | None = None):
    """Signature of vLLM's moe_kernel_quantize_input as the reference calls it
    (overlap/overlap_forward.py:257-259): only the dynamic FP8 1x128 form."""
    if A_scale is not None or quant_dtype != FP8 or per_act_token_quant or list(block_shape or []) != BLOCK_SHAPE:
        raise NotImplementedError("only dynamic float8_e4m3fn with block_shape [128,128] is implemented")
    return per_token_group_quant_fp8(A)


# ---------------------------------------------------------------------------
# A2 -- 128x128 weight quant (build time)
# ---------------------------------------------------------------------------

def quantize_block128(w: torch.Tensor, out_q: torch.Tensor | None = None,
                      out_s: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 [E,N,K] -> (e4m3fn [E,N,K], scales [E,ceil(N/128),ceil(K/128)]),
    moe_bench/data/checkpoint.py:28-40 on the GPU."""
    if w.dim() != 3:
        raise ValueError(f"w must be [E, N, K], got {tuple(w.shape)}")
    _need(w, "w", torch.float32)
    E, N, K = w.shape
    q = torch.empty((E, N, K), dtype=FP8, device=w.device) if out_q is None else out_q
    s = (torch.empty((E, _blocks128(N), _blocks128(K)), dtype=torch.float32, device=w.device)
         if out_s is None else out_s)
    _need(q, "out_q", FP8, (E, N, K))
    _need(s, "out_s", torch.float32, (E, _blocks128(N), _blocks128(K)))
    check(lib().moe_quant_block128(_ptr(w), E, N, K, _ptr(q), _ptr(s), _stream()), "moe_quant_block128")
    return q, s


# ---------------------------------------------------------------------------
# A3 -- moe_align_block_size
# ---------------------------------------------------------------------------

def align_max_padded(num_slots: int, num_experts: int, block_size: int) -> int:
    return int(lib().moe_align_max_padded(num_slots, num_experts, block_size))


def align_workspace_bytes(num_slots: int, num_experts: int) -> int:
    return int(lib().moe_align_workspace_bytes(num_slots, num_experts))


class AlignBuffers:
    """Preallocated outputs + workspace of moe_align_block_size for S slots."""

    def __init__(self, num_slots: int, num_experts: int, block_size: int, device: Any):
        self.S, self.E, self.BM = num_slots, num_experts, block_size
        self.max_padded = align_max_padded(num_slots, num_experts, block_size)
        self.max_blocks = (self.max_padded + block_size - 1) // block_size
        self.sorted_ids = torch.empty(max(self.max_padded, 1), dtype=torch.int32, device=device)
        self.expert_ids = torch.empty(max(self.max_blocks, 1), dtype=torch.int32, device=device)
        self.ntpp = torch.empty(1, dtype=torch.int32, device=device)
        self.workspace = torch.empty(align_workspace_bytes(num_slots, num_experts), dtype=torch.uint8,
                                     device=device)

    def run(self, topk_ids: torch.Tensor,
            expert_map: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """``expert_map`` (int32 [E], global -> local expert id or -1): block
        expert ids are reported as local ids (expert parallelism)."""
        _need(topk_ids, "topk_ids", torch.int32)
        if topk_ids.numel() != self.S:
            raise ValueError(f"topk_ids has {topk_ids.numel()} slots, buffers were sized for {self.S}")
        if expert_map is None:
            check(lib().moe_align_block_size(_ptr(topk_ids), self.S, self.E, self.BM, _ptr(self.sorted_ids),
                                             _ptr(self.expert_ids), _ptr(self.ntpp), self.max_padded,
                                             _ptr(self.workspace), _stream()), "moe_align_block_size")
        else:
            _need(expert_map, "expert_map", torch.int32)
            if expert_map.numel() != self.E:
                raise ValueError(f"expert_map must have {self.E} entries")
            check(lib().moe_align_block_size_mapped(_ptr(topk_ids), self.S, self.E, self.BM, _ptr(expert_map),
                                                    _ptr(self.sorted_ids), _ptr(self.expert_ids), _ptr(self.ntpp),
                                                    self.max_padded, _ptr(self.workspace), _stream()),
                  "moe_align_block_size_mapped")
        return self.sorted_ids[: self.max_padded], self.expert_ids[: self.max_blocks], self.ntpp


def moe_align_block_size(topk_ids: torch.Tensor, block_size: int, num_experts: int,
                         expert_map: torch.Tensor | None = None):
    """vLLM's moe_align_block_size(topk_ids, BM, E, expert_map) as called at
    overlap/overlap_forward.py:165-169 -> (sorted_token_ids, expert_ids,
    num_tokens_post_padded).  Stable order within each expert, pad value S.
    With ``expert_map`` the E global experts are sorted and padded and the
    block expert ids become local ids (-1 for experts not on this device)."""
    bufs = AlignBuffers(topk_ids.numel(), num_experts, block_size, topk_ids.device)
    em = None if expert_map is None else expert_map.to(torch.int32).contiguous()
    return bufs.run(topk_ids.contiguous().view(-1), em)


# ---------------------------------------------------------------------------
# A5 / A8 -- grouped GEMM;  A5+A6+A7 fused
# ---------------------------------------------------------------------------

def dispatch_fused_moe_kernel(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
                              A_scale: torch.Tensor, B_scale: torch.Tensor, B_zp: Any,
                              topk_weights: torch.Tensor | None, sorted_token_ids: torch.Tensor,
                              expert_ids: torch.Tensor, num_tokens_post_padded: torch.Tensor,
                              mul_routed_weight: bool, top_k: int, config: dict | None = None,
                              compute_type: Any = None, use_fp8_w8a8: bool = True,
                              use_int8_w8a8: bool = False, use_int8_w8a16: bool = False,
                              use_int4_w4a16: bool = False, per_channel_quant: bool = False,
                              block_shape: list[int] | None = None, B_bias: Any = None,
                              a_by_pos: bool = False, tile_order: int = 0, tile_m: int = 0) -> None:
    """The reference's grouped-GEMM call (overlap/kernels.py:288-310,
    schemes/shared_expert.py:102-123) on the FP8 w8a8 block-[128,128] form.
    C is [M, top_k, N] or [S, 1, N]; rows are written by slot.  ``tile_order``
    selects the workgroup -> tile order (TILE_ORDERS) and ``tile_m`` the rows
    of a workgroup tile (a multiple of BLOCK_SIZE_M up to 256; 0 = automatic);
    results depend on neither."""
    if not use_fp8_w8a8 or use_int8_w8a8 or use_int8_w8a16 or use_int4_w4a16 or per_channel_quant:
        raise NotImplementedError("only fp8_w8a8 block-scaled GEMM is implemented")
    if B_zp is not None or B_bias is not None:
        raise NotImplementedError("zero points / bias are not on this path")
    if block_shape is not None and list(block_shape) != BLOCK_SHAPE:
        raise NotImplementedError("only block_shape [128,128]")
    if B.dim() != 3:
        raise ValueError(f"B must be [E, N, K], got {tuple(B.shape)}")
    E, N, K = B.shape
    BM = int((config or {}).get("BLOCK_SIZE_M", 0)) or _block_m_from(sorted_token_ids, expert_ids)
    w = None
    if mul_routed_weight:
        if topk_weights is None:
            raise ValueError("mul_routed_weight requires topk_weights")
        w = topk_weights.contiguous().view(-1)
    S = _check_grouped_gemm(A, A_scale, B, B_scale, C, w, sorted_token_ids, expert_ids,
                            num_tokens_post_padded, top_k, a_by_pos, BM, N)
    if A.shape[1] != K:
        raise ValueError(f"A has {A.shape[1]} columns, B has K = {K}")
    check(lib().moe_grouped_gemm_tiled(_ptr(A), _ptr(A_scale), _ptr(B), _ptr(B_scale),
                                       _ptr(sorted_token_ids), _ptr(expert_ids),
                                       _ptr(num_tokens_post_padded), _ptr(w), S, top_k,
                                       1 if a_by_pos else 0, N, K, E, BM, sorted_token_ids.numel(),
                                       int(tile_order), int(tile_m), _ptr(C), _stream()), "moe_grouped_gemm")


def invoke_moe_kernel_n_split(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, A_scale: torch.Tensor,
                              B_scale: torch.Tensor, B_zp: Any, topk_weights: torch.Tensor | None,
                              sorted_token_ids: torch.Tensor, expert_ids: torch.Tensor,
                              num_tokens_post_padded: torch.Tensor, mul_routed_weight: bool, top_k: int,
                              config: dict | None, compute_type: Any = None, use_fp8_w8a8: bool = True,
                              use_int8_w8a8: bool = False, use_int8_w8a16: bool = False,
                              use_int4_w4a16: bool = False, per_channel_quant: bool = False,
                              N_offset: int = 0, N_chunk: int | None = None,
                              block_shape: list[int] | None = None, B_bias: Any = None,
                              a_by_pos: bool = False) -> None:
    """The reference's N-split grouped GEMM (overlap/kernels.py:219-310):
    C[..., N_offset:N_offset+N_chunk] from the matching rows of B and groups
    of B_scale.  C is [M, top_k, full_N] or [S, 1, full_N] (rows by slot)."""
    if not use_fp8_w8a8 or use_int8_w8a8 or use_int8_w8a16 or use_int4_w4a16 or per_channel_quant:
        raise NotImplementedError("only fp8_w8a8 block-scaled GEMM is implemented")
    if B_zp is not None or B_bias is not None:
        raise NotImplementedError("zero points / bias are not on this path")
    if block_shape is not None and list(block_shape) != BLOCK_SHAPE:
        raise NotImplementedError("only block_shape [128,128]")
    if B.dim() != 3:
        raise ValueError(f"B must be [E, N, K], got {tuple(B.shape)}")
    E, full_N, K = B.shape
    N_chunk = full_N - N_offset if N_chunk is None else N_chunk
    BM = int((config or {}).get("BLOCK_SIZE_M", 0)) or _block_m_from(sorted_token_ids, expert_ids)
    if mul_routed_weight and topk_weights is None:
        raise ValueError("mul_routed_weight requires topk_weights")
    w = topk_weights.contiguous().view(-1) if mul_routed_weight else None
    S = _check_grouped_gemm(A, A_scale, B, B_scale, C, w, sorted_token_ids, expert_ids,
                            num_tokens_post_padded, top_k, a_by_pos, BM, full_N)
    if A.shape[1] != K:
        raise ValueError(f"A has {A.shape[1]} columns, B has K = {K}")
    check(lib().moe_grouped_gemm_n_split(_ptr(A), _ptr(A_scale), _ptr(B), _ptr(B_scale), _ptr(sorted_token_ids),
                                         _ptr(expert_ids), _ptr(num_tokens_post_padded), _ptr(w), S, top_k,
                                         1 if a_by_pos else 0, full_N, N_offset, N_chunk, K, E, BM,
                                         sorted_token_ids.numel(), _ptr(C), _stream()), "moe_grouped_gemm_n_split")


def invoke_moe_kernel_k_split(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, A_scale: torch.Tensor,
                              B_scale: torch.Tensor, topk_weights: torch.Tensor | None,
                              sorted_token_ids: torch.Tensor, expert_ids: torch.Tensor,
                              num_tokens_post_padded: torch.Tensor, mul_routed_weight: bool, top_k: int,
                              config: dict | None, compute_type: Any = None, use_fp8_w8a8: bool = True,
                              use_int8_w8a8: bool = False, per_channel_quant: bool = False,
                              K_offset: int = 0, K_chunk: int | None = None, is_first_chunk: bool = True,
                              block_shape: list[int] | None = None, A_K_offset: int = -1,
                              a_by_pos: bool = False) -> None:
    """The reference's K-split accumulate GEMM (overlap/kernels.py:317-452):
    the partial product over A[:, A_K_offset:+K_chunk] and
    B[:, :, K_offset:+K_chunk] is stored into C on the first chunk and added
    to it (bf16) afterwards.  A_K_offset = -1 means K_offset (A and B sliced
    alike); 0 means A already is the K sub-range."""
    if not use_fp8_w8a8 or use_int8_w8a8 or per_channel_quant:
        raise NotImplementedError("only fp8_w8a8 block-scaled GEMM is implemented")
    if block_shape is not None and list(block_shape) != BLOCK_SHAPE:
        raise NotImplementedError("only block_shape [128,128]")
    if B.dim() != 3:
        raise ValueError(f"B must be [E, N, K], got {tuple(B.shape)}")
    E, N, full_K = B.shape
    K_chunk = full_K - K_offset if K_chunk is None else K_chunk
    a_k = K_offset if A_K_offset < 0 else A_K_offset
    BM = int((config or {}).get("BLOCK_SIZE_M", 0)) or _block_m_from(sorted_token_ids, expert_ids)
    if mul_routed_weight and topk_weights is None:
        raise ValueError("mul_routed_weight requires topk_weights")
    w = topk_weights.contiguous().view(-1) if mul_routed_weight else None
    S = _check_grouped_gemm(A, A_scale, B, B_scale, C, w, sorted_token_ids, expert_ids,
                            num_tokens_post_padded, top_k, a_by_pos, BM, N)
    check(lib().moe_grouped_gemm_k_split(_ptr(A), _ptr(A_scale), A.shape[-1], a_k, _ptr(B), _ptr(B_scale),
                                         _ptr(sorted_token_ids), _ptr(expert_ids), _ptr(num_tokens_post_padded),
                                         _ptr(w), S, top_k, 1 if a_by_pos else 0, N, full_K, K_offset, K_chunk,
                                         E, BM, sorted_token_ids.numel(), 1 if is_first_chunk else 0, _ptr(C),
                                         _stream()), "moe_grouped_gemm_k_split")


def _block_m_from(sorted_token_ids: torch.Tensor, expert_ids: torch.Tensor) -> int:
    n, b = sorted_token_ids.numel(), expert_ids.numel()
    for bm in SUPPORTED_BLOCK_M:
        if (n + bm - 1) // bm == b:
            return bm
    raise ValueError("cannot infer BLOCK_SIZE_M; pass config={'BLOCK_SIZE_M': ...}")


def gemm_w13_silu_quant(Aq: torch.Tensor, A_scale: torch.Tensor, w13: torch.Tensor,
                        w13_scale: torch.Tensor, sorted_token_ids: torch.Tensor,
                        expert_ids: torch.Tensor, num_tokens_post_padded: torch.Tensor,
                        num_slots: int, top_k: int, block_size_m: int,
                        hq: torch.Tensor | None = None, hs: torch.Tensor | None = None, tile_m: int = 0,
                        exact_dot: bool = False):
    """W13 GEMM + SiLU*up + 1x128 quant of h, outputs by sorted position:
    (hq [max_padded, I] e4m3fn, hs [max_padded, I/128] fp32).  ``tile_m`` as
    for dispatch_fused_moe_kernel.  ``exact_dot`` takes every 128-element dot
    exactly (the FP8 codes on the bf16 matrix core, about twice the
    matrix-core time) instead of with the FP8 instruction's in-group product
    truncation."""
    E, N2, H = _need_weights(w13, w13_scale, "w13")
    I = N2 // 2
    _need_routing(sorted_token_ids, expert_ids, num_tokens_post_padded, block_size_m)
    if top_k < 1:
        raise ValueError("top_k must be >= 1")
    _need_activations(Aq, A_scale, (num_slots + top_k - 1) // top_k, H)
    max_padded = sorted_token_ids.numel()
    if hq is None:
        hq = torch.empty((max_padded, I), dtype=FP8, device=Aq.device)
    if hs is None:
        hs = torch.empty((max_padded, I // 128), dtype=torch.float32, device=Aq.device)
    _need(hq, "hq", FP8, (max_padded, I))
    _need(hs, "hs", torch.float32, (max_padded, _blocks128(I)))
    if exact_dot:
        check(lib().moe_gemm_w13_silu_quant_exact(_ptr(Aq), _ptr(A_scale), _ptr(w13), _ptr(w13_scale),
                                                  _ptr(sorted_token_ids), _ptr(expert_ids),
                                                  _ptr(num_tokens_post_padded), num_slots, top_k, H, I, E,
                                                  block_size_m, max_padded, int(tile_m), 0, _ptr(hq), _ptr(hs),
                                                  _stream()),
              "moe_gemm_w13_silu_quant_exact")
        return hq, hs
    check(lib().moe_gemm_w13_silu_quant_tiled(_ptr(Aq), _ptr(A_scale), _ptr(w13), _ptr(w13_scale),
                                              _ptr(sorted_token_ids), _ptr(expert_ids),
                                              _ptr(num_tokens_post_padded), num_slots, top_k, H, I, E,
                                              block_size_m, max_padded, int(tile_m), _ptr(hq), _ptr(hs),
                                              _stream()),
          "moe_gemm_w13_silu_quant")
    return hq, hs


def gather_scales_by_position(scales: torch.Tensor, sorted_token_ids: torch.Tensor,
                              num_tokens_post_padded: torch.Tensor, num_slots: int, top_k: int,
                              out: torch.Tensor | None = None) -> torch.Tensor:
    """1x128 activation scales [rows, G] (by token) -> [G, max_padded] K-major by
    sorted position: out[kb, p] = scales[sorted_token_ids[p] // top_k, kb] for the
    positions that hold a slot and scales[0, kb] elsewhere (the row the
    row-major GEMMs read for a padding position).  The layout the position-major
    GEMMs of FusedExpertsRunner read (contiguous per K block and tile); it has
    no counterpart in the reference."""
    if scales.dim() != 2:
        raise ValueError(f"scales must be [rows, groups], got {tuple(scales.shape)}")
    if top_k < 1:
        raise ValueError("top_k must be >= 1")
    _need(scales, "scales", torch.float32)
    _need(sorted_token_ids, "sorted_token_ids", torch.int32)
    _need(num_tokens_post_padded, "num_tokens_post_padded", torch.int32)
    rows, G = scales.shape
    mp = sorted_token_ids.numel()
    if out is None:
        out = torch.empty((G, mp), dtype=torch.float32, device=scales.device)
    _need(out, "out", torch.float32, (G, mp))
    check(lib().moe_gather_scales_by_position(_ptr(scales), rows, G, _ptr(sorted_token_ids),
                                              _ptr(num_tokens_post_padded), num_slots, top_k, mp, _ptr(out),
                                              _stream()), "moe_gather_scales_by_position")
    return out


# ---------------------------------------------------------------------------
# A6 / A9
# ---------------------------------------------------------------------------

def silu_and_mul(out: torch.Tensor, x: torch.Tensor) -> None:
    """torch.ops._C.silu_and_mul(out, x): out[r,j] = silu(x[r,j]) * x[r,I+j]
    (overlap/overlap_forward.py:277-279)."""
    _need(x, "x", torch.bfloat16)
    R = x.numel() // x.shape[-1]
    I = x.shape[-1] // 2
    _need(out, "out", torch.bfloat16, tuple(x.shape[:-1]) + (I,))
    check(lib().moe_silu_and_mul(_ptr(x), R, I, _ptr(out), _stream()), "moe_silu_and_mul")


def silu_mul_quant_group128(x: torch.Tensor, out_q: torch.Tensor | None = None,
                            out_s: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """x [R, 2I] bf16 (gate | up) -> FP8 1x128 quant of bf16(silu(gate)*up):
    (q [R, I] e4m3fn, scales [R, I/128]).  One pass of silu_and_mul followed by
    moe_kernel_quantize_input (overlap/overlap_forward.py:277-284)."""
    _need(x, "x", torch.bfloat16)
    R = x.numel() // x.shape[-1]
    I = x.shape[-1] // 2
    q = torch.empty((R, I), dtype=FP8, device=x.device) if out_q is None else out_q
    s = torch.empty((R, I // 128), dtype=torch.float32, device=x.device) if out_s is None else out_s
    _need(q, "out_q", FP8, (R, I))
    _need(s, "out_s", torch.float32, (R, I // 128))
    check(lib().moe_silu_mul_quant_group128(_ptr(x), R, I, _ptr(q), _ptr(s), _stream()),
          "moe_silu_mul_quant_group128")
    return q, s


def moe_sum(D: torch.Tensor, out: torch.Tensor, top_k: int,
            addend: torch.Tensor | None = None) -> torch.Tensor:
    """out[t] = sum_i D[t*k+i] (fp32 accumulation, bf16 result), the reference's
    torch.sum(C_down.view(T,k,H), dim=1) (overlap/overlap_forward.py:304-313).
    With ``addend`` ([T, H] bf16, the shared expert's output) the bf16 sum is
    added to it in the same pass, as ``result + shared(hidden)`` does
    (schemes/vllm_tp.py:62-63)."""
    if out.dim() != 2:
        raise ValueError(f"out must be [T, H], got {tuple(out.shape)}")
    T, H = out.shape
    if D.numel() != T * top_k * H:
        raise ValueError(f"D has {D.numel()} elements, [T*top_k, H] = [{T * top_k}, {H}] needs {T * top_k * H}")
    _need(D, "D", torch.bfloat16)
    _need(out, "out", torch.bfloat16)
    if addend is None:
        check(lib().moe_reduce_topk(_ptr(D), T, top_k, H, _ptr(out), _stream()), "moe_reduce_topk")
    else:
        _need(addend, "addend", torch.bfloat16)
        if tuple(addend.shape) != (T, H):
            raise ValueError(f"addend must be [{T}, {H}]")
        check(lib().moe_reduce_topk_add(_ptr(D), _ptr(addend), T, top_k, H, _ptr(out), _stream()),
              "moe_reduce_topk_add")
    return out


def fp8_dequant_sum(recv_q: torch.Tensor, recv_s: torch.Tensor,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """The combine of the FP8-compressed reduce-scatter leg
    (overlap/overlap_forward.py:932-944): the R ranks' FP8 chunks of this
    rank's M rows, recv_q [R, M, N] e4m3fn, with their 1x128 scales recv_s
    ([R, M, G] or [R*M, G] fp32, G >= ceil(N/128); a column slice of a wider
    buffer is read in place) ->
    out [M, N] bf16 = sum over ranks of float(q) * scale (fp32 products, fp32
    sum over ascending rank, one bf16 rounding).  ``out`` may be a column
    slice of a wider [M, *] tensor (the reference's torch.cat of the chunk
    outputs, :946, then needs no copy).  The senders quantise with
    per_token_group_quant_fp8 (:900-905)."""
    if recv_q.dim() != 3:
        raise ValueError(f"recv_q must be [R, M, N], got {tuple(recv_q.shape)}")
    R, M, N = recv_q.shape
    groups = _blocks128(N)
    if recv_s.dim() == 3:
        if tuple(recv_s.shape[:2]) != (R, M) or recv_s.shape[2] < groups:
            raise ValueError(f"recv_s must be [{R}, {M}, >= {groups}], got {tuple(recv_s.shape)}")
        if recv_s.stride(2) != 1 or recv_s.stride(0) != M * recv_s.stride(1):
            raise ValueError("recv_s rows must be evenly strided with unit column stride")
        scale_ld = recv_s.stride(1)
    elif recv_s.dim() == 2:
        if recv_s.shape[0] != R * M or recv_s.shape[1] < groups:
            raise ValueError(f"recv_s must be [{R * M}, >= {groups}], got {tuple(recv_s.shape)}")
        if recv_s.stride(1) != 1:
            raise ValueError("recv_s must have unit column stride")
        scale_ld = recv_s.stride(0)
    else:
        raise ValueError(f"recv_s must be 2-D or 3-D, got {tuple(recv_s.shape)}")
    if recv_s.dtype != torch.float32:
        raise TypeError(f"recv_s must be torch.float32, got {recv_s.dtype}")
    if not recv_s.is_cuda:
        raise ValueError("recv_s must be a GPU tensor")
    _need(recv_q, "recv_q", FP8)
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=recv_q.device)
    if out.dtype != torch.bfloat16:
        raise TypeError(f"out must be torch.bfloat16, got {out.dtype}")
    if tuple(out.shape) != (M, N) or out.stride(1) != 1:
        raise ValueError(f"out must be [{M}, {N}] with unit column stride, got {tuple(out.shape)}")
    if not out.is_cuda:
        raise ValueError("out must be a GPU tensor")
    check(lib().moe_fp8_dequant_sum(_ptr(recv_q), _ptr(recv_s), R, M, N, scale_ld, _ptr(out),
                                    out.stride(0) if M > 1 else N, _stream()), "moe_fp8_dequant_sum")
    return out


# ---------------------------------------------------------------------------
# A4 -- tile configuration
# ---------------------------------------------------------------------------

def gemm_tile_rows(block_size_m: int, num_slots: int, num_experts: int, tile_m: int = 0) -> int:
    """Rows of the grouped GEMM's workgroup tile for this launch: ``tile_m`` if
    given, else 256 when the experts average at least 160 slots and
    ``block_size_m`` otherwise (the rule of the C entry points)."""
    if tile_m:
        return int(tile_m)
    return 256 if num_slots >= 160 * num_experts else int(block_size_m)


def get_moe_config(num_tokens: int, num_experts: int, top_k: int) -> dict[str, int]:
    """Replacement for vLLM's try_get_optimal_moe_config (overlap_forward.py:
    153-163): picks BLOCK_SIZE_M from the average rows per expert, avg =
    num_tokens * top_k / num_experts, by a sweep of the whole layer over
    block sizes 16-256 on MI355X (four expert shapes: H/I/E/top-k of
    DeepSeek-V3, Mixtral, Qwen3-30B-A3B and the reference's v1 GroupGEMM
    sweep, 4-1024 rows per expert):

    * avg <= 28: 32.  The layer streams its weights; the 32-row tile streams
      them faster than the 16-row one and wastes less than taller blocks.
    * avg <= 44: 64.  Most experts now fill a 32-row block and spill into a
      second one; 64-row blocks keep them in one tile (40 rows per expert:
      DeepSeek-V3 2151 us against 2588 at 32, Mixtral 336 against 402,
      Qwen3 161 against 176, v1 186 against 198; within 2 % of the best
      block size on all four shapes at 32 and 40 rows).
    * avg <= 100: 128.  Most experts fit one block; a 128-row tile reads
      fewer LDS bytes per MFMA than a 64-row one (v1 shape, 64 rows per
      expert: 195 us against 209 at 64; DeepSeek-V3: 2208 against 2606).
    * above: 256, so that an expert's rows stay in one tile instead of
      spilling a few rows into a second one (128 rows per expert: 237 against
      244 us at 128; Qwen3 at 160: 241 against 299) -- except when the average
      sits at 240-288 rows, where half the experts would spill a few rows into
      a second 256-row block and 128-row blocks split them evenly over two
      256-row tiles instead (DeepSeek-V3 at 256: 3920 against 4058 us)."""
    avg = num_tokens * top_k / max(num_experts, 1)
    if avg <= 28:
        bm = 32
    elif avg <= 44:
        bm = 64
    elif avg <= 100:
        bm = 128
    elif 240 <= avg <= 288:
        bm = 128
    else:
        bm = 256
    return {"BLOCK_SIZE_M": bm, "BLOCK_SIZE_N": 256, "BLOCK_SIZE_K": 128}


# ---------------------------------------------------------------------------
# A10 -- the whole layer
# ---------------------------------------------------------------------------

class SharedExpertRunner:
    """The shared expert (E = 1, top-1) through the same kernels, with every
    buffer and the align outputs built once (schemes/shared_expert.py:15-148).

    ``__call__(x, input_scale=None)``: a bf16 ``x`` [rows, H] is quantised
    1x128 first; an FP8 ``x`` is used directly with its [rows, H/128]
    ``input_scale`` -- no dequantise/requantise round trip
    (shared_expert.py:3-7, 83-93).  Returns a [rows, H] bf16 view of an
    internal buffer (valid until the next call).

    An H that is not a multiple of 128 runs at the padded width Hp =
    ceil(H/128)*128: the weights get zero codes in the padding when the
    runner is built, a bf16 ``x`` is quantised into zero-padded rows, and an
    FP8 ``x`` must come in that padded layout ([rows, Hp], as
    FusedExpertsRunner's own q1).  ``out`` then holds [max_tokens, Hp] rows
    and the call returns their first H columns.

    Every buffer is allocated when the runner is built (the builder-allocates
    contract of schemes/base.py:45-93): the align outputs exist for
    ``max_tokens`` rows and for each count in ``row_counts``, or added later
    with ``prepare(rows)``; a call with any other row count raises instead of
    allocating.

    ``exact_dot`` selects the exact-dot W13 (as FusedExpertsRunner's; a
    layer runner with a shared expert sets it to its own mode on every run)."""

    def __init__(self, w1: torch.Tensor, w1_scale: torch.Tensor, w2: torch.Tensor,
                 w2_scale: torch.Tensor, max_tokens: int, block_size_m: int | None = None,
                 row_counts: tuple[int, ...] = (), exact_dot: bool = False):
        E1, N2, H = _need_weights(w1, w1_scale, "w1")
        _need_weights(w2, w2_scale, "w2")
        if E1 != 1 or w2.shape[0] != 1:
            raise ValueError("the shared expert has exactly one expert")
        if w2.shape != (1, H, N2 // 2):
            raise ValueError(f"w2 shape {tuple(w2.shape)} does not match w1 {tuple(w1.shape)}")
        if (N2 // 2) % 128:
            raise ValueError(f"the intermediate size {N2 // 2} must be a multiple of 128")
        self.H, self.I, self.max_tokens = H, N2 // 2, max_tokens
        self.exact_dot = bool(exact_dot)
        self.Hp = _blocks128(H) * 128
        w1, w2 = _pad_fp8(w1, 2, self.Hp), _pad_fp8(w2, 1, self.Hp)
        self.w1, self.w1_scale, self.w2, self.w2_scale = w1, w1_scale, w2, w2_scale
        self.BM = block_size_m or get_moe_config(max_tokens, 1, 1)["BLOCK_SIZE_M"]
        dev = w1.device
        self._aligns: dict[int, AlignBuffers] = {}
        for rows in (max_tokens, *row_counts):
            self.prepare(rows)
        mp = self._aligns[max_tokens].max_padded
        self.q = torch.empty((max_tokens, self.Hp), dtype=FP8, device=dev)
        self.s = torch.empty((max_tokens, self.Hp // 128), dtype=torch.float32, device=dev)
        self.hq = torch.empty((mp, self.I), dtype=FP8, device=dev)
        self.hs = torch.empty((mp, self.I // 128), dtype=torch.float32, device=dev)
        self.out = torch.empty((max_tokens, self.Hp), dtype=torch.bfloat16, device=dev)

    def prepare(self, rows: int) -> None:
        """Build the align outputs for calls with ``rows`` tokens, all routed
        to expert 0 (build time: this allocates and launches the align)."""
        if rows > self.max_tokens:
            raise ValueError(f"{rows} rows exceed max_tokens={self.max_tokens}")
        if rows not in self._aligns:
            a = AlignBuffers(rows, 1, self.BM, self.w1.device)
            a.run(torch.zeros(rows, dtype=torch.int32, device=self.w1.device))
            self._aligns[rows] = a

    def _align_for(self, rows: int) -> AlignBuffers:
        a = self._aligns.get(rows)
        if a is None:
            raise ValueError(f"no align outputs prepared for {rows} rows (prepared: {sorted(self._aligns)}); "
                             "call prepare(rows) when building the runner")
        return a

    def __call__(self, x: torch.Tensor, input_scale: torch.Tensor | None = None) -> torch.Tensor:
        rows = x.shape[0]
        if rows > self.max_tokens:
            raise ValueError(f"{rows} rows exceed max_tokens={self.max_tokens}")
        if x.dtype == FP8:
            if input_scale is None:
                raise ValueError("FP8 shared expert input requires input_scale")
            if input_scale.shape[0] != rows:
                raise ValueError(f"input_scale rows {input_scale.shape[0]} do not match input rows {rows}")
            q, s = x, input_scale
        else:
            _need(x, "x", torch.bfloat16)
            if tuple(x.shape) != (rows, self.H):
                raise ValueError(f"x must be [rows, {self.H}], got {tuple(x.shape)}")
            q, s = self.q[:rows], self.s[:rows]
            check(lib().moe_quant_group128_padded(_ptr(x), rows, self.H, _ptr(q), self.Hp, _ptr(s), _stream()),
                  "moe_quant_group128_padded")
        _need(q, "x", FP8, (rows, self.Hp))
        _need(s, "input_scale", torch.float32, (rows, self.Hp // 128))
        a = self._align_for(rows)
        if self.exact_dot:
            check(lib().moe_gemm_w13_silu_quant_exact(_ptr(q), _ptr(s), _ptr(self.w1), _ptr(self.w1_scale),
                                                      _ptr(a.sorted_ids), _ptr(a.expert_ids), _ptr(a.ntpp), rows, 1,
                                                      self.Hp, self.I, 1, self.BM, a.max_padded, 0, 0,
                                                      _ptr(self.hq), _ptr(self.hs), _stream()),
                  "moe_gemm_w13_silu_quant_exact")
        else:
            check(lib().moe_gemm_w13_silu_quant(_ptr(q), _ptr(s), _ptr(self.w1), _ptr(self.w1_scale),
                                                _ptr(a.sorted_ids), _ptr(a.expert_ids), _ptr(a.ntpp), rows, 1,
                                                self.Hp, self.I, 1, self.BM, a.max_padded, _ptr(self.hq),
                                                _ptr(self.hs), _stream()), "moe_gemm_w13_silu_quant")
        out = self.out[:rows]
        check(lib().moe_grouped_gemm(_ptr(self.hq), _ptr(self.hs), _ptr(self.w2), _ptr(self.w2_scale),
                                     _ptr(a.sorted_ids), _ptr(a.expert_ids), _ptr(a.ntpp), None, rows, 1, 1,
                                     self.Hp, self.I, 1, self.BM, a.max_padded, _ptr(out), _stream()),
              "moe_grouped_gemm")
        return out[:, : self.H]


class FusedExpertsRunner:
    """Prebuilt A1->A9 chain for fixed (T, H, I, E, top_k, BM).

    Construction allocates every buffer; ``run`` only enqueues kernels
    (quant -> align -> [scale gather] -> W13+SiLU+quant -> W2 with routed
    weights -> [shared expert on the same FP8 input] -> top-k sum) on the
    current stream
    and returns the [T, H] bf16 output (``out`` if one was given).

    With ``scales_by_position`` (by default when the GEMM tiles have 128 or
    more rows, where a step's scales are worth a contiguous load) the
    activation scales travel K-major by sorted position between the kernels: the W13 stage first
    gathers the 1x128 scales into that layout, and the fused W13 writes its
    output scales in it for W2, so each GEMM step reads its tile's scales as
    one contiguous run.  Results are bit-identical to the row-major path.
    ``hs`` is then a [max_padded, I/128] view of the K-major buffer.  Run one
    stage at a time with ``stage_quant``, ``stage_align``, ``stage_scales``,
    ``stage_w13``, ``stage_w2``, ``stage_shared``, ``stage_reduce``, in that
    order.

    A hidden size H that is not a multiple of 128 runs at the padded width
    Hp = ceil(H/128)*128, which is what the reference's quant does to the
    activations (verify.py:111-113) and its weight quant to a ragged block
    (data/checkpoint.py:28-40): the weights get zero codes in the padding
    once, when the runner is built; the activations are quantised into
    zero-padded rows; W2 writes Hp columns, and the top-k sum's first H
    columns are the output.  The zero codes add nothing to any product, so
    the results are those of the unpadded computation.  The intermediate
    size I must be a multiple of 128 (the fused SiLU*up pairs whole gate and
    up groups).

    ``exact_dot`` (also settable on the runner between runs) makes the W13
    stage take every 128-element dot exactly: the FP8 codes converted to bf16
    on the bf16 matrix core, about twice the matrix-core time of the FP8
    instruction, whose in-group product truncation otherwise moves about
    0.2 % of the intermediate codes.  W2 and every other stage are the same
    in both modes, and a shared expert follows the layer's mode."""

    def __init__(self, w13: torch.Tensor, w13_scale: torch.Tensor, w2: torch.Tensor,
                 w2_scale: torch.Tensor, num_tokens: int, top_k: int, block_size_m: int | None = None,
                 shared: SharedExpertRunner | None = None, out: torch.Tensor | None = None,
                 global_num_experts: int | None = None, expert_map: torch.Tensor | None = None,
                 tile_m: int = 0, scales_by_position: bool | None = None, exact_dot: bool = False):
        E, N2, H = _need_weights(w13, w13_scale, "w13")
        _need_weights(w2, w2_scale, "w2")
        if w2.shape != (E, H, N2 // 2):
            raise ValueError(f"w2 shape {tuple(w2.shape)} does not match w13 {tuple(w13.shape)}")
        if (N2 // 2) % 128:
            raise ValueError(f"the intermediate size {N2 // 2} must be a multiple of 128")
        self.E, self.H, self.I, self.T, self.top_k = E, H, N2 // 2, num_tokens, top_k
        self.exact_dot = bool(exact_dot)
        self.Hp = Hp = _blocks128(H) * 128
        w13, w2 = _pad_fp8(w13, 2, Hp), _pad_fp8(w2, 1, Hp)
        self.S = num_tokens * top_k
        self.BM = block_size_m or get_moe_config(num_tokens, E, top_k)["BLOCK_SIZE_M"]
        if self.BM not in SUPPORTED_BLOCK_M:
            raise ValueError(f"block_size_m must be one of {SUPPORTED_BLOCK_M}")
        # GEMM workgroup tile rows (0 = automatic; never changes the results)
        self.tile_m = int(tile_m)
        if self.tile_m and (self.tile_m not in SUPPORTED_BLOCK_M or self.tile_m % self.BM):
            raise ValueError(f"tile_m must be a multiple of block_size_m in {SUPPORTED_BLOCK_M}")
        if shared is not None and (shared.H != H or shared.max_tokens < num_tokens):
            raise ValueError("shared expert does not match the layer's hidden size / token count")
        if shared is not None:
            shared.prepare(num_tokens)
        self.w13, self.w13_scale, self.w2, self.w2_scale = w13, w13_scale, w2, w2_scale
        self.shared = shared
        self.shared_out: torch.Tensor | None = None
        dev = w13.device
        self.q1 = torch.empty((self.T, Hp), dtype=FP8, device=dev)
        self.s1 = torch.empty((self.T, Hp // 128), dtype=torch.float32, device=dev)
        # Expert parallelism: align over the global experts, GEMMs over the
        # local ones (blocks of non-local experts are -1 and produce zeros).
        self.expert_map = None
        n_align = E
        if expert_map is not None:
            self.expert_map = expert_map.to(device=dev, dtype=torch.int32).contiguous()
            n_align = int(global_num_experts or self.expert_map.numel())
            if self.expert_map.numel() != n_align:
                raise ValueError("expert_map must have global_num_experts entries")
        elif global_num_experts not in (None, -1, E):
            raise ValueError("global_num_experts != local experts needs an expert_map")
        self.align = AlignBuffers(self.S, n_align, self.BM, dev)
        mp = max(self.align.max_padded, 1)
        self.hq = torch.empty((mp, self.I), dtype=FP8, device=dev)
        if scales_by_position is None:
            scales_by_position = gemm_tile_rows(self.BM, self.S, self.E, self.tile_m) >= 128
        self.scales_by_position = bool(scales_by_position)
        if self.scales_by_position:
            self.s1_pos = torch.empty((Hp // 128, mp), dtype=torch.float32, device=dev)
            self.hs_pos = torch.empty((self.I // 128, mp), dtype=torch.float32, device=dev)
            self.hs = self.hs_pos.t()  # [mp, I/128] view by position
        else:
            self.hs = torch.empty((mp, self.I // 128), dtype=torch.float32, device=dev)
        self.D = torch.empty((max(self.S, 1), Hp), dtype=torch.bfloat16, device=dev)
        if out is not None:
            _need(out, "out", torch.bfloat16)
            if tuple(out.shape) != (self.T, H):
                raise ValueError(f"out must be [{self.T}, {H}]")
        self.y = out if out is not None else torch.empty((self.T, H), dtype=torch.bfloat16, device=dev)
        # the top-k sum at the padded width, whose first H columns are y
        self.y_pad = self.y if Hp == H else torch.empty((self.T, Hp), dtype=torch.bfloat16, device=dev)

    def stage_quant(self, hidden: torch.Tensor) -> None:
        _need(hidden, "hidden_states", torch.bfloat16)
        if tuple(hidden.shape) != (self.T, self.H):
            raise ValueError(f"hidden_states must be [{self.T}, {self.H}]")
        if self.Hp == self.H:
            check(lib().moe_quant_group128(_ptr(hidden), self.T, self.H, _ptr(self.q1), _ptr(self.s1),
                                           _stream()), "moe_quant_group128")
        else:
            check(lib().moe_quant_group128_padded(_ptr(hidden), self.T, self.H, _ptr(self.q1), self.Hp,
                                                  _ptr(self.s1), _stream()), "moe_quant_group128_padded")

    def stage_align(self, topk_ids: torch.Tensor) -> None:
        self.align.run(topk_ids, self.expert_map)

    def stage_scales(self) -> None:
        """The activation scales K-major by sorted position for the W13 GEMM
        (nothing to do on the row-major path)."""
        if self.scales_by_position:
            a = self.align
            check(lib().moe_gather_scales_by_position(_ptr(self.s1), self.T, self.Hp // 128, _ptr(a.sorted_ids),
                                                      _ptr(a.ntpp), self.S, self.top_k, a.max_padded,
                                                      _ptr(self.s1_pos), _stream()), "moe_gather_scales_by_position")

    def stage_w13(self) -> None:
        a = self.align
        if self.exact_dot:
            by_pos = self.scales_by_position
            check(lib().moe_gemm_w13_silu_quant_exact(_ptr(self.q1), _ptr(self.s1_pos if by_pos else self.s1),
                                                      _ptr(self.w13), _ptr(self.w13_scale), _ptr(a.sorted_ids),
                                                      _ptr(a.expert_ids), _ptr(a.ntpp), self.S, self.top_k,
                                                      self.Hp, self.I, self.E, self.BM, a.max_padded, self.tile_m,
                                                      int(by_pos), _ptr(self.hq),
                                                      _ptr(self.hs_pos if by_pos else self.hs), _stream()),
                  "moe_gemm_w13_silu_quant_exact")
            return
        if self.scales_by_position:
            check(lib().moe_gemm_w13_silu_quant_pos(_ptr(self.q1), _ptr(self.s1_pos), _ptr(self.w13),
                                                    _ptr(self.w13_scale), _ptr(a.sorted_ids), _ptr(a.expert_ids),
                                                    _ptr(a.ntpp), self.S, self.top_k, self.Hp, self.I, self.E,
                                                    self.BM, a.max_padded, self.tile_m, _ptr(self.hq),
                                                    _ptr(self.hs_pos), _stream()), "moe_gemm_w13_silu_quant_pos")
            return
        check(lib().moe_gemm_w13_silu_quant_tiled(_ptr(self.q1), _ptr(self.s1), _ptr(self.w13),
                                                  _ptr(self.w13_scale), _ptr(a.sorted_ids), _ptr(a.expert_ids),
                                                  _ptr(a.ntpp), self.S, self.top_k, self.Hp, self.I, self.E,
                                                  self.BM, a.max_padded, self.tile_m, _ptr(self.hq),
                                                  _ptr(self.hs), _stream()), "moe_gemm_w13_silu_quant")

    def stage_w2(self, topk_weights: torch.Tensor) -> None:
        _need(topk_weights, "topk_weights", torch.float32)
        if topk_weights.numel() != self.S:
            raise ValueError(f"topk_weights has {topk_weights.numel()} entries for {self.S} slots")
        a = self.align
        if self.scales_by_position:
            check(lib().moe_grouped_gemm_pos(_ptr(self.hq), _ptr(self.hs_pos), _ptr(self.w2), _ptr(self.w2_scale),
                                             _ptr(a.sorted_ids), _ptr(a.expert_ids), _ptr(a.ntpp),
                                             _ptr(topk_weights), self.S, self.Hp, self.I, self.E, self.BM,
                                             a.max_padded, self.tile_m, _ptr(self.D), _stream()),
                  "moe_grouped_gemm_pos")
            return
        check(lib().moe_grouped_gemm_tiled(_ptr(self.hq), _ptr(self.hs), _ptr(self.w2), _ptr(self.w2_scale),
                                           _ptr(a.sorted_ids), _ptr(a.expert_ids), _ptr(a.ntpp),
                                           _ptr(topk_weights), self.S, 1, 1, self.Hp, self.I, self.E, self.BM,
                                           a.max_padded, 0, self.tile_m, _ptr(self.D), _stream()),
              "moe_grouped_gemm")

    def stage_shared(self) -> None:
        """The shared expert on the layer's own FP8 input (no second quant),
        in the layer's W13 mode."""
        if self.shared is not None:
            self.shared.exact_dot = self.exact_dot
            self.shared_out = self.shared(self.q1, self.s1)

    def stage_reduce(self) -> None:
        addend = None
        if self.shared is not None:  # the shared expert's rows at the padded width
            addend = self.shared.out[: self.T] if self.Hp != self.H else self.shared_out
        moe_sum(self.D[: self.S], self.y_pad, self.top_k, addend=addend)
        if self.y_pad is not self.y:
            self.y.copy_(self.y_pad[:, : self.H])

    def run(self, hidden: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor) -> torch.Tensor:
        self.stage_quant(hidden)
        self.stage_align(topk_ids)
        self.stage_scales()
        self.stage_w13()
        self.stage_w2(topk_weights)
        self.stage_shared()
        self.stage_reduce()
        return self.y

    def capture(self, hidden: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor) -> "LayerGraph":
        """Record the layer's launches once into a HIP graph bound to these
        input tensors; ``LayerGraph.replay()`` then re-runs the whole layer
        with one launch (new inputs go into the same tensors).  The layer's
        kernels take every size from their arguments and clear nothing with a
        memset, so a replay equals an eager run."""
        return LayerGraph(self, hidden, topk_weights, topk_ids)


class LayerGraph:
    """A captured FusedExpertsRunner.run (see FusedExpertsRunner.capture)."""

    def __init__(self, runner: "FusedExpertsRunner", hidden: torch.Tensor, topk_weights: torch.Tensor,
                 topk_ids: torch.Tensor):
        self.runner, self.inputs = runner, (hidden, topk_weights, topk_ids)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            runner.run(*self.inputs)  # first calls set kernel attributes outside the capture
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            runner.run(*self.inputs)

    def replay(self) -> torch.Tensor:
        self.graph.replay()
        return self.runner.y


class ChunkedExpertsRunner:
    """The layer over ``n_chunks`` token chunks pipelined on ``n_streams`` HIP
    streams of one device (the chunked quant/align/GEMM overlap of
    overlap/overlap_forward.py:252-321, single-GPU form).  Chunk c runs its
    whole chain on stream c mod n_streams; the streams start after the caller's
    stream and the caller's stream waits for all of them before ``run``
    returns (overlap_forward.py:336-342).  Each chunk writes its rows of the
    shared [T, H] output directly."""

    def __init__(self, w13: torch.Tensor, w13_scale: torch.Tensor, w2: torch.Tensor,
                 w2_scale: torch.Tensor, num_tokens: int, top_k: int, n_chunks: int, n_streams: int,
                 block_size_m: int | None = None, shared_weights: tuple | None = None):
        if n_chunks < 1 or n_streams < 1:
            raise ValueError("n_chunks and n_streams must be >= 1")
        n_chunks = min(n_chunks, num_tokens) if num_tokens > 0 else 1
        self.T, self.top_k, self.H = num_tokens, top_k, w13.shape[2]
        self.y = torch.empty((num_tokens, self.H), dtype=torch.bfloat16, device=w13.device)
        bounds = [num_tokens * c // n_chunks for c in range(n_chunks + 1)]
        self.bounds = list(zip(bounds[:-1], bounds[1:]))
        # one shared-expert runner per chunk (weights shared, buffers per chunk)
        self.runners = [FusedExpertsRunner(w13, w13_scale, w2, w2_scale, r1 - r0, top_k, block_size_m,
                                           shared=(SharedExpertRunner(*shared_weights, max_tokens=r1 - r0)
                                                   if shared_weights is not None else None),
                                           out=self.y[r0:r1]) for r0, r1 in self.bounds]
        # default-priority streams
        self.streams = [torch.cuda.Stream(device=w13.device) for _ in range(min(n_streams, n_chunks))]

    def run(self, hidden: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor) -> torch.Tensor:
        caller = torch.cuda.current_stream()
        start = torch.cuda.Event()
        start.record(caller)
        for st in self.streams:
            st.wait_event(start)
        k = self.top_k
        w, ids = topk_weights.reshape(-1), topk_ids.reshape(-1)
        for c, ((r0, r1), runner) in enumerate(zip(self.bounds, self.runners)):
            with torch.cuda.stream(self.streams[c % len(self.streams)]):
                runner.run(hidden[r0:r1], w[r0 * k:r1 * k], ids[r0 * k:r1 * k])
        for st in self.streams:
            done = torch.cuda.Event()
            done.record(st)
            caller.wait_event(done)
        return self.y


def _split_bounds(total: int, n: int) -> list[tuple[int, int]]:
    """``total`` (a multiple of 128) in ``n`` chunks of whole 128-blocks, as
    even as possible (the first chunks take the extra blocks)."""
    blocks = total // 128
    n = max(1, min(n, blocks))
    sizes = [blocks // n + (1 if c < blocks % n else 0) for c in range(n)]
    out, k = [], 0
    for b in sizes:
        out.append((k * 128, (k + b) * 128))
        k += b
    return out


class SplitExpertsRunner:
    """The reference pipeline's compute-stream structure on one device
    (overlap/overlap_forward.py:252-313 without its all-gather and
    reduce-scatter legs): W13 as ``n_chunks_gateup`` K-split GEMMs
    accumulating into a bf16 C13 (``invoke_moe_kernel_k_split``,
    overlap_forward.py:264-274), ``silu_and_mul`` (:277-279), the 1x128 quant
    of h (:282-284), W2 as ``n_chunks_down`` N-split GEMMs with routed weights
    (``invoke_moe_kernel_n_split``, :289-302) and the top-k sum (:304-313).
    Each weight slice is read once; SiLU*up and the quant cannot be fused into
    a K-split W13, so C13 [S, 2I] and h [S, I] exist in bf16, and every K
    chunk after the first re-reads and re-writes C13.

    The activation quant runs once over [T, H]: 1x128 groups never straddle a
    128-aligned chunk, so the codes and scales equal those of quantising each
    K chunk separately (the reference quantises each all-gathered chunk).
    With ``shared`` the shared expert runs on the layer's own FP8 input and
    its output is added to the top-k sum, bf16(bf16(sum) + shared), as the
    reference adds it to each reduced chunk (overlap_forward.py:238-245,
    315-320); the reduce runs once over all columns (the per-chunk reduce of
    the reference exists to feed each chunk's reduce-scatter).
    Every buffer is allocated here; ``run`` only launches."""

    def __init__(self, w13: torch.Tensor, w13_scale: torch.Tensor, w2: torch.Tensor,
                 w2_scale: torch.Tensor, num_tokens: int, top_k: int, n_chunks_gateup: int = 4,
                 n_chunks_down: int = 4, block_size_m: int | None = None,
                 shared: SharedExpertRunner | None = None):
        E, N2, H = _need_weights(w13, w13_scale, "w13")
        _need_weights(w2, w2_scale, "w2")
        if w2.shape != (E, H, N2 // 2):
            raise ValueError(f"w2 shape {tuple(w2.shape)} does not match w13 {tuple(w13.shape)}")
        self.E, self.H, self.I, self.T, self.top_k = E, H, N2 // 2, num_tokens, top_k
        self.S = num_tokens * top_k
        self.BM = block_size_m or get_moe_config(num_tokens, E, top_k)["BLOCK_SIZE_M"]
        if self.BM not in SUPPORTED_BLOCK_M:
            raise ValueError(f"block_size_m must be one of {SUPPORTED_BLOCK_M}")
        if H % 128 or self.I % 128:
            raise ValueError("the K/N-split runner cuts H into whole 128-column blocks: H and the intermediate "
                             "size must be multiples of 128 (FusedExpertsRunner pads other widths)")
        self.k_bounds = _split_bounds(H, n_chunks_gateup)
        self.n_bounds = _split_bounds(H, n_chunks_down)
        if shared is not None and (shared.H != H or shared.max_tokens < num_tokens):
            raise ValueError("shared expert does not match the layer's hidden size / token count")
        if shared is not None:
            shared.prepare(num_tokens)
        self.shared = shared
        self.shared_out: torch.Tensor | None = None
        self.w13, self.w13_scale, self.w2, self.w2_scale = w13, w13_scale, w2, w2_scale
        dev = w13.device
        S1 = max(self.S, 1)
        self.q1 = torch.empty((self.T, H), dtype=FP8, device=dev)
        self.s1 = torch.empty((self.T, H // 128), dtype=torch.float32, device=dev)
        self.align = AlignBuffers(self.S, E, self.BM, dev)
        self.C13 = torch.empty((S1, N2), dtype=torch.bfloat16, device=dev)
        self.h = torch.empty((S1, self.I), dtype=torch.bfloat16, device=dev)
        self.hq = torch.empty((S1, self.I), dtype=FP8, device=dev)
        self.hs = torch.empty((S1, self.I // 128), dtype=torch.float32, device=dev)
        self.D = torch.empty((S1, H), dtype=torch.bfloat16, device=dev)
        self.y = torch.empty((self.T, H), dtype=torch.bfloat16, device=dev)
        self.config = {"BLOCK_SIZE_M": self.BM}

    def run(self, hidden: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor) -> torch.Tensor:
        _need(hidden, "hidden_states", torch.bfloat16)
        if tuple(hidden.shape) != (self.T, self.H):
            raise ValueError(f"hidden_states must be [{self.T}, {self.H}]")
        if self.S == 0:
            return self.y  # no tokens: [0, H]
        per_token_group_quant_fp8(hidden, out_q=self.q1, out_s=self.s1)
        sorted_ids, eids, ntpp = self.align.run(topk_ids.reshape(-1))
        if self.shared is not None:
            self.shared_out = self.shared(self.q1, self.s1)
        for c, (k0, k1) in enumerate(self.k_bounds):
            invoke_moe_kernel_k_split(self.q1, self.w13, self.C13, self.s1, self.w13_scale, None, sorted_ids, eids,
                                      ntpp, False, self.top_k, self.config, K_offset=k0, K_chunk=k1 - k0,
                                      is_first_chunk=(c == 0))
        silu_and_mul(self.h, self.C13)
        per_token_group_quant_fp8(self.h, out_q=self.hq, out_s=self.hs)
        w = topk_weights.reshape(-1)
        for n0, n1 in self.n_bounds:
            invoke_moe_kernel_n_split(self.hq, self.w2, self.D, self.hs, self.w2_scale, None, w, sorted_ids, eids,
                                      ntpp, True, 1, self.config, N_offset=n0, N_chunk=n1 - n0)
        moe_sum(self.D[: self.S], self.y, self.top_k, addend=self.shared_out)
        return self.y


def fused_experts(hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                  topk_weights: torch.Tensor, topk_ids: torch.Tensor, global_num_experts: int = -1,
                  w1_scale: torch.Tensor | None = None, w2_scale: torch.Tensor | None = None,
                  block_size_m: int | None = None, quant_config: Any = None,
                  expert_map: torch.Tensor | None = None, exact_dot: bool = False) -> torch.Tensor:
    """vLLM ``fused_experts`` as the reference calls it (schemes/vllm_tp.py:
    52-60; with ``expert_map`` for expert parallelism, schemes/vllm_ep.py:
    57-66) for FP8 w8a8 with [128,128] weight blocks.  Scales come either as
    keywords or from ``quant_config`` (attributes ``w1_scale``/``w2_scale``).
    With an expert map, w1/w2 hold the local experts and slots routed to other
    devices contribute zeros.  ``exact_dot`` selects the exact-dot W13
    (FusedExpertsRunner).  Allocates per call; prebuild a FusedExpertsRunner
    for timed loops."""
    if quant_config is not None:
        w1_scale = getattr(quant_config, "w1_scale", w1_scale)
        w2_scale = getattr(quant_config, "w2_scale", w2_scale)
    if w1_scale is None or w2_scale is None:
        raise ValueError("fused_experts needs w1_scale and w2_scale")
    T, k = topk_ids.shape
    gne = None if global_num_experts in (-1, None) else global_num_experts
    runner = FusedExpertsRunner(w1, w1_scale, w2, w2_scale, T, k, block_size_m,
                                global_num_experts=gne, expert_map=expert_map, exact_dot=exact_dot)
    return runner.run(hidden_states.contiguous(), topk_weights.contiguous().view(-1),
                      topk_ids.contiguous().view(-1)).clone()
