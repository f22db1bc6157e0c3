/*
 * moe_mi355x.h -- C ABI of the MI355X (gfx950) rank-local FP8 MoE expert path.
 *
 * Every entry point takes raw device pointers, plain sizes and a HIP stream
 * (passed as void*, a hipStream_t; NULL = the default stream), enqueues its
 * kernels on that stream and returns immediately.  Nothing here allocates:
 * the caller owns every buffer (the reference's ownership model, torch
 * allocates and the ops write into caller buffers,
 * moe_bench/overlap/overlap_forward.py:187-213).  Kernels keep no global state.
 *
 * Return value: 0 on success, a negative MOE_ERR_* code for an argument error
 * (nothing is launched), MOE_ERR_LAUNCH if the HIP launch itself failed.
 *
 * Number formats: bf16 tensors are raw uint16 bit patterns; FP8 is OCP e4m3fn
 * (one byte); scales are fp32.  Row-major everywhere.  Notation: T tokens,
 * H hidden, I per-expert intermediate, E experts, k = top_k, S = T*k token
 * slots (slot s = t*k + i), BM = block_size_m.
 *
 * Reference citations are to stmoonar/td_benchmark (paths under moe_bench/);
 * the inner-op interfaces they replace are vLLM's as that code calls them.
 */
#ifndef MOE_MI355X_H
#define MOE_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_OK 0
#define MOE_ERR_NULL_POINTER (-1)
#define MOE_ERR_BAD_SHAPE (-2)      /* negative size, dimension not a multiple of 128, misaligned pointer */
#define MOE_ERR_BAD_BLOCK_SIZE (-3) /* block_size_m not in {16, 32, 64, 128, 256} */
#define MOE_ERR_CAPACITY (-4)       /* an output capacity is below what the shape needs */
#define MOE_ERR_BAD_TOPK (-5)
#define MOE_ERR_BAD_EXPERTS (-6)
#define MOE_ERR_LAUNCH (-100)

/* A1 / A7 -- dynamic 1x128 per-token-group FP8 activation quant.
 * Replaces vLLM moe_kernel_quantize_input(A, None, float8_e4m3fn, False,
 * [128,128]) as called at overlap/overlap_forward.py:257-259 and :282-284
 * (arithmetic of verify.py:108-117).
 * x [T,H] bf16 -> q [T,H] e4m3fn, scales [T, ceil(H/128)] fp32.  When H is
 * not a multiple of 128 a row's last group holds H mod 128 values; the
 * reference zero-pads it (verify.py:111-113), which changes neither its amax
 * nor its codes.  x 2-byte aligned; H % 128 == 0 with x 16-byte and q 8-byte
 * aligned takes the vectorised kernel. */
int moe_quant_group128(const void* x_bf16, int64_t T, int64_t H, void* q_fp8, float* scales,
                       void* stream);

/* The same quant into rows of ldq >= ceil(H/128)*128 bytes, with the zero
 * code in columns [H, ceil(H/128)*128): the quantised zero padding of
 * verify.py:111-113, so that a GEMM over the padded width equals one over H
 * (no counterpart in the reference: the layout of the layer runner for
 * widths that are not a multiple of 128). */
int moe_quant_group128_padded(const void* x_bf16, int64_t T, int64_t H, void* q_fp8, int64_t ldq,
                              float* scales, void* stream);

/* A2 -- 128x128 block FP8 weight quant (build time).
 * Replaces quantize_block128 (data/checkpoint.py:28-40).
 * w [E,N,K] fp32 -> q [E,N,K] e4m3fn, scales [E, ceil(N/128), ceil(K/128)]. */
int moe_quant_block128(const float* w, int64_t E, int64_t N, int64_t K, void* q_fp8,
                       float* scales, void* stream);

/* A3 -- moe_align_block_size.
 * Replaces vLLM moe_align_block_size(topk_ids, BM, E, None) as called at
 * overlap/overlap_forward.py:165-169 and schemes/shared_expert.py:61-62.
 * topk_ids [S] int32 (flattened [T,k]) -> sorted_ids [max_padded] int32,
 * expert_ids [ceil(max_padded/BM)] int32, ntpp [1] int32.  Canonical stable
 * order inside each expert; pad value S; expert_ids -1 past ntpp.  Ids outside
 * [0,E) are dropped.  E <= 1024.  max_padded >= moe_align_max_padded(S,E,BM);
 * workspace >= moe_align_workspace_bytes(S,E) bytes of device memory. */
int64_t moe_align_max_padded(int64_t S, int32_t E, int32_t block_size_m);
int64_t moe_align_workspace_bytes(int64_t S, int32_t E);
int moe_align_block_size(const int32_t* topk_ids, int64_t S, int32_t E, int32_t block_size_m,
                         int32_t* sorted_ids, int32_t* expert_ids, int32_t* ntpp,
                         int64_t max_padded, void* workspace, void* stream);

/* A3 without caller memory.  No counterpart in the reference: for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same outputs as moe_align_block_size;
 * the workspace is a static device array of MOE_ALIGN_NOALLOC_SCRATCH_BYTES
 * per GPU, held until the process ends, so moe_align_workspace_bytes(S, E)
 * must not exceed it (else MOE_ERR_CAPACITY; DeepSeek-V3's S = 65536, E = 256
 * needs 0.33 MiB).  Calls that overlap on one GPU share the array and race.
 * The first call on a device looks the array's address up on that device,
 * which must be current. */
#define MOE_ALIGN_NOALLOC_SCRATCH_BYTES (4 * 1024 * 1024)
int moe_align_block_size_noalloc(const int32_t* topk_ids, int64_t S, int32_t E, int32_t block_size_m,
                                 int32_t* sorted_ids, int32_t* expert_ids, int32_t* ntpp,
                                 int64_t max_padded, void* stream);

/* A3 with an expert map (expert parallelism) -- vLLM moe_align_block_size(
 * topk_ids, BM, E, expert_map) as called at overlap/overlap_forward.py:165-169
 * and schemes/vllm_ep.py:57-66: the sort and padding run over the E global
 * experts, then every block's expert id is replaced by expert_map[id] (its
 * local id, or -1 for an expert on another device; the GEMMs write zeros for
 * -1 blocks).  expert_map [E] int32. */
int moe_align_block_size_mapped(const int32_t* topk_ids, int64_t S, int32_t E, int32_t block_size_m,
                                const int32_t* expert_map, int32_t* sorted_ids, int32_t* expert_ids,
                                int32_t* ntpp, int64_t max_padded, void* workspace, void* stream);

/* A5 / A8 -- block-scaled FP8 grouped GEMM, plain bf16 epilogue.
 * Replaces vLLM dispatch_fused_moe_kernel(A, B, C, A_scale, B_scale, None,
 * topk_weights, sorted_token_ids, expert_ids, num_tokens_post_padded,
 * mul_routed_weight, top_k, config, compute_type=bf16, use_fp8_w8a8=True,
 * block_shape=[128,128]) as called at overlap/kernels.py:288-310 and
 * schemes/shared_expert.py:102-123; semantics of overlap/kernels.py:95-214.
 * C[s, n] = bf16( w[s]? * sum_kb dot(A[row,kb], B[e,n,kb]) * A_scale[row,kb] * B_scale[e,n/128,kb] )
 * for every placed slot s, row = a_by_pos ? (sorted position) : s / top_k.
 * topk_weights NULL = mul_routed_weight False.  A [rows,K], A_scale [rows,K/128],
 * B [E,N,K], B_scale [E,N/128,K/128], C [S,N] bf16.  N, K % 128 == 0.
 * Every GEMM entry point without an explicit tile_m runs 256-row workgroup
 * tiles (several consecutive align blocks of one expert) when S >= 160*E and
 * block_size_m rows otherwise; the choice never changes the results. */
int moe_grouped_gemm(const void* A, const float* A_scale, const void* B, const float* B_scale,
                     const int32_t* sorted_ids, const int32_t* expert_ids, const int32_t* ntpp,
                     const float* topk_weights, int64_t S, int32_t top_k, int32_t a_by_pos,
                     int64_t N, int64_t K, int32_t E, int32_t block_size_m, int64_t max_padded,
                     void* C, void* stream);

/* A5 / A8 with an explicit workgroup -> tile order (the knob the reference's
 * tile-order sweep varies, microbench/mb_tile_order_groupgemm.py:13):
 * 0 expert-major, XCD-contiguous (what moe_grouped_gemm uses); 1 shuffled
 * (a fixed bijective scramble of the expert-major order); 2 half-phase (the
 * first and second halves of the expert-major order interleaved).  Results
 * are identical for every order. */
int moe_grouped_gemm_ordered(const void* A, const float* A_scale, const void* B,
                             const float* B_scale, const int32_t* sorted_ids,
                             const int32_t* expert_ids, const int32_t* ntpp,
                             const float* topk_weights, int64_t S, int32_t top_k, int32_t a_by_pos,
                             int64_t N, int64_t K, int32_t E, int32_t block_size_m,
                             int64_t max_padded, int32_t tile_order, void* C, void* stream);

/* A5 / A8 with an explicit tile order and tile height: a workgroup computes
 * tile_m rows = tile_m / block_size_m consecutive align blocks of one expert
 * (the reference's kernel has one block per program, kernels.py:95-126; this
 * is its BLOCK_SIZE_M choice made per launch without changing the align
 * layout).  tile_m in {16, 32, 64, 128, 256}, a multiple of block_size_m;
 * 0 = the automatic choice above.  Results are identical for every tile_m. */
int moe_grouped_gemm_tiled(const void* A, const float* A_scale, const void* B, const float* B_scale,
                           const int32_t* sorted_ids, const int32_t* expert_ids, const int32_t* ntpp,
                           const float* topk_weights, int64_t S, int32_t top_k, int32_t a_by_pos,
                           int64_t N, int64_t K, int32_t E, int32_t block_size_m, int64_t max_padded,
                           int32_t tile_order, int32_t tile_m, void* C, void* stream);

/* A5 / A8 on an N slice -- the reference's N-split wrapper
 * invoke_moe_kernel_n_split (overlap/kernels.py:219-310): computes
 * C[:, N_offset:N_offset+N_chunk] from B[:, N_offset:N_offset+N_chunk, :] and
 * the matching B_scale groups.  B [E, full_N, K], B_scale [E, full_N/128,
 * K/128], C [S, full_N] bf16 (other columns untouched).  N_offset, N_chunk,
 * full_N, K multiples of 128. */
int moe_grouped_gemm_n_split(const void* A, const float* A_scale, const void* B,
                             const float* B_scale, const int32_t* sorted_ids,
                             const int32_t* expert_ids, const int32_t* ntpp,
                             const float* topk_weights, int64_t S, int32_t top_k, int32_t a_by_pos,
                             int64_t full_N, int64_t N_offset, int64_t N_chunk, int64_t K,
                             int32_t E, int32_t block_size_m, int64_t max_padded, void* C,
                             void* stream);

/* A5 / A8 over a K window with chunk accumulation -- the reference's K-split
 * wrapper invoke_moe_kernel_k_split + fused_moe_kernel_accumulate
 * (overlap/kernels.py:36-214, 317-452): the partial product over
 * A[:, A_K_offset:+K_chunk] (A [rows, A_cols], scales [rows, A_cols/128]) and
 * B[:, :, K_offset:+K_chunk] (B [E, N, full_K], scales [E, N/128, full_K/128])
 * is rounded to bf16 (routed weight applied first) and either stored
 * (is_first_chunk != 0) or added to C: C = bf16(C + partial).  Expert -1 blocks
 * write zeros on the first chunk only.  C [S, N] bf16. */
int moe_grouped_gemm_k_split(const void* A, const float* A_scale, int64_t A_cols, int64_t A_K_offset,
                             const void* B, const float* B_scale, const int32_t* sorted_ids,
                             const int32_t* expert_ids, const int32_t* ntpp,
                             const float* topk_weights, int64_t S, int32_t top_k, int32_t a_by_pos,
                             int64_t N, int64_t full_K, int64_t K_offset, int64_t K_chunk, int32_t E,
                             int32_t block_size_m, int64_t max_padded, int32_t is_first_chunk,
                             void* C, void* stream);

/* A5 + A6 + A7 fused -- W13 grouped GEMM with SiLU*up and 1x128 FP8 quant of
 * the intermediate in the epilogue.
 * Replaces the sequence dispatch_fused_moe_kernel(W13, mul_routed_weight=False,
 * top_k=k) -> torch.ops._C.silu_and_mul -> moe_kernel_quantize_input
 * (overlap/overlap_forward.py:261-284).  Outputs are indexed by sorted
 * position p (not by slot): hq [max_padded, I] e4m3fn, hs [max_padded, I/128]
 * fp32, so the W2 GEMM reads them with a_by_pos = 1.
 * Aq [T,H], A_scale [T,H/128], W13 [E,2I,H] (gate rows [0,I), up rows [I,2I),
 * verify.py:36), W13_scale [E,2I/128,H/128].  H, I % 128 == 0. */
int moe_gemm_w13_silu_quant(const void* Aq, const float* A_scale, const void* W13,
                            const float* W13_scale, const int32_t* sorted_ids,
                            const int32_t* expert_ids, const int32_t* ntpp, int64_t S,
                            int32_t top_k, int64_t H, int64_t I, int32_t E, int32_t block_size_m,
                            int64_t max_padded, void* hq, float* hs, void* stream);

/* The fused W13 with an explicit tile height (as moe_grouped_gemm_tiled). */
int moe_gemm_w13_silu_quant_tiled(const void* Aq, const float* A_scale, const void* W13,
                                  const float* W13_scale, const int32_t* sorted_ids,
                                  const int32_t* expert_ids, const int32_t* ntpp, int64_t S,
                                  int32_t top_k, int64_t H, int64_t I, int32_t E, int32_t block_size_m,
                                  int64_t max_padded, int32_t tile_m, void* hq, float* hs, void* stream);

/* Scales by sorted position (no counterpart in the reference: a layout between
 * the build's own kernels, for the prebuilt layer).  The GEMMs above read a
 * tile's activation scales for one K block as one scale per row, each from a
 * different row of A_scale; these variants take them K-major by sorted
 * position, so the tile's scales of one K block are contiguous.  Results are
 * bit-identical to the variants above.
 *
 * moe_gather_scales_by_position: out [groups, max_padded] fp32,
 *   out[kb, p] = scales[sorted_ids[p] / top_k, kb] for p < *ntpp holding a
 *   slot (< S), and scales[0, kb] for padding positions and p >= *ntpp (the
 *   row the row-major GEMMs read for a padding position, so the outputs at
 *   padding positions agree too).  scales [rows, groups] with rows >=
 *   ceil(S / top_k) (the 1x128 quant's scales). */
int moe_gather_scales_by_position(const float* scales, int64_t rows, int64_t groups,
                                  const int32_t* sorted_ids, const int32_t* ntpp, int64_t S, int32_t top_k,
                                  int64_t max_padded, float* out, void* stream);

/* The fused W13 with A_scale_pos [H/128, max_padded] (gathered as above) and
 * its output scales hs_pos [I/128, max_padded] K-major by sorted position
 * (hq as for moe_gemm_w13_silu_quant). */
int moe_gemm_w13_silu_quant_pos(const void* Aq, const float* A_scale_pos, const void* W13,
                                const float* W13_scale, const int32_t* sorted_ids,
                                const int32_t* expert_ids, const int32_t* ntpp, int64_t S,
                                int32_t top_k, int64_t H, int64_t I, int32_t E, int32_t block_size_m,
                                int64_t max_padded, int32_t tile_m, void* hq, float* hs_pos, void* stream);

/* The fused W13 with exact dot products (an opt-in mode; its dots follow the
 * reference's per-block product, overlap/kernels.py:172-179, without the FP8
 * matrix core's truncation).  The FP8 16x16x128 instruction truncates the
 * products of each group of 8 inside a 128-element dot, which moves about 1 %
 * of the bf16 C13 values across a rounding boundary and about 0.2 % of the
 * intermediate codes by up to a few ULPs.  This variant converts the FP8
 * codes exactly to bf16 and takes every 128-element dot as four bf16 MFMAs,
 * whose products are exact, and applies the scales as the reference does,
 * acc + (dot * a_scale) * b_scale with each operation rounded in fp32, at
 * about twice the matrix-core time of the FP8 form.  Same arguments and outputs as moe_gemm_w13_silu_quant_tiled with
 * scales_by_position == 0, and as moe_gemm_w13_silu_quant_pos (A_scale and
 * hs K-major by sorted position) with scales_by_position != 0. */
int moe_gemm_w13_silu_quant_exact(const void* Aq, const float* A_scale, const void* W13,
                                  const float* W13_scale, const int32_t* sorted_ids,
                                  const int32_t* expert_ids, const int32_t* ntpp, int64_t S,
                                  int32_t top_k, int64_t H, int64_t I, int32_t E, int32_t block_size_m,
                                  int64_t max_padded, int32_t tile_m, int32_t scales_by_position, void* hq,
                                  float* hs, void* stream);

/* The W2 GEMM (A rows by sorted position, as a_by_pos = 1, C rows by slot,
 * routed weights if topk_weights is not null) with A_scale_pos [K/128,
 * max_padded] K-major by sorted position, as moe_gemm_w13_silu_quant_pos
 * writes it. */
int moe_grouped_gemm_pos(const void* A, const float* A_scale_pos, const void* B, const float* B_scale,
                         const int32_t* sorted_ids, const int32_t* expert_ids, const int32_t* ntpp,
                         const float* topk_weights, int64_t S, int64_t N, int64_t K, int32_t E,
                         int32_t block_size_m, int64_t max_padded, int32_t tile_m, void* C, void* stream);

/* A6 -- silu_and_mul.  Replaces torch.ops._C.silu_and_mul(out, in)
 * (overlap/overlap_forward.py:277-279): h[r,j] = bf16(silu(c[r,j]) * c[r,I+j]).
 * c [R, 2I] bf16 -> h [R, I] bf16; I % 8 == 0. */
int moe_silu_and_mul(const void* c_bf16, int64_t R, int64_t I, void* h_bf16, void* stream);

/* A6 + A7 standalone -- SiLU*up then 1x128 FP8 quant of the bf16 product, one
 * pass: replaces silu_and_mul followed by moe_kernel_quantize_input
 * (overlap/overlap_forward.py:277-284) where C13 exists (the unfused chain;
 * the reference's swiglu_group128 kernel, tdx/kernels/swiglu_quantize_fp8.py:
 * 80-85, microbench/mb_quant_kernels.py:11).  Codes and scales equal those of
 * moe_silu_and_mul followed by moe_quant_group128 bit for bit.
 * c [R, 2I] bf16 -> q [R, I] e4m3fn, scales [R, I/128]; I % 128 == 0. */
int moe_silu_mul_quant_group128(const void* c_bf16, int64_t R, int64_t I, void* q_fp8,
                                float* scales, void* stream);

/* A9 -- top-k un-permute / reduce.  Replaces torch.sum(C_down.view(T,k,H),
 * dim=1) (overlap/overlap_forward.py:304-313): y[t] = bf16(sum_i D[t*k+i]),
 * fp32 accumulation.  D [T*k, H] bf16 -> y [T, H] bf16; H % 8 == 0, k <= 32. */
int moe_reduce_topk(const void* D_bf16, int64_t T, int32_t top_k, int64_t H, void* y_bf16,
                    void* stream);

/* A9 + shared expert -- the reduce followed by the bf16 add of the shared
 * expert's output: y[t] = bf16(bf16(sum_i D[t*k+i]) + addend[t]), replacing
 * `result + shared(hidden)` (schemes/vllm_tp.py:62-63, schemes/vllm_ep.py:
 * 66-67) without re-reading the [T,H] sum.  addend [T, H] bf16. */
int moe_reduce_topk_add(const void* D_bf16, const void* addend_bf16, int64_t T, int32_t top_k,
                        int64_t H, void* y_bf16, void* stream);

/* FP8 reduce-scatter combine -- the dequantise-and-sum of the FP8 chunks a
 * rank receives in the FP8-compressed reduce-scatter leg, replacing
 * `(fp8.to(float32) * scale.repeat_interleave(128)).sum(dim=0).to(bfloat16)`
 * (overlap/overlap_forward.py:932-944; the senders quantise with
 * moe_quant_group128, :900-905):
 *   out[m, n] = bf16( sum_{r<R} float(q[r, m, n]) * s[r*M + m, n/128] ),
 * each product rounded to fp32, the sum in fp32 over ascending r.
 * q [R, M, N] e4m3fn (R ranks' chunks of M rows, contiguous); s fp32 with a
 * row of scale_ld >= ceil(N/128) entries per (r, m); out bf16 with rows of
 * out_ld >= N elements (a column slice of a wider output may be written in
 * place).  N % 16 == 0, out_ld % 8 == 0, q and out 16-byte aligned;
 * 1 <= R <= 64. */
int moe_fp8_dequant_sum(const void* q_fp8, const float* scales, int64_t R, int64_t M, int64_t N,
                        int64_t scale_ld, void* out_bf16, int64_t out_ld, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOE_MI355X_H */
