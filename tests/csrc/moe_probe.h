/*
 * moe_probe.h -- test-only probes of the gfx950 FP8 matrix core, built into
 * tests/libmoe_probe.so (not part of the shipped library or its C ABI).
 *
 * They run the grouped GEMM's own fragment code (td_benchmark_amd/csrc/
 * mfma_frag.hpp) so that the tests can check the operand layout and measure
 * how the matrix core accumulates a 128-element FP8 dot in each instruction
 * form.  Return values follow moe_mi355x.h (0 = ok, negative = argument
 * error, -100 = launch failure).
 *
 * Dot forms (`form`):
 *   0  one v_mfma_scale_f32_16x16x128_f8f6f4 (the form the GEMM uses)
 *   1  four v_mfma_f32_16x16x32_fp8_fp8, the accumulator chained through
 *      the instruction (C input = previous result)
 *   2  four v_mfma_f32_16x16x32_fp8_fp8 from zero, summed by fp32 adds
 *   3  four 16x16x128 f8f6f4 instructions, each with only one 32-element
 *      quarter of K non-zero, summed by fp32 adds
 *   4  the codes converted to bf16 (exactly) and four
 *      v_mfma_f32_16x16x32_bf16, the accumulator chained through the
 *      instruction: the exact-dot form of moe_gemm_w13_silu_quant_exact,
 *      through the same code
 *   5  (moe_probe_block_gemm only) form 4's dots with the reference's scale
 *      chain, acc = acc + (dot * a_s) * b_s, three roundings, in place of
 *      fma(dot, a_s * b_s, acc)
 */
#ifndef MOE_PROBE_H
#define MOE_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* n independent problems: A [n,16,128], B [n,16,128] e4m3fn ->
 * C [n,16,16] fp32, C[p][i][j] = sum_k A[p][i][k] * B[p][j][k], through the
 * GEMM's LDS swizzle and fragment loader.  1 <= n <= 2^20. */
int moe_probe_mfma_dot(const void* A, const void* B, float* C, int64_t n, int32_t form, void* stream);

/* Dense block-scaled GEMM with the grouped GEMM's arithmetic, one dot form:
 * acc = sum over K blocks of fma(dot_kb, As[m,kb] * Bs[n/128,kb], acc),
 * C[m,n] = bf16(acc); the weight row is the MFMA's first operand, as in the
 * grouped GEMM.  A [M,K], B [N,K] e4m3fn, As [M,K/128], Bs [N/128,K/128]
 * fp32, C [M,N] bf16.  M, N multiples of 16; K a multiple of 128; A and B
 * 16-byte aligned. */
int moe_probe_block_gemm(const void* A, const float* As, const void* B, const float* Bs, int64_t M,
                         int64_t N, int64_t K, int32_t form, void* C, void* stream);

/* Matrix-core throughput of one dot form: `waves` waves each run `iters`
 * iterations of 8 independent 128-element dots on register operands and
 * write one checksum per lane to sink [waves * 64] (so nothing is elided). */
int moe_probe_mfma_rate(int64_t waves, int32_t iters, int32_t form, float* sink, void* stream);

/* The exact-dot form's FP8 -> bf16 converter: n e4m3fn codes (n a multiple
 * of 8, 8-byte aligned) -> n bf16 bit patterns. */
int moe_probe_fp8_to_bf16(const void* codes, int64_t n, void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOE_PROBE_H */
