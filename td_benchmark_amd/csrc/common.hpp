// Shared device helpers for the gfx950 MoE expert path.
//
// Number formats: activations and outputs are bf16 (raw uint16 bits), FP8 is
// OCP e4m3fn (the format gfx950's conversion and MFMA f8f6f4 instructions use
// with format code 0), scales are fp32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moe_mi355x.h"

#define MOE_HOST_DEVICE __host__ __device__ __forceinline__
#define MOE_DEVICE __device__ __forceinline__

namespace moe {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));

constexpr float kFp8Max = 448.0f;
constexpr float kScaleFloor = 1e-12f;   // verify.py:115 clamp(min=1e-12)

// Status codes returned by every extern "C" entry point.
enum Status : int {
  kOk = 0,
  kErrNullPointer = -1,
  kErrBadShape = -2,        // a size is negative, or a dimension is not a multiple of 128
  kErrBadBlockSize = -3,    // block_size_m not in {16, 32, 64, 128, 256}
  kErrCapacity = -4,        // an output buffer is smaller than the shape needs
  kErrBadTopK = -5,
  kErrBadExperts = -6,
  kErrLaunch = -100,        // hipGetLastError() reported a launch failure
};
static_assert(kErrNullPointer == MOE_ERR_NULL_POINTER && kErrBadShape == MOE_ERR_BAD_SHAPE &&
                  kErrBadBlockSize == MOE_ERR_BAD_BLOCK_SIZE && kErrCapacity == MOE_ERR_CAPACITY &&
                  kErrBadTopK == MOE_ERR_BAD_TOPK && kErrBadExperts == MOE_ERR_BAD_EXPERTS &&
                  kErrLaunch == MOE_ERR_LAUNCH,
              "status codes must match the C header");

// Block sizes the align and GEMM kernels are instantiated for.
inline bool block_m_ok(int BM) { return BM == 16 || BM == 32 || BM == 64 || BM == 128 || BM == 256; }

MOE_DEVICE float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// fp32 -> bf16, round to nearest even (finite values; NaN stays NaN).
MOE_DEVICE uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

MOE_DEVICE float round_bf16(float f) { return __uint_as_float(f32_to_bf16_bits(f) << 16); }

// Two fp32 -> packed bf16 pair (round to nearest even, v_cvt_pk_bf16_f32);
// a in the low half.
MOE_DEVICE uint32_t pack_bf16x2(float a, float b) {
  typedef float v2f __attribute__((ext_vector_type(2)));
  typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
  const v2bf r = __builtin_convertvector((v2f){a, b}, v2bf);
  return __builtin_bit_cast(uint32_t, r);
}
MOE_DEVICE float lo_bf16(uint32_t p) { return __uint_as_float(p << 16); }
MOE_DEVICE float hi_bf16(uint32_t p) { return __uint_as_float(p & 0xFFFF0000u); }

// silu(g) * u = g / (1 + exp(-g)) * u in fp32 (reciprocal form), rounded to
// bf16.  g and u are the bf16-rounded gate / up values of the chain
// C (bf16) -> silu_and_mul (fp32 math, bf16 out).  Shared by the standalone
// silu_and_mul kernel and the fused W13 epilogue so the two agree bit for bit.
MOE_DEVICE float silu_mul_bf16(float g, float u) {
  const float s = g * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
  return lo_bf16(pack_bf16x2(s * u, 0.0f));
}

// Correctly rounded x / s given inv = RN(1/s): q0 = RN(x*inv); the residual
// x - q0*s is exact under fma; one correction step gives RN(x/s) (Markstein's
// final-step theorem for round-to-nearest, valid away from overflow and
// subnormal quotients).  The sign is copied from x so that -0 / s stays -0
// (the correction step alone would return +0 for x = -0).  s > 0 always.
MOE_DEVICE float div_by(float x, float s, float inv) {
  float q0 = x * inv;
  float r = __builtin_fmaf(-q0, s, x);
  return __builtin_copysignf(__builtin_fmaf(r, inv, q0), x);
}

MOE_DEVICE float clamp_fp8(float v) { return __builtin_amdgcn_fmed3f(v, -kFp8Max, kFp8Max); }

// Four fp32 (already clamped to +-448) -> four packed e4m3fn bytes, RNE.
// The hardware conversion returns +0 for a negative input that rounds to
// zero, where OCP e4m3fn (and torch's cast) keep the sign (-0 = 0x80): each
// input's sign bit is ORed into its byte, a no-op for non-zero results.
MOE_DEVICE uint32_t pack4_e4m3(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  const uint32_t sg = ((__float_as_uint(a) >> 24) & 0x80u) | ((__float_as_uint(b) >> 16) & 0x8000u) |
                      ((__float_as_uint(c) >> 8) & 0x800000u) | (__float_as_uint(d) & 0x80000000u);
  return (uint32_t)w | sg;
}

// Four values of one 1x128 group with scale s > 0 (inv = RN(1/s)) -> four
// packed e4m3fn codes, e4m3_RNE(clamp(RN(x / s), +-448)).  The quotient is
// the correctly rounded one of div_by without its sign copy: a quotient that
// is zero or rounds to zero in e4m3 gets x's sign from the sign bytes ORed in
// below (x / s has x's sign, and -0 / s = -0), as torch's cast keeps -0;
// for every other code the OR is a no-op.  Two v_perm_b32 gather the four
// sign bytes; bit-identical to pack4_e4m3 of clamp_fp8(div_by(x, s, inv)).
MOE_DEVICE uint32_t quant4_e4m3(float a, float b, float c, float d, float s, float inv) {
  auto q = [&](float x) {
    const float q0 = x * inv;
    const float r = __builtin_fmaf(-q0, s, x);
    return clamp_fp8(__builtin_fmaf(r, inv, q0));
  };
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(q(a), q(b), 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(q(c), q(d), w, true);
  // byte 3 of a, b -> bytes 0, 1; byte 3 of c, d -> bytes 2, 3
  const uint32_t ab = __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x0c0c0703u);
  const uint32_t cd = __builtin_amdgcn_perm(__float_as_uint(d), __float_as_uint(c), 0x07030c0cu);
  return (uint32_t)w | ((ab | cd) & 0x80808080u);
}

// Group scale of verify.py:115: max(amax / 448, 1e-12), IEEE division.
MOE_DEVICE float group_scale(float amax) {
  float s = amax / kFp8Max;
  return s < kScaleFloor ? kScaleFloor : s;
}

}  // namespace moe
