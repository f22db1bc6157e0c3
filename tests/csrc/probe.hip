// Test-only probes of the gfx950 FP8 matrix core (declared in moe_probe.h).
// The fragments come from the grouped GEMM's own loader (mfma_frag.hpp): lane
// (fr = lane mod 16, kseg = lane / 16) holds K bytes [32 kseg, 32 kseg + 32)
// of row fr.  Every form feeds both operands the same K placement, so each
// form computes the same dot whatever order the hardware takes K in.
#include "mfma_frag.hpp"
#include "moe_probe.h"

namespace moe_probe {

using namespace moe;

// Bytes [8q, 8q + 8) of a lane's 32-byte fragment: the 8 K values one
// 16x16x32 instruction takes from that lane.
__device__ __forceinline__ long quarter(const v8i& f, int q) {
  return (long)(((uint64_t)(uint32_t)f[2 * q + 1] << 32) | (uint32_t)f[2 * q]);
}

// The fragment with every byte outside quarter q cleared.
__device__ __forceinline__ v8i only_quarter(const v8i& f, int q) {
  v8i r = {0, 0, 0, 0, 0, 0, 0, 0};
  r[2 * q] = f[2 * q];
  r[2 * q + 1] = f[2 * q + 1];
  return r;
}

__device__ __forceinline__ v4f dot_form(const v8i& a, const v8i& b, int form) {
  const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
  if (form == 0) return mfma_fp8(a, b);
  if (form == 4) {  // the exact-dot form of the grouped GEMM (mfma_frag.hpp)
    v8bf aq[4], bq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      aq[q] = fp8_quarter_bf16(a, q);
      bq[q] = fp8_quarter_bf16(b, q);
    }
    return mfma_bf16_dot128(aq, bq);
  }
  v4f acc = zero;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (form == 1) {
      acc = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(quarter(a, q), quarter(b, q), acc, 0, 0, 0);
    } else if (form == 2) {
      const v4f p = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(quarter(a, q), quarter(b, q), zero, 0, 0, 0);
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[v] = acc[v] + p[v];
    } else {
      const v4f p = mfma_fp8(only_quarter(a, q), b);
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[v] = acc[v] + p[v];
    }
  }
  return acc;
}

// One wave per problem: A and B staged through the GEMM's swizzled LDS rows.
__global__ __launch_bounds__(64) void dot_kernel(const uint8_t* __restrict__ A, const uint8_t* __restrict__ B,
                                                 float* __restrict__ C, int form) {
  __shared__ __attribute__((aligned(16))) uint8_t sAB[2 * 16 * 128];
  const int lane = threadIdx.x;
  const int64_t p = blockIdx.x;
  const uint8_t* a = A + p * 2048;
  const uint8_t* b = B + p * 2048;
  for (int ci = lane; ci < 256; ci += 64) {
    const int row = (ci >> 3) & 15, cc = ci & 7;
    const uint8_t* src = (ci < 128 ? a : b) + row * 128 + cc * 16;
    *reinterpret_cast<v4i*>(sAB + (ci < 128 ? 0 : 2048) + row * 128 + (slot_of(cc, row) << 4)) =
        *reinterpret_cast<const v4i*>(src);
  }
  __syncthreads();
  const int fr = lane & 15, kseg = lane >> 4;
  const uint8_t* p0 = sAB + fr * 128 + (slot_of(2 * kseg, fr) << 4);
  const uint8_t* p1 = sAB + fr * 128 + (slot_of(2 * kseg + 1, fr) << 4);
  const v4f r = dot_form(frag_at<0>(p0, p1), frag_at<2048>(p0, p1), form);
  // lane holds D[4 kseg + v][fr]: rows of the first operand (A), columns of the second
#pragma unroll
  for (int v = 0; v < 4; ++v) C[p * 256 + (4 * kseg + v) * 16 + fr] = r[v];
}

// One wave per 16 (tokens) x 16 (columns) output tile; fragments straight
// from global memory in the same K placement as the LDS path.
__global__ __launch_bounds__(64) void block_gemm_kernel(const uint8_t* __restrict__ A, const float* __restrict__ As,
                                                        const uint8_t* __restrict__ B, const float* __restrict__ Bs,
                                                        int64_t N, int64_t K, int form,
                                                        uint16_t* __restrict__ C) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x, fr = lane & 15, kseg = lane >> 4;
  const int64_t m0 = (int64_t)blockIdx.y * 16, n0 = (int64_t)blockIdx.x * 16;
  const int64_t KB = K / 128;
  const uint8_t* arow = A + (m0 + fr) * K + 32 * kseg;
  const uint8_t* brow = B + (n0 + fr) * K + 32 * kseg;
  v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int64_t kb = 0; kb < KB; ++kb) {
    const v4i a0 = *reinterpret_cast<const v4i*>(arow + kb * 128);
    const v4i a1 = *reinterpret_cast<const v4i*>(arow + kb * 128 + 16);
    const v4i b0 = *reinterpret_cast<const v4i*>(brow + kb * 128);
    const v4i b1 = *reinterpret_cast<const v4i*>(brow + kb * 128 + 16);
    const v8i fa = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
    const v8i fb = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
    // weight fragment first: lane (fr, kseg) holds token fr, columns 4 kseg + v
    const v4f p = dot_form(fb, fa, form == 5 ? 4 : form);
    const float sa = As[(m0 + fr) * KB + kb], sb = Bs[(n0 / 128) * KB + kb];
    if (form == 5) {
      // the reference's chain, acc += dot * a_s * b_s with three roundings
      // (overlap/kernels.py:179), in place of the kernel's fma(dot, a_s * b_s, acc)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float t = p[v] * sa;
        t = t * sb;
        acc[v] = acc[v] + t;
      }
    } else {
      const float sab = sa * sb;
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[v] = __builtin_fmaf(p[v], sab, acc[v]);
    }
  }
  v2u pk;
  pk[0] = pack_bf16x2(acc[0], acc[1]);
  pk[1] = pack_bf16x2(acc[2], acc[3]);
  *reinterpret_cast<v2u*>(C + (m0 + fr) * N + n0 + 4 * kseg) = pk;
}

__global__ __launch_bounds__(256) void rate_kernel(int iters, int form, float* __restrict__ sink) {
  const int64_t gl = (int64_t)blockIdx.x * 256 + threadIdx.x;
  v8i a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    // finite e4m3 codes that vary by lane and register (no NaN byte 0x7f/0xff)
    const uint32_t x = (uint32_t)(gl * 2654435761u + i * 40503u);
    a[i] = (int)(x & 0x3e3e3e3eu);
    b[i] = (int)((x >> 3) & 0x3d3d3d3du);
  }
  v4f acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const v4f p = dot_form(a, b, form);
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[c][v] += p[v];
    }
    a[0] ^= (it & 0x1e);  // vary the operands; bytes stay within 0x3e (finite, no 0x7f)
  }
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < 8; ++c) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
  sink[gl] = s;
}

// Each thread converts 8 codes (two dwords, quarter 0 of a fragment) with
// the exact-dot form's converter and writes their bf16 bits.
__global__ __launch_bounds__(256) void fp8_bf16_kernel(const uint32_t* __restrict__ codes, int64_t n8,
                                                        uint16_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  v8i f = {0, 0, 0, 0, 0, 0, 0, 0};
  f[0] = (int)codes[2 * i];
  f[1] = (int)codes[2 * i + 1];
  const v4u w = __builtin_bit_cast(v4u, fp8_quarter_bf16(f, 0));  // whole-vector cast (see mfma_frag.hpp)
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    out[8 * i + 2 * c] = (uint16_t)(w[c] & 0xFFFFu);
    out[8 * i + 2 * c + 1] = (uint16_t)(w[c] >> 16);
  }
}

}  // namespace moe_probe

using namespace moe_probe;

extern "C" int moe_probe_fp8_to_bf16(const void* codes, int64_t n, void* out, void* stream) {
  if (!codes || !out) return kErrNullPointer;
  if (n <= 0 || n % 8 || n > ((int64_t)1 << 30) || ((uintptr_t)codes & 7) || ((uintptr_t)out & 1))
    return kErrBadShape;
  const int64_t n8 = n / 8;
  hipLaunchKernelGGL(fp8_bf16_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint32_t*)codes, n8, (uint16_t*)out);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

extern "C" int moe_probe_mfma_dot(const void* A, const void* B, float* C, int64_t n, int32_t form, void* stream) {
  if (!A || !B || !C) return kErrNullPointer;
  if (n <= 0 || n > (1 << 20) || form < 0 || form > 4) return kErrBadShape;
  if (((uintptr_t)A & 15) || ((uintptr_t)B & 15)) return kErrBadShape;
  hipLaunchKernelGGL(dot_kernel, dim3((unsigned)n), dim3(64), 0, (hipStream_t)stream, (const uint8_t*)A,
                     (const uint8_t*)B, C, (int)form);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

extern "C" int moe_probe_block_gemm(const void* A, const float* As, const void* B, const float* Bs, int64_t M,
                                    int64_t N, int64_t K, int32_t form, void* C, void* stream) {
  if (!A || !As || !B || !Bs || !C) return kErrNullPointer;
  if (M <= 0 || N <= 0 || K <= 0 || M % 16 || N % 16 || K % 128 || form < 0 || form > 5) return kErrBadShape;
  if (M / 16 > 65535 || N / 16 > (int64_t)1 << 30) return kErrBadShape;
  if (((uintptr_t)A & 15) || ((uintptr_t)B & 15) || ((uintptr_t)C & 7)) return kErrBadShape;
  hipLaunchKernelGGL(block_gemm_kernel, dim3((unsigned)(N / 16), (unsigned)(M / 16)), dim3(64), 0,
                     (hipStream_t)stream, (const uint8_t*)A, As, (const uint8_t*)B, Bs, N, K, (int)form,
                     (uint16_t*)C);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

extern "C" int moe_probe_mfma_rate(int64_t waves, int32_t iters, int32_t form, float* sink, void* stream) {
  if (!sink) return kErrNullPointer;
  if (waves <= 0 || waves % 4 || waves > (1 << 22) || iters <= 0 || form < 0 || form > 4) return kErrBadShape;
  hipLaunchKernelGGL(rate_kernel, dim3((unsigned)(waves / 4)), dim3(256), 0, (hipStream_t)stream, (int)iters,
                     (int)form, sink);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}
