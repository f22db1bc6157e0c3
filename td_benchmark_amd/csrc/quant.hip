// A1 / A7: dynamic 1x128 per-token-group FP8 quant of bf16 activations, and
//          the standalone SiLU*up + 1x128 quant (A6 + A7) of the unfused chain.
// A2:      128x128 block FP8 quant of fp32 weights (build time).
//
// Arithmetic follows reference moe_bench/verify.py:108-117 and
// data/checkpoint.py:28-40: scale = max(amax/448, 1e-12) by IEEE division,
// code = e4m3fn_RNE(clamp(x / scale, +-448)).
//
// quant_group128 is HBM-bound: 2 B in + 1 B out per element + 4 B of scale per
// 128 elements (widths that are not a multiple of 128, or unaligned rows, take
// a general one-wave-per-group kernel instead).  Sixteen lanes own one 128-element group (16 B = 8 bf16 each),
// so every wave reads 1 KiB and writes 512 B contiguously with 128-bit loads;
// the group amax is a 16-lane xor-shuffle reduction.  Non-temporal
// (streaming) loads and stores and a shallow per-thread unroll measured best
// on MI355X: many short waves keep more requests in flight than a deep unroll.
#include "common.hpp"

namespace moe {

constexpr int kQuantThreads = 256;
// 16 B chunks per thread (measured on MI355X: 2 for the plain quant, 4 for
// the SiLU*up form, which reads twice the bytes per output chunk).
template <bool SWIGLU>
constexpr int quant_unroll() { return SWIGLU ? 4 : 2; }

// SWIGLU = false: x [rows, W] bf16 is quantised directly (A1 / A7).
// SWIGLU = true:  x [rows, 2W] bf16 holds gate | up; the quantised value is
//   h = bf16(silu(gate) * up) (A6 then A7, the standalone form of what the
//   fused W13 epilogue does), with the same rounding chain as the separate
//   silu_and_mul and quant kernels, so the codes agree bit for bit.
// A chunk is 8 consecutive output columns of one row; W/8 chunks per row.
template <bool SWIGLU>
__global__ __launch_bounds__(kQuantThreads) void quant_group128_kernel(
    const uint16_t* __restrict__ x, uint8_t* __restrict__ q, float* __restrict__ s,
    int64_t n_chunks, int64_t chunks_per_row) {
  constexpr int kQuantUnroll = quant_unroll<SWIGLU>();
  const int tid = threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * kQuantThreads * kQuantUnroll;
  constexpr int NLOAD = SWIGLU ? 2 : 1;
  v4i raw[kQuantUnroll][NLOAD];
#pragma unroll
  for (int i = 0; i < kQuantUnroll; ++i) {
    const int64_t ch = base + tid + i * kQuantThreads;
    if (ch < n_chunks) {
      if constexpr (SWIGLU) {
        const int64_t r = ch / chunks_per_row, cc = ch % chunks_per_row;
        const uint16_t* row = x + r * chunks_per_row * 16;
        raw[i][0] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(row + cc * 8));
        raw[i][NLOAD - 1] =
            __builtin_nontemporal_load(reinterpret_cast<const v4i*>(row + chunks_per_row * 8 + cc * 8));
      } else {
        raw[i][0] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(x + ch * 8));
      }
    } else {
#pragma unroll
      for (int l = 0; l < NLOAD; ++l) raw[i][l] = (v4i){0, 0, 0, 0};
    }
  }
#pragma unroll
  for (int i = 0; i < kQuantUnroll; ++i) {
    const int64_t ch = base + tid + i * kQuantThreads;
    float v[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w = (uint32_t)raw[i][0][j];
      if constexpr (SWIGLU) {
        const uint32_t u = (uint32_t)raw[i][NLOAD - 1][j];
        v[2 * j] = silu_mul_bf16(lo_bf16(w), lo_bf16(u));
        v[2 * j + 1] = silu_mul_bf16(hi_bf16(w), hi_bf16(u));
      } else {
        v[2 * j] = lo_bf16(w);
        v[2 * j + 1] = hi_bf16(w);
      }
    }
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
    // 16 lanes of one group are 16 consecutive lanes of the wave.
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    amax = fmaxf(amax, __shfl_xor(amax, 4));
    amax = fmaxf(amax, __shfl_xor(amax, 8));
    const float sc = group_scale(amax);
    const float inv = 1.0f / sc;
    const uint32_t lo = quant4_e4m3(v[0], v[1], v[2], v[3], sc, inv);
    const uint32_t hi = quant4_e4m3(v[4], v[5], v[6], v[7], sc, inv);
    if (ch < n_chunks) {
      __builtin_nontemporal_store((v2u){lo, hi}, reinterpret_cast<v2u*>(q + ch * 8));
      if ((tid & 15) == 0) s[ch >> 4] = sc;
    }
  }
}

// Any width and row strides (the vectorised kernel above needs W % 128 == 0
// and aligned rows): one wave per 128-column group of one row, two columns
// per lane.  A row's last group holds W mod 128 columns when W is not a
// multiple of 128; the reference zero-pads it to 128 (verify.py:111-113), and
// zeros change neither the group's amax nor the other codes, so only the W
// columns are read and their codes written.  Columns [W, pad_to) of q get the
// zero code (the zero padding, quantised).
__global__ __launch_bounds__(256) void quant_group128_any_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int64_t rows, int64_t W, int64_t pad_to,
    uint8_t* __restrict__ q, int64_t ldq, float* __restrict__ s, int64_t lds) {
  const int lane = threadIdx.x & 63;
  const int64_t groups = (pad_to + 127) / 128;
  const int64_t g = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (row, group) of this wave
  if (g >= rows * groups) return;
  const int64_t r = g / groups, c0 = (g % groups) * 128 + 2 * lane;
  float v[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) v[j] = c0 + j < W ? bf16_to_f32(x[r * ldx + c0 + j]) : 0.0f;
  float amax = fmaxf(fabsf(v[0]), fabsf(v[1]));
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  const float sc = group_scale(amax);
  const float inv = 1.0f / sc;
  const uint32_t codes = pack4_e4m3(clamp_fp8(div_by(v[0], sc, inv)), clamp_fp8(div_by(v[1], sc, inv)), 0.0f, 0.0f);
#pragma unroll
  for (int j = 0; j < 2; ++j)
    if (c0 + j < pad_to) q[r * ldq + c0 + j] = c0 + j < W ? (uint8_t)(codes >> (8 * j)) : 0;
  if (lane == 0 && g % groups * 128 < W) s[r * lds + g % groups] = sc;
}

// One workgroup per 128x128 block of one expert.  w fp32 [E, N, K] row-major.
__global__ __launch_bounds__(256) void quant_block128_kernel(
    const float* __restrict__ w, uint8_t* __restrict__ q, float* __restrict__ s,
    int64_t N, int64_t K, int64_t NB, int64_t KB) {
  const int64_t blk = blockIdx.x;
  const int64_t kb = blk % KB;
  const int64_t nb = (blk / KB) % NB;
  const int64_t e = blk / (KB * NB);
  const int tid = threadIdx.x;
  const int col = (tid & 31) * 4;          // 32 threads x 4 columns = 128
  const int row0 = tid >> 5;               // 8 rows per pass, 16 passes
  const int64_t k = kb * 128 + col;
  float vals[16][4];
  float amax = 0.0f;
#pragma unroll
  for (int p = 0; p < 16; ++p) {
    int64_t n = nb * 128 + row0 + p * 8;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v = 0.0f;
      if (n < N && k + j < K) v = w[(e * N + n) * K + k + j];
      vals[p][j] = v;
      amax = fmaxf(amax, fabsf(v));
    }
  }
  __shared__ float red[8];
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float sc = group_scale(amax);
  if (tid == 0) s[(e * NB + nb) * KB + kb] = sc;
#pragma unroll
  for (int p = 0; p < 16; ++p) {
    int64_t n = nb * 128 + row0 + p * 8;
    if (n >= N) continue;
    float a = clamp_fp8(vals[p][0] / sc), b = clamp_fp8(vals[p][1] / sc);
    float c = clamp_fp8(vals[p][2] / sc), d = clamp_fp8(vals[p][3] / sc);
    uint32_t packed = pack4_e4m3(a, b, c, d);
    uint8_t* dst = q + (e * N + n) * K + k;
    if (k + 3 < K && ((K & 3) == 0)) {
      *reinterpret_cast<uint32_t*>(dst) = packed;
    } else {
      for (int j = 0; j < 4; ++j)
        if (k + j < K) dst[j] = (uint8_t)(packed >> (8 * j));
    }
  }
}

}  // namespace moe

using namespace moe;

// Rows of x (stride ldx) -> rows of q (stride ldq) with codes in [0, H) and
// zero codes in [H, pad_to), scales [T, ceil(H/128)] with stride lds.
static int quant_any(const void* x_bf16, int64_t ldx, int64_t T, int64_t H, int64_t pad_to, void* q_fp8,
                     int64_t ldq, float* scales, int64_t lds, void* stream) {
  const int64_t waves = T * ((pad_to + 127) / 128);
  hipLaunchKernelGGL(quant_group128_any_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)x_bf16, ldx, T, H, pad_to, (uint8_t*)q_fp8, ldq, scales,
                     lds);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

extern "C" int moe_quant_group128(const void* x_bf16, int64_t T, int64_t H, void* q_fp8,
                                  float* scales, void* stream) {
  if (T < 0 || H < 0) return kErrBadShape;
  if (T == 0 || H == 0) return kOk;
  if (!x_bf16 || !q_fp8 || !scales) return kErrNullPointer;
  if ((H % 128 != 0 || ((uintptr_t)x_bf16 & 15) != 0 || ((uintptr_t)q_fp8 & 7) != 0)) {
    if (((uintptr_t)x_bf16 & 1) != 0) return kErrBadShape;
    if (T * ((H + 127) / 128) > (int64_t)0xFFFFFFFF * 4) return kErrBadShape;
    return quant_any(x_bf16, H, T, H, H, q_fp8, H, scales, (H + 127) / 128, stream);
  }
  const int64_t n_chunks = T * H / 8;
  constexpr int64_t per_block = kQuantThreads * quant_unroll<false>();
  const int64_t blocks = (n_chunks + per_block - 1) / per_block;
  hipLaunchKernelGGL(quant_group128_kernel<false>, dim3((unsigned)blocks), dim3(kQuantThreads), 0,
                     (hipStream_t)stream, (const uint16_t*)x_bf16, (uint8_t*)q_fp8, scales,
                     n_chunks, H / 8);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

extern "C" int moe_quant_group128_padded(const void* x_bf16, int64_t T, int64_t H, void* q_fp8, int64_t ldq,
                                         float* scales, void* stream) {
  if (T < 0 || H < 0) return kErrBadShape;
  const int64_t hp = (H + 127) / 128 * 128;
  if (ldq < hp) return kErrBadShape;
  if (T == 0 || H == 0) return kOk;
  if (!x_bf16 || !q_fp8 || !scales) return kErrNullPointer;
  if (ldq == H) return moe_quant_group128(x_bf16, T, H, q_fp8, scales, stream);
  if (((uintptr_t)x_bf16 & 1) != 0) return kErrBadShape;
  if (T * (hp / 128) > (int64_t)0xFFFFFFFF * 4) return kErrBadShape;
  return quant_any(x_bf16, H, T, H, hp, q_fp8, ldq, scales, hp / 128, stream);
}

extern "C" int moe_silu_mul_quant_group128(const void* c_bf16, int64_t R, int64_t I, void* q_fp8,
                                           float* scales, void* stream) {
  if (R < 0 || I < 0) return kErrBadShape;
  if (R == 0 || I == 0) return kOk;
  if (!c_bf16 || !q_fp8 || !scales) return kErrNullPointer;
  if (I % 128 != 0) return kErrBadShape;
  if (((uintptr_t)c_bf16 & 15) != 0 || ((uintptr_t)q_fp8 & 7) != 0) return kErrBadShape;
  const int64_t n_chunks = R * I / 8;
  constexpr int64_t per_block = kQuantThreads * quant_unroll<true>();
  const int64_t blocks = (n_chunks + per_block - 1) / per_block;
  hipLaunchKernelGGL(quant_group128_kernel<true>, dim3((unsigned)blocks), dim3(kQuantThreads), 0,
                     (hipStream_t)stream, (const uint16_t*)c_bf16, (uint8_t*)q_fp8, scales,
                     n_chunks, I / 8);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

extern "C" int moe_quant_block128(const float* w, int64_t E, int64_t N, int64_t K, void* q_fp8,
                                  float* scales, void* stream) {
  if (E < 0 || N < 0 || K < 0) return kErrBadShape;
  if (E == 0 || N == 0 || K == 0) return kOk;
  if (!w || !q_fp8 || !scales) return kErrNullPointer;
  const int64_t NB = (N + 127) / 128, KB = (K + 127) / 128;
  hipLaunchKernelGGL(quant_block128_kernel, dim3((unsigned)(E * NB * KB)), dim3(256), 0,
                     (hipStream_t)stream, w, (uint8_t*)q_fp8, scales, N, K, NB, KB);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}
