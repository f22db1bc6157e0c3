// A9: top-k un-permute / reduce, and A6 as a standalone op.
//
// moe_reduce_topk: y[t, :] = bf16( sum_{i<k} float(D[t*k + i, :]) ), fp32
// accumulation in ascending i -- the reference's
// torch.sum(C_down.view(T, k, H), dim=1) (overlap/overlap_forward.py:304-313);
// the routed weights were already applied by the W2 GEMM epilogue.
// HBM-bound: 2*k*H bytes read + 2*H written per token; each thread owns 16 B
// (8 columns) of one token and keeps its k row loads in flight together.
//
// moe_silu_and_mul: h[r, j] = bf16( silu(c[r, j]) * c[r, I + j] ) with fp32
// math (torch.ops._C.silu_and_mul, overlap/overlap_forward.py:277-279).  The
// fused W13 kernel performs the same arithmetic in its epilogue; this op
// serves the unfused chain.
//
// moe_fp8_dequant_sum: the combine of the FP8-compressed reduce-scatter leg
// (overlap/overlap_forward.py:932-944): out[m, n] = bf16( sum_r
// float(q[r, m, n]) * s[r, m, n/128] ), the product rounded to fp32 (no fused
// multiply-add), the sum in fp32 over ascending r.  HBM-bound: R*N + 4*R*N/128
// bytes read and 2*N written per row; each thread owns 16 columns of one row
// and keeps up to kDequantBatch ranks' loads in flight.
#include "common.hpp"

namespace moe {

constexpr int kMaxTopK = 32;

// ADD: y[t] = bf16( float(bf16(sum)) + float(addend[t]) ), the bf16 sum of the
// routed output and the shared expert's output (result + shared(hidden) of
// schemes/vllm_tp.py:62-63 and schemes/vllm_ep.py:66-67), fused into the
// reduce so the [T,H] sum is not re-read.
template <int KMAX, bool ADD>
__global__ __launch_bounds__(256) void reduce_topk_kernel(const uint16_t* __restrict__ D,
                                                          const uint16_t* __restrict__ addend,
                                                          uint16_t* __restrict__ y, int64_t T,
                                                          int k, int64_t chunks_per_row) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= T * chunks_per_row) return;
  const int64_t t = idx / chunks_per_row;
  const int64_t cc = idx % chunks_per_row;
  const int64_t H = chunks_per_row * 8;
  v4i rows[KMAX];
#pragma unroll
  for (int i = 0; i < KMAX; ++i)
    if (i < k) rows[i] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(D + (t * k + i) * H + cc * 8));
  v4i add = {0, 0, 0, 0};
  if constexpr (ADD) add = *reinterpret_cast<const v4i*>(addend + t * H + cc * 8);
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < KMAX; ++i) {
    if (i < k) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t w = (uint32_t)rows[i][j];
        acc[2 * j] += __uint_as_float(w << 16);
        acc[2 * j + 1] += __uint_as_float(w & 0xFFFF0000u);
      }
    }
  }
  v4i out;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t lo = f32_to_bf16_bits(acc[2 * j]), hi = f32_to_bf16_bits(acc[2 * j + 1]);
    if constexpr (ADD) {
      const uint32_t a = (uint32_t)add[j];
      lo = f32_to_bf16_bits(bf16_to_f32(lo) + lo_bf16(a));
      hi = f32_to_bf16_bits(bf16_to_f32(hi) + hi_bf16(a));
    }
    out[j] = (int)(lo | (hi << 16));
  }
  __builtin_nontemporal_store(out, reinterpret_cast<v4i*>(y + t * H + cc * 8));
}

constexpr int kMaxRanks = 64;
constexpr int kDequantBatch = 8;

__global__ __launch_bounds__(256) void fp8_dequant_sum_kernel(const uint8_t* __restrict__ q,
                                                              const float* __restrict__ s,
                                                              uint16_t* __restrict__ out, int R,
                                                              int64_t M, int64_t N, int64_t scale_ld,
                                                              int64_t out_ld) {
#pragma clang fp contract(off)
  const int64_t cpr = N / 16;  // 16-column chunks per row
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= M * cpr) return;
  const int64_t m = idx / cpr, c = idx % cpr;
  const int64_t grp = c / 8;  // 128-column scale group of the chunk
  float acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
  for (int r0 = 0; r0 < R; r0 += kDequantBatch) {
    v4i qv[kDequantBatch];
    float sc[kDequantBatch];
#pragma unroll
    for (int b = 0; b < kDequantBatch; ++b) {
      if (r0 + b < R) {
        const int64_t row = (int64_t)(r0 + b) * M + m;
        qv[b] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(q + row * N + c * 16));
        sc[b] = s[row * scale_ld + grp];
      }
    }
#pragma unroll
    for (int b = 0; b < kDequantBatch; ++b) {
      if (r0 + b < R) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int word = qv[b][w];
          const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(word, false);  // bytes 0, 1
          const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(word, true);   // bytes 2, 3
          acc[4 * w + 0] = acc[4 * w + 0] + lo[0] * sc[b];
          acc[4 * w + 1] = acc[4 * w + 1] + lo[1] * sc[b];
          acc[4 * w + 2] = acc[4 * w + 2] + hi[0] * sc[b];
          acc[4 * w + 3] = acc[4 * w + 3] + hi[1] * sc[b];
        }
      }
    }
  }
  v4i o0, o1;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    o0[w] = (int)pack_bf16x2(acc[2 * w], acc[2 * w + 1]);
    o1[w] = (int)pack_bf16x2(acc[8 + 2 * w], acc[8 + 2 * w + 1]);
  }
  uint16_t* dst = out + m * out_ld + c * 16;
  __builtin_nontemporal_store(o0, reinterpret_cast<v4i*>(dst));
  __builtin_nontemporal_store(o1, reinterpret_cast<v4i*>(dst + 8));
}

__global__ __launch_bounds__(256) void silu_and_mul_kernel(const uint16_t* __restrict__ c,
                                                           uint16_t* __restrict__ h, int64_t R,
                                                           int64_t I) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t chunks = I / 8;
  if (idx >= R * chunks) return;
  const int64_t r = idx / chunks, cc = idx % chunks;
  const v4i gv = *reinterpret_cast<const v4i*>(c + r * 2 * I + cc * 8);
  const v4i uv = *reinterpret_cast<const v4i*>(c + r * 2 * I + I + cc * 8);
  v4i out;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t gw = (uint32_t)gv[j], uw = (uint32_t)uv[j];
    const float h0 = silu_mul_bf16(lo_bf16(gw), lo_bf16(uw));
    const float h1 = silu_mul_bf16(hi_bf16(gw), hi_bf16(uw));
    out[j] = (int)pack_bf16x2(h0, h1);
  }
  *reinterpret_cast<v4i*>(h + r * I + cc * 8) = out;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }  // null passes



static int launch_reduce(const void* D_bf16, const void* addend, int64_t T, int32_t top_k,
                         int64_t H, void* y, void* stream) {
  if (T < 0 || H < 0) return kErrBadShape;
  if (top_k <= 0 || top_k > kMaxTopK) return kErrBadTopK;
  if (T == 0 || H == 0) return kOk;
  if (!D_bf16 || !y) return kErrNullPointer;
  if (H % 8 != 0 || !aligned16(D_bf16) || !aligned16(y) || !aligned16(addend)) return kErrBadShape;
  const int64_t cpr = H / 8;
  const int64_t blocks = (T * cpr + 255) / 256;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* d = (const uint16_t*)D_bf16;
  const uint16_t* a = (const uint16_t*)addend;
  uint16_t* out = (uint16_t*)y;
  const dim3 grid((unsigned)blocks);
  if (top_k <= 8) {
    if (a)
      hipLaunchKernelGGL((reduce_topk_kernel<8, true>), grid, dim3(256), 0, st, d, a, out, T, (int)top_k, cpr);
    else
      hipLaunchKernelGGL((reduce_topk_kernel<8, false>), grid, dim3(256), 0, st, d, a, out, T, (int)top_k, cpr);
  } else {
    if (a)
      hipLaunchKernelGGL((reduce_topk_kernel<kMaxTopK, true>), grid, dim3(256), 0, st, d, a, out, T,
                         (int)top_k, cpr);
    else
      hipLaunchKernelGGL((reduce_topk_kernel<kMaxTopK, false>), grid, dim3(256), 0, st, d, a, out, T,
                         (int)top_k, cpr);
  }
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // namespace moe

using namespace moe;

extern "C" int moe_reduce_topk(const void* D_bf16, int64_t T, int32_t top_k, int64_t H, void* y,
                               void* stream) {
  return launch_reduce(D_bf16, nullptr, T, top_k, H, y, stream);
}

extern "C" int moe_reduce_topk_add(const void* D_bf16, const void* addend_bf16, int64_t T,
                                   int32_t top_k, int64_t H, void* y, void* stream) {
  if (T > 0 && H > 0 && !addend_bf16) return kErrNullPointer;
  return launch_reduce(D_bf16, addend_bf16, T, top_k, H, y, stream);
}

extern "C" int moe_silu_and_mul(const void* c_bf16, int64_t R, int64_t I, void* h_bf16,
                                void* stream) {
  if (R < 0 || I < 0) return kErrBadShape;
  if (R == 0 || I == 0) return kOk;
  if (!c_bf16 || !h_bf16) return kErrNullPointer;
  if (I % 8 != 0 || !aligned16(c_bf16) || !aligned16(h_bf16)) return kErrBadShape;
  const int64_t blocks = (R * (I / 8) + 255) / 256;
  hipLaunchKernelGGL(silu_and_mul_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)c_bf16, (uint16_t*)h_bf16, R, I);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

extern "C" int moe_fp8_dequant_sum(const void* q_fp8, const float* scales, int64_t R, int64_t M, int64_t N,
                                   int64_t scale_ld, void* out_bf16, int64_t out_ld, void* stream) {
  if (R < 1 || R > kMaxRanks || M < 0 || N < 0) return kErrBadShape;
  if (M == 0 || N == 0) return kOk;
  if (!q_fp8 || !scales || !out_bf16) return kErrNullPointer;
  if (N % 16 != 0 || scale_ld < (N + 127) / 128 || out_ld < N || out_ld % 8 != 0) return kErrBadShape;
  if (!aligned16(q_fp8) || !aligned16(out_bf16)) return kErrBadShape;
  const int64_t blocks = (M * (N / 16) + 255) / 256;
  hipLaunchKernelGGL(fp8_dequant_sum_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t*)q_fp8, scales, (uint16_t*)out_bf16, (int)R, M, N, scale_ld, out_ld);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}
