// A5 / A6 / A7 / A8: ragged, 128x128 block-scaled FP8 grouped GEMM on CDNA4
// FP8 MFMA (v_mfma_f32_16x16x128_f8f6f4, OCP e4m3 operands).
//
// Semantics follow the reference's in-repo copy of vLLM's fused_moe_kernel
// (moe_bench/overlap/kernels.py:95-214):
//   for block b with expert e = expert_ids[b] (e == -1 -> zeros, :112-120),
//   for every position p of the block with slot s = sorted_ids[p] < S:
//     row  = a_by_pos ? p : s / top_k                          (:124-126)
//     acc  = sum_kb dot128(A[row, kb], B[e, n, kb]) * a_s[row, kb] * b_s[e, n/128, kb]
//                                                              (:162-188)
//     acc *= topk_w[s] if routed weights are applied           (:192-194)
//     C[s, n] = bf16(acc)                                      (:198-210)
// The fused W13 variant keeps gate columns [j*128, j*128+128) and up columns
// [I + j*128, ...) of the same workgroup, and finishes in the epilogue with
// SiLU*up (overlap_forward.py:277-279, rounding C to bf16 and h to bf16 as the
// unfused chain does) and the 1x128 quant of h (overlap_forward.py:282-284),
// writing FP8 codes + scales by sorted position so that W2 reads its A rows
// contiguously.
//
// Tiling (one workgroup = 4 waves = 256 threads, one expert block of BM rows,
// 256 B-rows = two 128-row scale groups, K step 128 = one scale block):
//   * every K step is exactly one 16x16x128 MFMA per 16x16 output subtile,
//     started from a zero accumulator, so the per-block scales are applied as
//     acc = fma(partial, a_s[row] * b_s[group], acc) -- no second accumulator;
//   * A (gathered rows) and B tiles are double-buffered in LDS (BM*128 +
//     256*128 bytes per stage), 16-byte chunks XOR-swizzled by row so that the
//     MFMA fragment reads (two ds_read_b128 per lane) are bank-conflict free;
//   * a lane's fragment is 32 contiguous K bytes of one row; A and B use the
//     same K placement, so the contraction is independent of how the hardware
//     orders K inside the instruction;
//   * the launch is XCD-aware: workgroup ids are dealt round-robin to the 8
//     XCDs, so consecutive ids on one XCD are mapped to the n-tiles of a small
//     group of consecutive M blocks (same expert), which then share their A rows
//     and weight tiles in that XCD's L2.
#include "common.hpp"

namespace moe {

constexpr int kGemmThreads = 256;
constexpr int kXcds = 8;
constexpr int kGroupM = 2;  // consecutive M blocks sharing an XCD's L2

template <int BM>
struct Tile {
  static constexpr int WM = (BM == 128) ? 2 : 1;  // waves along M
  static constexpr int WN = 4 / WM;               // waves along N
  static constexpr int RS = BM / WM / 16;         // 16-row subtiles per wave
  static constexpr int CS = 8 / WN;               // 16-col subtiles per wave per group
  static constexpr int A_BYTES = BM * 128;
  static constexpr int B_BYTES = 256 * 128;
  static constexpr int A_CHUNKS = BM * 8;
  static constexpr int A_PER_THREAD = (A_CHUNKS + kGemmThreads - 1) / kGemmThreads;
  static constexpr int B_PER_THREAD = 256 * 8 / kGemmThreads;
  // LDS carve-up: [A0 A1][B0 B1][sa0 sa1][sb0 sb1 (2 floats each)][row amax WN*BM]
  static constexpr int OFF_B = 2 * A_BYTES;
  static constexpr int OFF_SA = OFF_B + 2 * B_BYTES;
  static constexpr int OFF_SB = OFF_SA + 2 * BM * 4;
  static constexpr int OFF_RED = OFF_SB + 16;
  static constexpr int LDS_BYTES = OFF_RED + WN * BM * 4;
  static_assert(BM * 512 <= OFF_SA, "bf16 output staging must fit in the operand buffers");
};

struct GemmArgs {
  const uint8_t* A;        // fp8 [rows, K]
  const float* As;         // [rows, K/128]
  const uint8_t* B;        // fp8 [E, N, K]
  const float* Bs;         // [E, N/128, K/128]
  const int32_t* sorted;   // [max_padded]
  const int32_t* eids;     // [max_blocks]
  const int32_t* ntpp;     // [1]
  const float* topk_w;     // [S] or null
  uint16_t* C;             // bf16 [S, N]            (plain epilogue)
  uint8_t* hq;             // fp8 [max_padded, I]    (fused epilogue)
  float* hs;               // [max_padded, I/128]    (fused epilogue)
  int64_t S;
  int64_t N;
  int64_t K;
  int64_t I;
  int64_t max_blocks;
  int64_t n_tiles;
  int top_k;
  int a_by_pos;
  int E;
};

MOE_DEVICE int swz(int row) { return (row ^ (row >> 3)) & 7; }

MOE_DEVICE v8i lds_frag(const uint8_t* tile, int row, int kseg) {
  const int sw = swz(row);
  const v4i x = *reinterpret_cast<const v4i*>(tile + row * 128 + (((2 * kseg) ^ sw) << 4));
  const v4i y = *reinterpret_cast<const v4i*>(tile + row * 128 + (((2 * kseg + 1) ^ sw) << 4));
  return (v8i){x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
}

MOE_DEVICE v4f mfma_fp8(v8i a, v8i b) {
  const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, zero, 0, 0, 0, 0, 0, 0);
}

template <int BM, bool FUSED>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void grouped_gemm_kernel(GemmArgs g) {
  using T = Tile<BM>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* smA = smem;
  uint8_t* smB = smem + T::OFF_B;
  float* smSA = reinterpret_cast<float*>(smem + T::OFF_SA);
  float* smSB = reinterpret_cast<float*>(smem + T::OFF_SB);
  float* smRed = reinterpret_cast<float*>(smem + T::OFF_RED);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / T::WN;
  const int wn = wave % T::WN;

  // ---- XCD-aware tile mapping -------------------------------------------
  const int64_t pid = blockIdx.x;
  const int64_t xcd = pid % kXcds;
  const int64_t li = pid / kXcds;
  const int64_t per_group = (int64_t)kGroupM * g.n_tiles;
  const int64_t mgl = li / per_group;
  const int64_t within = li % per_group;
  const int64_t j = within / kGroupM;
  const int64_t b = (mgl * kXcds + xcd) * kGroupM + within % kGroupM;
  if (b >= g.max_blocks) return;
  const int ntpp = *g.ntpp;
  if (b * BM >= ntpp) return;
  const int e = g.eids[b];
  const int64_t K = g.K;
  const int64_t KB = K / 128;
  const int64_t NBt = g.N / 128;
  int64_t g0, g1;
  bool g1_store = true;
  if (FUSED) {
    g0 = j;
    g1 = g.I / 128 + j;
  } else {
    g0 = 2 * j;
    g1 = 2 * j + 1;
    if (g1 >= NBt) {
      g1 = NBt - 1;
      g1_store = false;
    }
  }

  if (e < 0 || e >= g.E) {
    // Expert not local: zero output rows (kernels.py:112-120).
    if (FUSED) {
      const int64_t hcols = g.I;
      for (int ci = tid; ci < BM * 8; ci += kGemmThreads) {
        const int row = ci >> 3, cc = ci & 7;
        *reinterpret_cast<v4i*>(g.hq + (b * BM + row) * hcols + j * 128 + cc * 16) =
            (v4i){0, 0, 0, 0};
      }
      for (int row = tid; row < BM; row += kGemmThreads)
        g.hs[(b * BM + row) * (g.I / 128) + j] = kScaleFloor;
    } else {
      for (int ci = tid; ci < BM * 32; ci += kGemmThreads) {
        const int row = ci >> 5, cc = ci & 31;
        const int64_t slot = g.sorted[b * BM + row];
        if (slot >= g.S) continue;
        const int grp = (cc * 8) >> 7;
        if (grp == 1 && !g1_store) continue;
        const int64_t n = (grp ? g1 : g0) * 128 + ((cc * 8) & 127);
        *reinterpret_cast<v4i*>(g.C + slot * g.N + n) = (v4i){0, 0, 0, 0};
      }
    }
    return;
  }

  // ---- per-thread global source pointers ---------------------------------
  const uint8_t* a_src[T::A_PER_THREAD];
  int a_dst[T::A_PER_THREAD];
#pragma unroll
  for (int i = 0; i < T::A_PER_THREAD; ++i) {
    const int ci = tid + i * kGemmThreads;
    const int row = (ci < T::A_CHUNKS) ? (ci >> 3) : 0;
    const int cc = ci & 7;
    const int64_t pos = b * BM + row;
    int64_t arow;
    if (g.a_by_pos) {
      arow = pos;
    } else {
      const int64_t slot = g.sorted[pos];
      arow = (slot < g.S) ? slot / g.top_k : 0;
    }
    a_src[i] = g.A + arow * K + cc * 16;
    a_dst[i] = row * 128 + ((cc ^ swz(row)) << 4);
  }
  const float* sa_src = g.As;
  if (tid < BM) {
    const int64_t pos = b * BM + tid;
    int64_t arow;
    if (g.a_by_pos) {
      arow = pos;
    } else {
      const int64_t slot = g.sorted[pos];
      arow = (slot < g.S) ? slot / g.top_k : 0;
    }
    sa_src = g.As + arow * KB;
  }
  const float* sb_src = g.Bs + ((int64_t)e * NBt + (tid == 0 ? g0 : g1)) * KB;
  // B rows: chunk ci = tid + i*256 -> row r = (tid>>3) + 32*i, col chunk tid&7.
  const int b_row0 = tid >> 3;
  const int b_cc = tid & 7;
  const uint8_t* b_src0 = g.B + ((int64_t)e * g.N + g0 * 128 + b_row0) * K + b_cc * 16;
  const uint8_t* b_src1 = g.B + ((int64_t)e * g.N + g1 * 128 + b_row0) * K + b_cc * 16;
  int b_dst[T::B_PER_THREAD];
#pragma unroll
  for (int i = 0; i < T::B_PER_THREAD; ++i) {
    const int r = b_row0 + 32 * i;
    b_dst[i] = r * 128 + ((b_cc ^ swz(r)) << 4);
  }

  v4i ra[T::A_PER_THREAD];
  v4i rb[T::B_PER_THREAD];
  float rsa = 0.0f, rsb = 0.0f;

  auto load_tile = [&](int64_t kk) {
#pragma unroll
    for (int i = 0; i < T::A_PER_THREAD; ++i)
      if (tid + i * kGemmThreads < T::A_CHUNKS)
        ra[i] = *reinterpret_cast<const v4i*>(a_src[i] + kk * 128);
#pragma unroll
    for (int i = 0; i < T::B_PER_THREAD; ++i) {
      const uint8_t* src = (i < 4) ? b_src0 + (int64_t)(32 * i) * K
                                   : b_src1 + (int64_t)(32 * (i - 4)) * K;
      rb[i] = *reinterpret_cast<const v4i*>(src + kk * 128);
    }
    if (tid < BM) rsa = sa_src[kk];
    if (tid < 2) rsb = sb_src[kk];
  };
  auto store_tile = [&](int buf) {
    uint8_t* dA = smA + buf * T::A_BYTES;
    uint8_t* dB = smB + buf * T::B_BYTES;
#pragma unroll
    for (int i = 0; i < T::A_PER_THREAD; ++i)
      if (tid + i * kGemmThreads < T::A_CHUNKS) *reinterpret_cast<v4i*>(dA + a_dst[i]) = ra[i];
#pragma unroll
    for (int i = 0; i < T::B_PER_THREAD; ++i) *reinterpret_cast<v4i*>(dB + b_dst[i]) = rb[i];
    if (tid < BM) smSA[buf * BM + tid] = rsa;
    if (tid < 2) smSB[buf * 2 + tid] = rsb;
  };

  v4f acc[T::RS][2][T::CS];
#pragma unroll
  for (int r = 0; r < T::RS; ++r)
#pragma unroll
    for (int gg = 0; gg < 2; ++gg)
#pragma unroll
      for (int c = 0; c < T::CS; ++c) acc[r][gg][c] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};

  const int row_base = wm * T::RS * 16;
  const int col_base = wn * T::CS * 16;
  const int frag_row = lane & 15;
  const int kseg = lane >> 4;

  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int64_t kk = 0; kk < KB; ++kk) {
    const int cur = (int)(kk & 1);
    if (kk + 1 < KB) load_tile(kk + 1);
    const uint8_t* tA = smA + cur * T::A_BYTES;
    const uint8_t* tB = smB + cur * T::B_BYTES;
    v8i af[T::RS];
    float sab[T::RS][2][4];
    const float sb0 = smSB[cur * 2 + 0];
    const float sb1 = smSB[cur * 2 + 1];
#pragma unroll
    for (int r = 0; r < T::RS; ++r) {
      af[r] = lds_frag(tA, row_base + r * 16 + frag_row, kseg);
      const v4f sa4 =
          *reinterpret_cast<const v4f*>(smSA + cur * BM + row_base + r * 16 + 4 * kseg);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        sab[r][0][v] = sa4[v] * sb0;
        sab[r][1][v] = sa4[v] * sb1;
      }
    }
#pragma unroll
    for (int gg = 0; gg < 2; ++gg) {
#pragma unroll
      for (int c = 0; c < T::CS; ++c) {
        const v8i bf = lds_frag(tB, gg * 128 + col_base + c * 16 + frag_row, kseg);
#pragma unroll
        for (int r = 0; r < T::RS; ++r) {
          const v4f p = mfma_fp8(af[r], bf);
#pragma unroll
          for (int v = 0; v < 4; ++v)
            acc[r][gg][c][v] = __builtin_fmaf(p[v], sab[r][gg][v], acc[r][gg][c][v]);
        }
      }
    }
    if (kk + 1 < KB) store_tile(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogues ----------------------------------------------------------
  // Output element (r, gg, c, v) of this lane: row = row_base + r*16 + 4*kseg + v,
  // column (within group gg) = col_base + c*16 + frag_row.
  if constexpr (FUSED) {
    float pmax[T::RS][4];
#pragma unroll
    for (int r = 0; r < T::RS; ++r)
#pragma unroll
      for (int v = 0; v < 4; ++v) pmax[r][v] = 0.0f;
#pragma unroll
    for (int r = 0; r < T::RS; ++r)
#pragma unroll
      for (int c = 0; c < T::CS; ++c)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float cg = round_bf16(acc[r][0][c][v]);
          const float cu = round_bf16(acc[r][1][c][v]);
          const float h = round_bf16(cg / (1.0f + __expf(-cg)) * cu);
          acc[r][0][c][v] = h;
          pmax[r][v] = fmaxf(pmax[r][v], fabsf(h));
        }
#pragma unroll
    for (int r = 0; r < T::RS; ++r)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float m = pmax[r][v];
        m = fmaxf(m, __shfl_xor(m, 1));
        m = fmaxf(m, __shfl_xor(m, 2));
        m = fmaxf(m, __shfl_xor(m, 4));
        m = fmaxf(m, __shfl_xor(m, 8));
        if (frag_row == 0) smRed[wn * BM + row_base + r * 16 + 4 * kseg + v] = m;
      }
    __syncthreads();
    uint8_t* stage = smem;  // [BM][128] fp8 codes
    const int64_t hgroups = g.I / 128;
#pragma unroll
    for (int r = 0; r < T::RS; ++r)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = row_base + r * 16 + 4 * kseg + v;
        float amax = 0.0f;
#pragma unroll
        for (int w = 0; w < T::WN; ++w) amax = fmaxf(amax, smRed[w * BM + row]);
        const float sc = group_scale(amax);
        const float inv = 1.0f / sc;
        if (wn == 0 && frag_row == 0) g.hs[(b * BM + row) * hgroups + j] = sc;
#pragma unroll
        for (int c = 0; c < T::CS; c += 2) {
          // two columns per cvt; columns differ by 16 so write bytes separately
          const float q0 = clamp_fp8(div_by(acc[r][0][c][v], sc, inv));
          const float q1 = clamp_fp8(div_by(acc[r][0][c + 1][v], sc, inv));
          const uint32_t pk = pack4_e4m3(q0, q1, 0.0f, 0.0f);
          stage[row * 128 + col_base + c * 16 + frag_row] = (uint8_t)(pk & 0xFF);
          stage[row * 128 + col_base + (c + 1) * 16 + frag_row] = (uint8_t)((pk >> 8) & 0xFF);
        }
      }
    __syncthreads();
    for (int ci = tid; ci < BM * 8; ci += kGemmThreads) {
      const int row = ci >> 3, cc = ci & 7;
      *reinterpret_cast<v4i*>(g.hq + (b * BM + row) * g.I + j * 128 + cc * 16) =
          *reinterpret_cast<const v4i*>(stage + row * 128 + cc * 16);
    }
  } else {
    uint16_t* stage = reinterpret_cast<uint16_t*>(smem);  // [BM][256] bf16
#pragma unroll
    for (int r = 0; r < T::RS; ++r)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = row_base + r * 16 + 4 * kseg + v;
        float w = 1.0f;
        if (g.topk_w) {
          const int64_t slot = g.sorted[b * BM + row];
          if (slot < g.S) w = g.topk_w[slot];
        }
#pragma unroll
        for (int gg = 0; gg < 2; ++gg)
#pragma unroll
          for (int c = 0; c < T::CS; ++c) {
            float val = acc[r][gg][c][v];
            if (g.topk_w) val = val * w;
            stage[row * 256 + gg * 128 + col_base + c * 16 + frag_row] =
                (uint16_t)f32_to_bf16_bits(val);
          }
      }
    __syncthreads();
    for (int ci = tid; ci < BM * 32; ci += kGemmThreads) {
      const int row = ci >> 5, cc = ci & 31;
      const int64_t slot = g.sorted[b * BM + row];
      if (slot >= g.S) continue;
      const int grp = cc >> 4;
      if (grp == 1 && !g1_store) continue;
      const int64_t n = (grp ? g1 : g0) * 128 + (cc & 15) * 8;
      *reinterpret_cast<v4i*>(g.C + slot * g.N + n) =
          *reinterpret_cast<const v4i*>(stage + row * 256 + cc * 8);
    }
  }
}

template <int BM, bool FUSED>
static int launch_gemm(const GemmArgs& args, hipStream_t st) {
  using T = Tile<BM>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)grouped_gemm_kernel<BM, FUSED>,
                            hipFuncAttributeMaxDynamicSharedMemorySize,
                            T::LDS_BYTES) != hipSuccess)
      return kErrLaunch;
    attr_set = true;
  }
  const int64_t n_groups = (args.max_blocks + kGroupM - 1) / kGroupM;
  const int64_t grid = (n_groups + kXcds - 1) / kXcds * kXcds * kGroupM * args.n_tiles;
  if (grid <= 0) return kOk;
  hipLaunchKernelGGL((grouped_gemm_kernel<BM, FUSED>), dim3((unsigned)grid), dim3(kGemmThreads),
                     T::LDS_BYTES, st, args);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

template <bool FUSED>
static int dispatch_gemm(int BM, const GemmArgs& args, hipStream_t st) {
  switch (BM) {
    case 16: return launch_gemm<16, FUSED>(args, st);
    case 32: return launch_gemm<32, FUSED>(args, st);
    case 64: return launch_gemm<64, FUSED>(args, st);
    case 128: return launch_gemm<128, FUSED>(args, st);
    default: return kErrBadBlockSize;
  }
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace moe

using namespace moe;

extern "C" int moe_grouped_gemm(const void* A, const float* A_scale, const void* B,
                                const float* B_scale, const int32_t* sorted_ids,
                                const int32_t* expert_ids, const int32_t* ntpp,
                                const float* topk_weights, int64_t S, int32_t top_k,
                                int32_t a_by_pos, int64_t N, int64_t K, int32_t E, int32_t BM,
                                int64_t max_padded, void* C, void* stream) {
  if (S < 0 || N <= 0 || K <= 0 || max_padded < 0) return kErrBadShape;
  if (N % 128 != 0 || K % 128 != 0) return kErrBadShape;
  if (top_k <= 0) return kErrBadTopK;
  if (E <= 0) return kErrBadExperts;
  if (BM != 16 && BM != 32 && BM != 64 && BM != 128) return kErrBadBlockSize;
  if (max_padded == 0 || S == 0) return kOk;
  if (!A || !A_scale || !B || !B_scale || !sorted_ids || !expert_ids || !ntpp || !C)
    return kErrNullPointer;
  if (!aligned16(A) || !aligned16(B) || !aligned16(C)) return kErrBadShape;
  GemmArgs g{};
  g.A = (const uint8_t*)A;
  g.As = A_scale;
  g.B = (const uint8_t*)B;
  g.Bs = B_scale;
  g.sorted = sorted_ids;
  g.eids = expert_ids;
  g.ntpp = ntpp;
  g.topk_w = topk_weights;
  g.C = (uint16_t*)C;
  g.S = S;
  g.N = N;
  g.K = K;
  g.I = 0;
  g.max_blocks = (max_padded + BM - 1) / BM;
  g.n_tiles = (N / 128 + 1) / 2;
  g.top_k = top_k;
  g.a_by_pos = a_by_pos ? 1 : 0;
  g.E = E;
  return dispatch_gemm<false>(BM, g, (hipStream_t)stream);
}

extern "C" int moe_gemm_w13_silu_quant(const void* Aq, const float* A_scale, const void* W13,
                                       const float* W13_scale, const int32_t* sorted_ids,
                                       const int32_t* expert_ids, const int32_t* ntpp, int64_t S,
                                       int32_t top_k, int64_t H, int64_t I, int32_t E,
                                       int32_t BM, int64_t max_padded, void* hq, float* hs,
                                       void* stream) {
  if (S < 0 || H <= 0 || I <= 0 || max_padded < 0) return kErrBadShape;
  if (H % 128 != 0 || I % 128 != 0) return kErrBadShape;
  if (top_k <= 0) return kErrBadTopK;
  if (E <= 0) return kErrBadExperts;
  if (BM != 16 && BM != 32 && BM != 64 && BM != 128) return kErrBadBlockSize;
  if (max_padded == 0 || S == 0) return kOk;
  if (!Aq || !A_scale || !W13 || !W13_scale || !sorted_ids || !expert_ids || !ntpp || !hq || !hs)
    return kErrNullPointer;
  if (!aligned16(Aq) || !aligned16(W13) || !aligned16(hq)) return kErrBadShape;
  GemmArgs g{};
  g.A = (const uint8_t*)Aq;
  g.As = A_scale;
  g.B = (const uint8_t*)W13;
  g.Bs = W13_scale;
  g.sorted = sorted_ids;
  g.eids = expert_ids;
  g.ntpp = ntpp;
  g.topk_w = nullptr;
  g.hq = (uint8_t*)hq;
  g.hs = hs;
  g.S = S;
  g.N = 2 * I;
  g.K = H;
  g.I = I;
  g.max_blocks = (max_padded + BM - 1) / BM;
  g.n_tiles = I / 128;
  g.top_k = top_k;
  g.a_by_pos = 0;
  g.E = E;
  return dispatch_gemm<true>(BM, g, (hipStream_t)stream);
}

// Layout probe: one wave computes C[16][16] = A[16][128] . B[16][128]^T through
// the same fragment loader and MFMA call as the GEMM, reading A/B through LDS
// with the GEMM's swizzle and writing C with the GEMM's output mapping.
__global__ void mfma_probe_kernel(const uint8_t* A, const uint8_t* B, float* C) {
  __shared__ __attribute__((aligned(16))) uint8_t sA[16 * 128];
  __shared__ __attribute__((aligned(16))) uint8_t sB[16 * 128];
  const int lane = threadIdx.x;
  for (int ci = lane; ci < 128; ci += 64) {
    const int row = ci >> 3, cc = ci & 7;
    *reinterpret_cast<v4i*>(sA + row * 128 + ((cc ^ swz(row)) << 4)) =
        *reinterpret_cast<const v4i*>(A + row * 128 + cc * 16);
    *reinterpret_cast<v4i*>(sB + row * 128 + ((cc ^ swz(row)) << 4)) =
        *reinterpret_cast<const v4i*>(B + row * 128 + cc * 16);
  }
  __syncthreads();
  const v4f p = mfma_fp8(lds_frag(sA, lane & 15, lane >> 4), lds_frag(sB, lane & 15, lane >> 4));
  for (int v = 0; v < 4; ++v) C[(4 * (lane >> 4) + v) * 16 + (lane & 15)] = p[v];
}

extern "C" int moe_debug_mfma_probe(const void* A, const void* B, float* C, void* stream) {
  if (!A || !B || !C) return kErrNullPointer;
  if (!aligned16(A) || !aligned16(B)) return kErrBadShape;
  hipLaunchKernelGGL(mfma_probe_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     (const uint8_t*)A, (const uint8_t*)B, C);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}
