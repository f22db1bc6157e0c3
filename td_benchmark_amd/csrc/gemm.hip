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
// [I + j*128, ...) in the same workgroup and finishes in the epilogue with
// SiLU*up (overlap_forward.py:277-279; C rounded to bf16 and h rounded to bf16
// as the unfused chain does) and the 1x128 quant of h (overlap_forward.py:
// 282-284), writing FP8 codes + scales by sorted position so that the W2 GEMM
// reads its A rows contiguously.
//
// Tiling: one workgroup computes TM rows x 256 B-rows (two 128-row scale
// groups).  TM is block_size_m, or 256 when the experts average at least 160
// slots: a 256-row tile then spans consecutive align blocks of one expert,
// split evenly over the expert's tiles, so a weight tile is fetched once per
// up to 256 rows.  8 waves (2 per SIMD, so one wave's MFMAs run while the other
// waits on LDS or the barrier) for TM >= 32, 4 for TM = 16; at TM = 256 they
// are 4 x 2 waves of 64 x 128.  TM = 32 runs two workgroups per CU.  The K step is 128 = one scale block, and every
// K step is exactly one 16x16x128 MFMA per 16x16 output subtile started from
// zero, so the per-block scales are applied as acc = fma(partial,
// a_s[row]*b_s[group], acc) (kScaleLag MFMAs later) with no second
// accumulator.  The fp32 promotion at every 128-K block also bounds the matrix
// core's reduced-precision accumulation inside one instruction.  16-row
// subtiles that hold only padding rows issue no MFMA at all, and a tile with
// at most kTailRows valid rows runs a kTailRows-row body (in a 256-row launch,
// a tile with at most 128 valid rows runs the 128-row body).
//
// Pipeline: operand tiles go to LDS by direct-to-LDS loads
// (global_load_lds_dwordx4: each lane moves 16 B from its own global address
// -- a gathered A row -- straight into LDS, no VGPR staging; addresses are a
// uniform base plus a fixed 32-bit lane offset).  For TM = 64 and 128 a 3-stage
// ring (A TM*128 B + B 32 KiB per stage, plus the A scales): step k waits until
// only step k+1's loads are in flight, passes one barrier, issues step k+2's
// loads into the buffer freed at step k-1, then computes.  TM = 16 (a
// weight-streaming decode tile) keeps a 4-stage ring, two younger stages in
// flight.  At TM = 256 three 64 KiB stages exceed the LDS, so the ring has two
// stages and every step waits for all of its loads; A rows of subtiles without
// a valid row are then not fetched.  TM = 32 (the default decode tile) also
// has two stages, in two workgroups per CU that stream independently.  The activation scales of a stage are one
// 4-byte direct-to-LDS load per row: from the row's own scale row, or -- when
// they are laid out K-major by sorted position (as_pos_ld) -- one contiguous
// run of the tile's rows per K block.  The weight scales of the tile (both
// groups, every K block) arrive by direct-to-LDS loads before stage 0.  All
// direct-to-LDS loads are issued from inline asm (see dma16), weight rows
// before A rows, at raised wave priority.  In 16- and 32-row launches, the
// weight loads of an expert with a single row tile carry the non-temporal
// hint: that tile is the only reader of its weight tiles.
//
// The MFMA takes the weight fragment as its first operand and the activation
// fragment as its second, so the four results of a lane are four consecutive
// columns of one token: a K step needs one scale product a_s * b_s per 16-row
// subtile and group (not one per row), and the epilogue stages a lane's
// results with one 4- or 8-byte LDS write.
//
// LDS rows are 128 B; the 16 B chunk index of a row is XORed with
// swz(row) = (row mod 8) ^ bit3(row), which depends only on the row's
// position inside its 16-row MFMA subtile.  A fragment read (lane = row fr,
// K segment kseg: 32 contiguous K bytes = two ds_read_b128) is therefore one of
// two per-lane base addresses plus a compile-time offset for every subtile,
// and the 8 / 16 lanes serviced together hit distinct banks.  The swizzle is
// applied on the global side (lane L of a DMA instruction fetches the logical
// chunk that belongs at its LDS slot).  A and B use the same K placement, so
// the contraction does not depend on how the hardware orders K inside the
// instruction.
//
// Launch: workgroup ids are dealt round-robin to the 8 XCDs; the id -> tile map
// gives each XCD a contiguous range of an expert-major tile order, so all row
// tiles of one expert that read the same weight tile run together on one
// XCD (weights leave HBM once) and a row tile's A rows are shared by its
// n-tiles in that XCD's L2.
#include <type_traits>

#include "common.hpp"
#include "mfma_frag.hpp"

#define MOE_LDS(p) ((__attribute__((address_space(3))) void*)(p))

namespace moe {

constexpr int kXcds = 8;
constexpr int kMaxKB = 128;  // K <= 16384
constexpr int kTailRows = 64;  // row tiles with at most this many valid rows run the short body
// Plain launches with K of at least this many columns order the tiles of an
// n-tile group column-major (Mixtral's W2, K = 14336: 1-3 % faster; W13 of
// every shape and the W2 of DeepSeek-V3 and Qwen3, K <= 7168, lose 1-7 % that
// way).
constexpr int64_t kColMajorK = 8192;
// MFMAs issued between an MFMA and the FMAs that scale its result: the VALU
// reads a result that is complete, without hazard waits.
constexpr int kScaleLag = 2;

template <int BM>
struct Tile {
  static constexpr int NW = BM >= 32 ? 8 : 4;     // waves per workgroup (2 per SIMD at 8)
  static constexpr int THREADS = 64 * NW;
  // waves along M: 4 x 2 waves of 64 x 128 at BM = 256 (fewer LDS bytes per MFMA)
  static constexpr int WM = BM == 256 ? 4 : ((NW == 8 || BM == 128) ? 2 : 1);
  // LDS ring depth: three 64 KiB stages of the 256-row tile exceed 160 KiB;
  // the 34 KiB stages of the 16-row tile (weight streaming) fit four; the
  // 32-row tile runs two workgroups per CU with two 36 KiB stages each, so one
  // workgroup's pipeline fill and epilogue overlap the other's weight stream
  static constexpr int KS = (BM == 256 || BM == 32) ? 2 : (BM == 16 ? 4 : 3);
  static constexpr int WG_PER_CU = BM == 32 ? 2 : 1;
  static constexpr int WN = NW / WM;              // waves along N
  static constexpr int RS = BM / WM / 16;         // 16-row subtiles per wave
  static constexpr int CS = 8 / WN;               // 16-col subtiles per wave per group
  static constexpr int A_BYTES = BM * 128;
  static constexpr int B_BYTES = 256 * 128;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int NA = BM / 8;               // 1 KiB A DMA instructions per stage
  static constexpr int NB = 32;                   // 1 KiB B DMA instructions per stage
  static constexpr int NS = (BM + 63) / 64;       // 256 B A-scale DMA instructions per stage
  static constexpr int NA_W = (NA + NW - 1) / NW; // A instructions of the busiest wave
  static constexpr int NB_W = NB / NW;            // B instructions per wave
  static constexpr int na(int w) { return w < NA ? (NA - w + NW - 1) / NW : 0; }
  static constexpr int ns(int w) { return (NW - 1 - w) < NS ? 1 : 0; }  // the last waves issue scales
  static constexpr int cnt(int w) { return na(w) + NB_W + ns(w); }
  static constexpr int vm_min() {
    int m = cnt(0);
    for (int w = 1; w < NW; ++w) m = cnt(w) < m ? cnt(w) : m;
    return m;
  }
  // loads of one stage per wave that may stay in flight while the older stage is consumed
  static constexpr int VM = vm_min();
  static constexpr int OFF_SA = KS * STAGE;
  static constexpr int OFF_SB = OFF_SA + KS * NS * 256;
  static constexpr int OFF_RED = OFF_SB + 2 * kMaxKB * 4;
  static constexpr int OFF_ROW = OFF_RED + WN * BM * 4;  // per-row slot id and routed weight
  static constexpr int LDS_BYTES = OFF_ROW + BM * 8;
  static_assert(BM * 512 <= OFF_SA, "bf16 output staging must fit in the operand ring");
  static_assert(LDS_BYTES * WG_PER_CU <= 160 * 1024, "LDS budget");
  static_assert(VM * (KS - 2) < 64, "vmcnt immediate");
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
  int64_t max_blocks;      // (virtual) blocks that fit in max_padded
  int64_t n_tiles;         // 256-column n-tiles
  int bma;                 // rows per align block (block_size_m); a tile spans BM / bma of them
  // Exact-dot launches only: the tile map counts virtual blocks of bma >> vshift
  // rows (align block b is virtual blocks b << vshift ..), so 128-row tiles can
  // run over 256-row align blocks.  0 everywhere else.
  int vshift;
  int top_k;
  int a_by_pos;
  int E;
  int tile_order;          // 0 expert-major (XCD-contiguous), 1 shuffled, 2 half-phase
  // Strides of the (possibly sliced) operands; base pointers are pre-offset.
  int64_t lda;             // A row stride, bytes
  int64_t as_ld;           // A_scale row stride, floats
  int64_t ldb;             // B row stride, bytes
  int64_t b_es;            // B expert stride, bytes
  int64_t bs_ld;           // B_scale stride between 128-row groups, floats
  int64_t bs_es;           // B_scale expert stride, floats
  int64_t ldc;             // C row stride, elements (plain epilogue)
  int accumulate;          // plain epilogue: C = bf16(C + bf16(result)) instead of C = bf16(result)
  // Activation scales K-major by sorted position, As[kb * as_pos_ld + pos] (0: As[a_row * as_ld + kb]).
  // Each K step's scales of a tile are then one contiguous run of its rows.
  int64_t as_pos_ld;
  // Fused epilogue: hs K-major, hs[j * hs_pos_ld + pos] (0: hs[pos * I/128 + j]).
  int64_t hs_pos_ld;
};

// Element (position pos, group j) of the fused epilogue's scale output.
MOE_DEVICE float* hs_at(const GemmArgs& g, int64_t pos, int64_t j) {
  return g.hs_pos_ld ? g.hs + j * g.hs_pos_ld + pos : g.hs + pos * (g.I / 128) + j;
}

// Dense (unsliced) strides for A [rows, K], B [E, N, K], C [S, N].
static inline void dense_strides(GemmArgs& g) {
  const int64_t KB = g.K / 128;
  g.lda = g.K;
  g.as_ld = KB;
  g.ldb = g.K;
  g.b_es = g.N * g.K;
  g.bs_ld = KB;
  g.bs_es = (g.N / 128) * KB;
  g.ldc = g.N;
  g.accumulate = 0;
}

// Barrier / counter waits as compiler-opaque memory clobbers, so that no LDS
// access is moved across them and no fence forces a full vmcnt(0) drain.
MOE_DEVICE void block_barrier() { asm volatile("s_barrier" ::: "memory"); }
template <int N>
MOE_DEVICE void wait_vmcnt() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

// Direct-to-LDS loads, issued from inline asm.  The compiler's wait-count
// pass treats its own form of these loads as pending on both the vector-memory
// and the LDS counters, and while one is in flight it waits for every
// outstanding LDS read (lgkmcnt 0) at each use of an LDS read, so the fragment
// reads of a K step could not overlap each other.  The kernel waits for these
// loads itself (s_waitcnt vmcnt + s_barrier before the stage is read).  M0
// holds the LDS destination (a wave-uniform byte address), the global address
// is the uniform 64-bit base plus the lane's 32-bit offset.  M0 is declared
// clobbered (the compiler reserves it and warns that it may not honour the
// clobber), and it is written here only: the kernels that call these use no
// other M0-based instruction, which a test checks on the compiled assembly.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
MOE_DEVICE void dma16(const uint8_t* base, uint32_t off, uint8_t* lds) {
  const uint32_t m = (uint32_t)(uintptr_t)MOE_LDS(lds);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(m)
               : "memory", "m0");
}
// The same load with the non-temporal hint: for weight tiles that one row tile
// streams alone, so their lines do not displace reused lines in L2.
MOE_DEVICE void dma16_nt(const uint8_t* base, uint32_t off, uint8_t* lds) {
  const uint32_t m = (uint32_t)(uintptr_t)MOE_LDS(lds);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(off), "s"(base), "s"(m)
               : "memory", "m0");
}
MOE_DEVICE void dma4(const uint8_t* base, uint32_t off, uint8_t* lds) {
  const uint32_t m = (uint32_t)(uintptr_t)MOE_LDS(lds);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "s"(m)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Column scale groups of n-tile j: W13 gate group j and up group I/128 + j; the
// plain GEMM groups 2j and 2j+1 (the second absent past N).
template <bool FUSED>
MOE_DEVICE void groups_of(const GemmArgs& g, int64_t j, int64_t& g0, int64_t& g1, bool& g1_store) {
  if (FUSED) {
    g0 = j;
    g1 = g.I / 128 + j;
    g1_store = true;
  } else {
    const int64_t nbt = g.N / 128;
    g0 = 2 * j;
    g1 = 2 * j + 1;
    g1_store = g1 < nbt;
    if (!g1_store) g1 = nbt - 1;
  }
}

// The epilogue of one tile, shared by every tile height: SiLU*up and the
// 1x128 quant of h written by sorted position (fused W13), or the bf16 rows
// (routed weights applied) written by slot.  `staging` is LDS for BM x 512 B.
// Output element (r, gg, c, v) of a lane: token row = row_base + r*16 + fr,
// column (within group gg) = col_base + c*16 + 4*kseg + v -- the MFMA takes
// the weight fragment first, so a lane holds four consecutive columns of one
// token and stages them with one 4-byte (codes) or 8-byte (bf16) LDS write.
// Staging rows XOR their 16-byte chunk index with the row (mod 8 for codes,
// mod 16 for bf16), so the 16 tokens a write instruction covers hit distinct
// bank groups.
template <int BM, bool FUSED>
__device__ __forceinline__ void tile_epilogue(const GemmArgs& g, v4f (&acc)[Tile<BM>::RS][2][Tile<BM>::CS],
                                              int64_t j, int64_t pos0, int rows_avail, int64_t g0,
                                              int64_t g1, bool g1_store, uint8_t* staging, float* smRed,
                                              const int32_t* smSlot, const float* smW) {
  using T = Tile<BM>;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / T::WN;
  const int wn = wave % T::WN;
  const int row_base = wm * T::RS * 16;
  const int col_base = wn * T::CS * 16;
  const int fr = lane & 15;
  const int kseg = lane >> 4;
  if constexpr (FUSED) {
    float pmax[T::RS];
#pragma unroll
    for (int r = 0; r < T::RS; ++r) pmax[r] = 0.0f;
#pragma unroll
    for (int r = 0; r < T::RS; ++r)
#pragma unroll
      for (int c = 0; c < T::CS; ++c)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const uint32_t gu = pack_bf16x2(acc[r][0][c][v], acc[r][1][c][v]);
          const float h = silu_mul_bf16(lo_bf16(gu), hi_bf16(gu));
          acc[r][0][c][v] = h;
          pmax[r] = fmaxf(pmax[r], fabsf(h));
        }
#pragma unroll
    for (int r = 0; r < T::RS; ++r) {
      float m = pmax[r];
      m = fmaxf(m, __shfl_xor(m, 16));
      m = fmaxf(m, __shfl_xor(m, 32));
      if (kseg == 0) smRed[wn * BM + row_base + r * 16 + fr] = m;
    }
    __syncthreads();
    uint8_t* stage_out = staging;  // [BM][128] fp8 codes
#pragma unroll
    for (int r = 0; r < T::RS; ++r) {
      const int row = row_base + r * 16 + fr;
      float amax = 0.0f;
#pragma unroll
      for (int w = 0; w < T::WN; ++w) amax = fmaxf(amax, smRed[w * BM + row]);
      const float sc = group_scale(amax);
      const float inv = 1.0f / sc;
      if (wn == 0 && kseg == 0 && row < rows_avail) *hs_at(g, pos0 + row, j) = sc;
#pragma unroll
      for (int c = 0; c < T::CS; ++c) {
        const int col = col_base + c * 16 + 4 * kseg;
        *reinterpret_cast<uint32_t*>(stage_out + row * 128 + ((((col >> 4) ^ (row & 7)) << 4) | (col & 15))) =
            quant4_e4m3(acc[r][0][c][0], acc[r][0][c][1], acc[r][0][c][2], acc[r][0][c][3], sc, inv);
      }
    }
    __syncthreads();
    for (int ci = tid; ci < rows_avail * 8; ci += T::THREADS) {
      const int row = ci >> 3, cc = ci & 7;
      *reinterpret_cast<v4i*>(g.hq + (pos0 + row) * g.I + j * 128 + cc * 16) =
          *reinterpret_cast<const v4i*>(stage_out + row * 128 + ((cc ^ (row & 7)) << 4));
    }
  } else {
    // Both 128-column groups staged at once as [BM][256] bf16, then each row's
    // chunks (up to 512 B) written by slot.
    uint16_t* stage_out = reinterpret_cast<uint16_t*>(staging);
#pragma unroll
    for (int r = 0; r < T::RS; ++r) {
      const int row = row_base + r * 16 + fr;
      const float w = smW[row];
#pragma unroll
      for (int gg = 0; gg < 2; ++gg)
#pragma unroll
        for (int c = 0; c < T::CS; ++c) {
          v4f val = acc[r][gg][c];
          if (g.topk_w) val = val * w;
          const int col = gg * 128 + col_base + c * 16 + 4 * kseg;  // bf16 column
          v2u pk;
          pk[0] = pack_bf16x2(val[0], val[1]);
          pk[1] = pack_bf16x2(val[2], val[3]);
          *reinterpret_cast<v2u*>(stage_out + row * 256 + (((col >> 3) ^ (row & 15)) << 3) + (col & 7)) = pk;
        }
    }
    __syncthreads();
    const int nchunks = g1_store ? 32 : 16;  // 16 B chunks of a row to store
    if (!g.accumulate) {
      for (int ci = tid; ci < BM * 32; ci += T::THREADS) {
        const int row = ci >> 5, cc = ci & 31;
        if (cc >= nchunks) continue;
        const int64_t slot = smSlot[row];
        if (slot >= g.S) continue;
        const int64_t n = (cc < 16 ? g0 : g1) * 128 + (cc & 15) * 8;
        *reinterpret_cast<v4i*>(g.C + slot * g.ldc + n) =
            *reinterpret_cast<const v4i*>(stage_out + row * 256 + ((cc ^ (row & 15)) << 3));
      }
    } else {
      // K-split accumulation: the bf16 partial is added to the bf16 C of the
      // earlier chunks and rounded again.  A thread's chunks are read in
      // batches of NBATCH before any of them is written back, so the reads of
      // C overlap instead of forming one round trip per chunk.
      constexpr int PER = BM * 32 / T::THREADS;
      constexpr int NBATCH = PER < 8 ? PER : 8;
      static_assert(PER * T::THREADS == BM * 32 && PER % NBATCH == 0, "copy-out batches");
      for (int b0 = 0; b0 < PER; b0 += NBATCH) {
        v4i old[NBATCH];
        v4i* dst[NBATCH];
#pragma unroll
        for (int b = 0; b < NBATCH; ++b) {
          const int ci = tid + (b0 + b) * T::THREADS;
          const int row = ci >> 5, cc = ci & 31;
          const int64_t slot = smSlot[row];
          dst[b] = nullptr;
          if (cc < nchunks && slot < g.S) {
            const int64_t n = (cc < 16 ? g0 : g1) * 128 + (cc & 15) * 8;
            dst[b] = reinterpret_cast<v4i*>(g.C + slot * g.ldc + n);
            old[b] = *dst[b];
          }
        }
#pragma unroll
        for (int b = 0; b < NBATCH; ++b) {
          if (!dst[b]) continue;
          const int ci = tid + (b0 + b) * T::THREADS;
          const int row = ci >> 5, cc = ci & 31;
          v4i val = *reinterpret_cast<const v4i*>(stage_out + row * 256 + ((cc ^ (row & 15)) << 3));
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t a = (uint32_t)old[b][q], v = (uint32_t)val[q];
            val[q] = (int)pack_bf16x2(lo_bf16(a) + lo_bf16(v), hi_bf16(a) + hi_bf16(v));
          }
          *dst[b] = val;
        }
      }
    }
  }
}

// The K loop and epilogue of one tile: n-tile j of rows [pos0, pos0 +
// rows_avail) of the sorted order (a prefix of nvalid of them hold slots) of
// expert e, with BM-row operand tiles.  A body with BM smaller than the tile
// computes its first BM rows; the caller has checked that the rest are padding.
template <int BM, bool FUSED, bool EXACT = false>
__device__ __forceinline__ void gemm_tile(const GemmArgs& g, int64_t j, int64_t pos0, int rows_avail, int e,
                                          int nvalid, bool b_nt) {
  using T = Tile<BM>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  float* smSB = reinterpret_cast<float*>(smem + T::OFF_SB);  // [2 groups][kMaxKB]
  float* smRed = reinterpret_cast<float*>(smem + T::OFF_RED);
  int32_t* smSlot = reinterpret_cast<int32_t*>(smem + T::OFF_ROW);
  float* smW = reinterpret_cast<float*>(smem + T::OFF_ROW + BM * 4);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave-uniform values live in scalar registers
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / T::WN;
  const int wn = wave % T::WN;
  const int64_t K = g.K;
  const int KB = (int)(K / 128);
  if (rows_avail > BM) rows_avail = BM;

  auto a_row_of = [&](int row) -> int64_t {
    if (row >= rows_avail) return 0;
    const int64_t pos = pos0 + row;
    if (g.a_by_pos) return pos;
    const int64_t slot = g.sorted[pos];
    return (slot < g.S) ? slot / g.top_k : 0;
  };

  // The tile's slot ids (and routed weights) for the epilogues; the barriers
  // of the K loop order these writes before their use.
  if (tid < BM) {
    const int32_t slot = tid < rows_avail ? g.sorted[pos0 + tid] : (int32_t)g.S;
    smSlot[tid] = slot;
    if (!FUSED) smW[tid] = (g.topk_w && slot < g.S) ? g.topk_w[slot] : 1.0f;
  }

  // ---- per-lane DMA offsets (32-bit, relative to uniform bases) ----------
  // A instruction gi = wave + NW*i covers tile rows 8*gi .. 8*gi+7; lane L fills
  // LDS slot L&7 of row R = 8*gi + L/8 with logical chunk slot_of(L&7, R).
  uint32_t a_off[T::NA_W > 0 ? T::NA_W : 1];
#pragma unroll
  for (int i = 0; i < T::NA_W; ++i) {
    const int gi = wave + T::NW * i;
    const int row = (gi < T::NA) ? 8 * gi + (lane >> 3) : 0;
    const int cc = slot_of(lane & 7, row);
    a_off[i] = (uint32_t)(a_row_of(row) * g.lda) + (uint32_t)(cc * 16);
  }
  // B instruction gi = wave + NW*i covers B-tile rows 8*gi .. 8*gi+7; tile rows
  // 0..127 are scale group g0, rows 128..255 group g1.  The lane's row inside its
  // group is 8*wave + 8*NW*(i mod NB_W/2) + L/8, and its rotation does not
  // depend on i (8*NW*i leaves row mod 16 and bit 3 unchanged), so one lane
  // offset serves every instruction; the rest is a uniform base.
  uint32_t b_off;
  {
    const int r0 = 8 * wave + (lane >> 3);
    const int cc = slot_of(lane & 7, r0);
    b_off = (uint32_t)(r0 * g.ldb) + (uint32_t)(cc * 16);
  }
  // A scales: instruction s (issued by wave NW-1-s) covers rows 64*s .. 64*s+63.
  const int s_idx = T::NW - 1 - wave;
  uint32_t sa_off = 0;
  if (s_idx < T::NS) {
    const int row = 64 * s_idx + lane;
    // by position, rows past the run read the tile's first row (their outputs are not stored)
    sa_off = g.as_pos_ld ? (uint32_t)(pos0 + (row < rows_avail ? row : 0)) * 4u
                         : (uint32_t)(a_row_of(row < BM ? row : 0) * g.as_ld) * 4u;
  }
  int64_t g0, g1;
  bool g1_store;
  groups_of<FUSED>(g, j, g0, g1, g1_store);
  const uint8_t* b_expert = g.B + (int64_t)e * g.b_es;
  const float* bs_expert = g.Bs + (int64_t)e * g.bs_es;
  const uint8_t* bg0 = b_expert + g0 * 128 * g.ldb;  // the tile's two weight groups
  const uint8_t* bg1 = b_expert + g1 * 128 * g.ldb;

  // With the two-stage ring every step waits for all of its loads (vmcnt 0), so
  // the per-wave load count may vary: A rows of 16-row subtiles without a valid
  // row (their MFMAs are skipped) are not fetched.  The three-stage ring's
  // partial waits need the same count in every wave, so it fetches them all.
  const int a_rows_needed = T::KS == 2 ? (nvalid + 15) / 16 * 16 : BM;
  // Stage `stage` <- K block kk of the A rows and of weight groups at bg0, bg1.
  // The 32-bit lane offsets pass through an empty asm at every issue, so the
  // 64-bit per-lane addresses are formed where they are used instead of being
  // hoisted and kept live (which exhausts the registers of the 256-row tile).
  auto issue_stage = [&](int kk, int stage, const uint8_t* bg0, const uint8_t* bg1) {
    uint8_t* dst = smem + stage * T::STAGE;
    // Weight rows first: they come from HBM, the A rows mostly from L2.
    uint32_t boff = b_off;
    asm volatile("" : "+v"(boff));
    constexpr int HALF = T::NB_W / 2;
    if constexpr (BM <= 32) {
      auto issue_b = [&](auto load) {
#pragma unroll
        for (int i = 0; i < T::NB_W; ++i) {
          const uint8_t* bbase = (i < HALF ? bg0 : bg1) + (int64_t)(8 * T::NW * (i % HALF)) * g.ldb + kk * 128;
          load(bbase, boff, dst + T::A_BYTES + (wave + T::NW * i) * 1024);
        }
      };
      if (b_nt)
        issue_b(dma16_nt);
      else
        issue_b(dma16);
    } else {
#pragma unroll
      for (int i = 0; i < T::NB_W; ++i) {
        const uint8_t* bbase = (i < HALF ? bg0 : bg1) + (int64_t)(8 * T::NW * (i % HALF)) * g.ldb + kk * 128;
        dma16(bbase, boff, dst + T::A_BYTES + (wave + T::NW * i) * 1024);
      }
    }
    const uint8_t* abase = g.A + kk * 128;
#pragma unroll
    for (int i = 0; i < T::NA_W; ++i) {
      const int gi = wave + T::NW * i;
      uint32_t off = a_off[i];
      asm volatile("" : "+v"(off));
      if (gi < T::NA && 8 * gi < a_rows_needed) dma16(abase, off, dst + gi * 1024);
    }
    if (s_idx < T::NS) {
      uint32_t soff = sa_off;
      asm volatile("" : "+v"(soff));
      dma4(reinterpret_cast<const uint8_t*>(g.as_pos_ld ? g.As + kk * g.as_pos_ld : g.As + kk), soff,
           smem + T::OFF_SA + stage * T::NS * 256 + s_idx * 256);
    }
  };

  // Weight scales of both groups for every K block, smSB[g * kMaxKB + kk]:
  // one 4-byte direct-to-LDS load per lane of waves 0-3 (entry 64 * wave +
  // lane), issued before stage 0, so that step 0's wait covers them.  Entries
  // past KB read a valid scale and are never used.
  static_assert(2 * kMaxKB == 4 * 64 && Tile<BM>::NW >= 4, "four waves load the weight scales");
  auto issue_weight_scales = [&] {
    if (wave < 4) {
      const int idx = 64 * wave + lane;
      const int kb = idx % kMaxKB;
      const int64_t grp = idx < kMaxKB ? g0 : g1;
      uint32_t off = (uint32_t)((grp * g.bs_ld + (kb < KB ? kb : 0)) * 4);
      asm volatile("" : "+v"(off));
      dma4(reinterpret_cast<const uint8_t*>(bs_expert), off, reinterpret_cast<uint8_t*>(smSB) + 256 * wave);
    }
  };

  const int row_base = wm * T::RS * 16;
  const int col_base = wn * T::CS * 16;
  const int fr = lane & 15;
  const int kseg = lane >> 4;
  // Per-lane fragment byte offsets within a stage (chunk h of the lane's 32 B).
  const int lane0 = fr * 128 + (slot_of(2 * kseg, fr) << 4);
  const int lane1 = fr * 128 + (slot_of(2 * kseg + 1, fr) << 4);
  const int a_lane0 = row_base * 128 + lane0, a_lane1 = row_base * 128 + lane1;
  const int b_lane0 = T::A_BYTES + col_base * 128 + lane0;
  const int b_lane1 = T::A_BYTES + col_base * 128 + lane1;
  const float* smSA = reinterpret_cast<const float*>(smem + T::OFF_SA);
  const int sa_lane = row_base + fr;  // the lane's token (the MFMA's second operand)

  issue_weight_scales();
  issue_stage(0, 0, bg0, bg1);
#pragma unroll
  for (int st = 1; st < T::KS - 1; ++st)
    if (st < KB) issue_stage(st, st, bg0, bg1);

  int ra = (nvalid - row_base + 15) / 16;
  ra = ra < 0 ? 0 : (ra > T::RS ? T::RS : ra);

  v4f acc[T::RS][2][T::CS];
#pragma unroll
  for (int r = 0; r < T::RS; ++r)
#pragma unroll
    for (int gg = 0; gg < 2; ++gg)
#pragma unroll
      for (int c = 0; c < T::CS; ++c) acc[r][gg][c] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};

  auto kloop = [&](auto ra_c) {
    constexpr int RA = decltype(ra_c)::value;  // active 16-row subtiles of this wave
    int stage = 0;
    for (int kk = 0; kk < KB; ++kk) {
      // Step kk's loads complete; the younger stages' loads (up to KS - 2 of
      // them, as many as were issued) may stay in flight.
      if (T::KS == 4 && kk + 2 < KB) wait_vmcnt<2 * T::VM>();
      else if (T::KS >= 3 && kk + 1 < KB) wait_vmcnt<T::VM>();
      else wait_vmcnt<0>();
      block_barrier();
      // The buffer read at step kk-1 is free once every wave has passed the barrier.
      // The waves issue the stage's loads at raised priority, so that all of
      // them are in flight before the MFMAs of any wave take the issue slots.
      __builtin_amdgcn_s_setprio(3);
      if (kk + T::KS - 1 < KB) issue_stage(kk + T::KS - 1, stage == 0 ? T::KS - 1 : stage - 1, bg0, bg1);
      __builtin_amdgcn_s_setprio(0);
      if constexpr (RA > 0) {
        const uint8_t* st = smem + stage * T::STAGE;
        const uint8_t* pa0 = st + a_lane0;
        const uint8_t* pa1 = st + a_lane1;
        const uint8_t* pb0 = st + b_lane0;
        const uint8_t* pb1 = st + b_lane1;
        const float* tSA = smSA + stage * T::NS * 64 + sa_lane;
        // a_s * b_s of the step for each 16-row subtile and column group
        float sab[2][RA];
        auto scale_products = [&] {
          const float sb0 = smSB[kk];
          const float sb1 = smSB[kMaxKB + kk];
#pragma unroll
          for (int r = 0; r < RA; ++r) {
            const float sa = tSA[r * 16];
            sab[0][r] = sa * sb0;
            sab[1][r] = sa * sb1;
          }
        };
        constexpr int NQ = 2 * T::CS;  // weight fragments per step
        if constexpr (EXACT) {
#pragma clang fp contract(off)
          // Exact dots on the bf16 matrix core: the step's A fragments are
          // converted once, each weight fragment as it is read; every 128-K
          // dot is four chained bf16 MFMAs.  The dot is scaled into acc by the
          // reference's own chain, acc + (dot * a_s) * b_s with three
          // roundings (overlap/kernels.py:179), not the fused form below: with
          // exact dots the scale chain is the main remaining difference from
          // the reference's arithmetic (it moves about 20x more C13 values).
          float sa[RA];
#pragma unroll
          for (int r = 0; r < RA; ++r) sa[r] = tSA[r * 16];
          const float sbg[2] = {smSB[kk], smSB[kMaxKB + kk]};
          v8bf abf[RA][4];
          [&]<int... R>(std::integer_sequence<int, R...>) {
            (
                [&] {
                  const v8i f = frag_at<R * 2048>(pa0, pa1);
#pragma unroll
                  for (int q = 0; q < 4; ++q) abf[R][q] = fp8_quarter_bf16(f, q);
                }(),
                ...);
          }(std::make_integer_sequence<int, RA>{});
          [&]<int... Q>(std::integer_sequence<int, Q...>) {
            (
                [&] {
                  constexpr int gq = Q / T::CS, cq = Q % T::CS;
                  const v8i fb = frag_at<(gq * 128 + cq * 16) * 128>(pb0, pb1);
                  v8bf bbf[4];
#pragma unroll
                  for (int q = 0; q < 4; ++q) bbf[q] = fp8_quarter_bf16(fb, q);
#pragma unroll
                  for (int r = 0; r < RA; ++r) {
                    const v4f p = mfma_bf16_dot128(bbf, abf[r]);
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                      float t = p[v] * sa[r];
                      t = t * sbg[gq];
                      acc[r][gq][cq][v] = acc[r][gq][cq][v] + t;
                    }
                  }
                }(),
                ...);
          }(std::make_integer_sequence<int, NQ>{});
        } else {
          v8i af[RA];
          [&]<int... R>(std::integer_sequence<int, R...>) {
            ((af[R] = frag_at<R * 2048>(pa0, pa1)), ...);
          }(std::make_integer_sequence<int, RA>{});
          // Weight fragments triple-buffered (two LDS reads in flight ahead of the
          // MFMAs that use them); MFMA t is issued before the scale FMAs of MFMA
          // t - kScaleLag, whose result is ready by then.  The MFMA takes the
          // weight fragment first, so a lane's four results are four columns of
          // one token: one scale product a_s * b_s per 16-row subtile and group.
          constexpr int LG = kScaleLag;
          constexpr int NT = NQ * RA;
          constexpr int NBQ = 3;
          v8i bq[NBQ];
          v4f p[LG + 1];
          scale_products();
          bq[0] = frag_at<0>(pb0, pb1);
          if constexpr (NQ > 1) bq[1] = frag_at<(1 / T::CS * 128 + 1 % T::CS * 16) * 128>(pb0, pb1);
          [&]<int... Q>(std::integer_sequence<int, Q...>) {
            (
                [&] {
                  if constexpr (Q + NBQ - 1 < NQ) {
                    constexpr int gn = (Q + NBQ - 1) / T::CS, cn = (Q + NBQ - 1) % T::CS;
                    bq[(Q + NBQ - 1) % NBQ] = frag_at<(gn * 128 + cn * 16) * 128>(pb0, pb1);
                  }
#pragma unroll
                  for (int r = 0; r < RA; ++r) {
                    const int t = Q * RA + r;
                    p[t % (LG + 1)] = mfma_fp8(bq[Q % NBQ], af[r]);
                    if (t >= LG) {
                      const int u = t - LG, uq = u / RA, ur = u % RA;
                      const int ug = uq / T::CS, uc = uq % T::CS;
#pragma unroll
                      for (int v = 0; v < 4; ++v)
                        acc[ur][ug][uc][v] = __builtin_fmaf(p[u % (LG + 1)][v], sab[ug][ur], acc[ur][ug][uc][v]);
                    }
                  }
                }(),
                ...);
          }(std::make_integer_sequence<int, NQ>{});
          [&]<int... D>(std::integer_sequence<int, D...>) {  // drain the last LG MFMAs
            (
                [&] {
                  constexpr int u = NT - LG + D;
                  if constexpr (u >= 0) {
                    constexpr int uq = u / RA, ur = u % RA;
                    constexpr int ug = uq / T::CS, uc = uq % T::CS;
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                      acc[ur][ug][uc][v] = __builtin_fmaf(p[u % (LG + 1)][v], sab[ug][ur], acc[ur][ug][uc][v]);
                  }
                }(),
                ...);
          }(std::make_integer_sequence<int, LG>{});
        }
      }
      stage = (stage == T::KS - 1) ? 0 : stage + 1;
    }
  };
  switch (ra) {
    case 0: kloop(std::integral_constant<int, 0>{}); break;
    case 1: if constexpr (T::RS >= 1) kloop(std::integral_constant<int, (T::RS >= 1 ? 1 : 0)>{}); break;
    case 2: if constexpr (T::RS >= 2) kloop(std::integral_constant<int, (T::RS >= 2 ? 2 : 0)>{}); break;
    case 3: if constexpr (T::RS >= 3) kloop(std::integral_constant<int, (T::RS >= 3 ? 3 : 0)>{}); break;
    default: if constexpr (T::RS >= 4) kloop(std::integral_constant<int, (T::RS >= 4 ? 4 : 0)>{}); break;
  }
  // Every wave is done with the operand ring (the last step waited for all of
  // its loads); the epilogue stages the output at its base.
  block_barrier();
  tile_epilogue<BM, FUSED>(g, acc, j, pos0, rows_avail, g0, g1, g1_store, smem, smRed, smSlot, smW);

}

// A tile of a BM-row launch whose valid rows fit SUB rows, run with the
// SUB-row body.  Positions [SUB, rows_avail) are padding: the fused outputs
// there are the zero codes and floor scales an all-zero row quantises to.
template <int SUB, int BM, bool FUSED, bool EXACT>
__device__ __forceinline__ void short_tile(const GemmArgs& g, int64_t j, int64_t pos0, int rows_avail, int e,
                                           int nvalid) {
  static_assert(Tile<SUB>::THREADS == Tile<BM>::THREADS, "same workgroup size");
  gemm_tile<SUB, FUSED, EXACT>(g, j, pos0, rows_avail, e, nvalid, false);
  if (FUSED) {
    const int tid = threadIdx.x;
    for (int ci = SUB * 8 + tid; ci < rows_avail * 8; ci += Tile<BM>::THREADS) {
      const int row = ci >> 3, cc = ci & 7;
      *reinterpret_cast<v4i*>(g.hq + (pos0 + row) * g.I + j * 128 + cc * 16) = (v4i){0, 0, 0, 0};
    }
    for (int row = SUB + tid; row < rows_avail; row += Tile<BM>::THREADS) *hs_at(g, pos0 + row, j) = kScaleFloor;
  }
}

// Dynamic LDS of a launch with BM-row tiles (the larger of the bodies it may run).
template <int BM>
constexpr int kernel_lds() {
  return BM == 256 && Tile<128>::LDS_BYTES > Tile<256>::LDS_BYTES ? Tile<128>::LDS_BYTES : Tile<BM>::LDS_BYTES;
}

// One workgroup of a BM-row launch: the tile map below, then the tile's body.
// EXACT (fused W13 only) takes the dots on the bf16 matrix core; its 256-row
// launch runs each tile as two 128-row bodies, since the bf16 fragments of the
// 256-row body do not fit in the registers.
template <int BM, bool FUSED, bool EXACT>
__device__ __forceinline__ void grouped_gemm_body(const GemmArgs& g) {
  using T = Tile<BM>;
  static_assert(FUSED || !EXACT, "the exact-dot form is built for the fused W13 GEMM");
  static_assert(BM <= kTailRows || Tile<kTailRows>::LDS_BYTES <= kernel_lds<BM>(),
                "the short body must fit in the launch's LDS");
  const int tid = threadIdx.x;

  // ---- expert-aligned, XCD-aware tile mapping ----------------------------
  // A workgroup computes one row tile by one n-tile.  Tiles are ordered
  // run-major: for each run of consecutive blocks with the same expert (blocks
  // [b0, b0+n)), its tiles are t in [b0*NT, (b0+n)*NT), in groups of a few
  // n-tiles (all row tiles of the run inside a group), so the row tiles that
  // read one weight tile are close together.  Workgroup ids are dealt
  // round-robin to the XCDs; XCD x takes the contiguous range t in
  // [x*C, (x+1)*C), so those row tiles run at the same time on one XCD and
  // fetch the weight tile from HBM once.
  const int ntpp = *g.ntpp;
  const int vsh = EXACT ? g.vshift : 0;
  const int64_t vb = (int64_t)g.bma >> vsh;  // rows of a (virtual) block
  const int64_t n_blocks = ntpp / vb;
  const int64_t total = n_blocks * g.n_tiles;
  const int64_t per_xcd = (total + kXcds - 1) / kXcds;
  const int64_t pid = blockIdx.x;
  int64_t t;
  if (g.tile_order == 0) {
    const int64_t local = pid / kXcds;
    if (local >= per_xcd) return;
    t = (pid % kXcds) * per_xcd + local;
  } else if (g.tile_order == 1) {
    // Shuffled arrival order: bit reversal within the next power of two,
    // walked back into [0, total) (bit reversal is an involution, so a
    // reversed index outside the range maps the id to itself: a bijection).
    if (pid >= total) return;
    int m = 0;
    while (((int64_t)1 << m) < total) ++m;
    const int64_t r = m ? (int64_t)(__builtin_bitreverse64((uint64_t)pid) >> (64 - m)) : 0;
    t = r < total ? r : pid;
  } else {
    // Half-phase: the first and second halves of the expert-major order,
    // interleaved tile by tile.
    if (pid >= total) return;
    const int64_t half = (total + 1) / 2;
    t = (pid & 1) ? half + pid / 2 : pid / 2;
  }
  if (t >= total) return;
  const int64_t bq = t / g.n_tiles;  // a block of the tile's run
  // The run of blocks with bq's expert: the expert ids of bq and of the 64
  // blocks on either side are loaded together (one memory round trip for runs
  // of up to 65 blocks), longer runs continue 64 blocks at a time.
  int64_t back = 0, fwd = 0;
  int e;
  {
    const int ln = threadIdx.x & 63;
    const int64_t ib = bq - 1 - ln, jf = bq + 1 + ln;
    e = g.eids[bq >> vsh];
    const int xb = ib >= 0 ? g.eids[ib >> vsh] : 0;
    const int xf = jf < n_blocks ? g.eids[jf >> vsh] : 0;
    uint64_t end = __ballot(!(ib >= 0 && xb == e));  // blocks before bq with the same expert
    for (int64_t base = bq - 1 - 64; !end; base -= 64) {
      back += 64;
      const int64_t idx = base - ln;
      end = __ballot(!(idx >= 0 && g.eids[idx >> vsh] == e));
    }
    back += __ffsll((unsigned long long)end) - 1;
    end = __ballot(!(jf < n_blocks && xf == e));      // and after it
    for (int64_t base = bq + 1 + 64; !end; base += 64) {
      fwd += 64;
      const int64_t idx = base + ln;
      end = __ballot(!(idx < n_blocks && g.eids[idx >> vsh] == e));
    }
    fwd += __ffsll((unsigned long long)end) - 1;
  }
  const int64_t b0 = bq - back;
  const int64_t run = back + 1 + fwd;
  // A row tile spans up to ub consecutive align blocks of the run (one when BM
  // equals the align block size); the run's `units` row tiles take its first
  // units * NT tile ids and the rest of its ids are idle.  The run's blocks are
  // split over its row tiles as evenly as possible, the larger tiles last:
  // a run of three blocks in 2-block tiles becomes 1 + 2 blocks, two tiles
  // that stream the same weight tiles at the same pace, rather than 2 + 1,
  // a full tile and a tile of a few padded rows.  Only the last align block
  // of a run holds padding, so a tile's valid rows are still a prefix (with
  // virtual blocks, the run's last one may hold no valid row at all).
  const int64_t ub = BM / vb;
  const int64_t units = (run + ub - 1) / ub;
  const int64_t in_run = t - b0 * g.n_tiles;
  if (in_run >= units * g.n_tiles) return;
  // Inside a run, n-tiles go in groups of GG, row-tile-major within a group:
  // the GG workgroups that share an A tile start together and reuse it from
  // L2, and a weight tile is still read by all row tiles of the run close in time.
  // Plain launches with a long K (kColMajorK and up: W2 of wide experts, whose
  // weight tiles are large) go column-major within a group instead: the row
  // tiles that share a weight tile start together.
  constexpr int64_t GG = 4;  // 2, 8 and 16 (W13), 2, 3, 7 and 14 (W2) measured slower
  const int64_t gj0 = in_run / (GG * units) * GG;
  const int64_t gsz = (g.n_tiles - gj0) < GG ? (g.n_tiles - gj0) : GG;
  const int64_t in_grp = in_run - gj0 * units;
  const bool by_col = !FUSED && g.K >= kColMajorK;
  const int64_t j = gj0 + (by_col ? in_grp / units : in_grp % gsz);
  const int64_t u = by_col ? in_grp % units : in_grp / gsz;  // row tile of the run
  const int64_t base = run / units, n_short = units - run % units;  // n_short tiles of `base` blocks
  const int64_t b = b0 + (u < n_short ? u * base : n_short * base + (u - n_short) * (base + 1));
  const int64_t pos0 = b * vb;                  // sorted position of tile row 0
  // tile rows that belong to this run (the rest are not read or written)
  const int rows_avail = (int)((u < n_short ? base : base + 1) * vb);

  if (e < 0 || e >= g.E) {
    // Expert not local: zero output rows (kernels.py:112-120).
    if (!FUSED && g.accumulate) return;  // later K chunks leave C as it is (kernels.py:112-120)
    int64_t g0, g1;
    bool g1_store;
    groups_of<FUSED>(g, j, g0, g1, g1_store);
    if (FUSED) {
      for (int ci = tid; ci < rows_avail * 8; ci += T::THREADS) {
        const int row = ci >> 3, cc = ci & 7;
        *reinterpret_cast<v4i*>(g.hq + (pos0 + row) * g.I + j * 128 + cc * 16) = (v4i){0, 0, 0, 0};
      }
      for (int row = tid; row < rows_avail; row += T::THREADS)
        *hs_at(g, pos0 + row, j) = kScaleFloor;
    } else {
      for (int ci = tid; ci < rows_avail * 32; ci += T::THREADS) {
        const int row = ci >> 5, cc = ci & 31;
        const int64_t slot = g.sorted[pos0 + row];
        if (slot >= g.S) continue;
        const int grp = cc >> 4;
        if (grp == 1 && !g1_store) continue;
        const int64_t n = (grp ? g1 : g0) * 128 + (cc & 15) * 8;
        *reinterpret_cast<v4i*>(g.C + slot * g.ldc + n) = (v4i){0, 0, 0, 0};
      }
    }
    return;
  }

  // Rows of the tile that hold real slots (a prefix: padding follows them).
  bool row_valid = false;
  if (tid < BM && tid < rows_avail) row_valid = g.sorted[pos0 + tid] < g.S;
  const int nvalid = __syncthreads_count(row_valid);
  if constexpr (EXACT) {
    // The second half of a 256-row align block whose slots all sit in its
    // first half: padding only, written as the zero codes and floor scales
    // that the two-body tile writes there.
    if (nvalid == 0) {
      for (int ci = tid; ci < rows_avail * 8; ci += T::THREADS) {
        const int row = ci >> 3, cc = ci & 7;
        *reinterpret_cast<v4i*>(g.hq + (pos0 + row) * g.I + j * 128 + cc * 16) = (v4i){0, 0, 0, 0};
      }
      for (int row = tid; row < rows_avail; row += T::THREADS) *hs_at(g, pos0 + row, j) = kScaleFloor;
      return;
    }
  }
  // A tile with few valid rows (an expert's last rows, or a one-block tile of
  // a run split over tiles) runs a shorter body: kTailRows rows, bound by
  // streaming its weight tile with a three-deep LDS ring; or, in a 256-row
  // launch, the 128-row body, whose eight waves split the 128 rows into 64 x 64
  // subtiles instead of leaving half of the 256-row body's MFMAs on padding.
  if constexpr (BM > kTailRows) {
    if (nvalid <= kTailRows) {
      short_tile<kTailRows, BM, FUSED, EXACT>(g, j, pos0, rows_avail, e, nvalid);
      return;
    }
  }
  if constexpr (BM == 256) {
    if (nvalid <= 128) {
      short_tile<128, BM, FUSED, EXACT>(g, j, pos0, rows_avail, e, nvalid);
      return;
    }
    if constexpr (EXACT) {
      // rows [0, 128) and then [128, rows_avail), whose valid rows are
      // [128, nvalid); the barrier keeps the second body's first loads out of
      // the LDS the first one's copy-out still reads
      gemm_tile<128, FUSED, EXACT>(g, j, pos0, 128, e, 128, false);
      __syncthreads();
      gemm_tile<128, FUSED, EXACT>(g, j, pos0 + 128, rows_avail - 128, e, nvalid - 128, false);
      return;
    }
  }
  // Weight-streaming tiles (16 and 32 rows) of an expert with one row tile are
  // the only readers of their weight tiles: those loads carry the
  // non-temporal hint.  Experts with several row tiles, and taller tiles,
  // share weight tiles through L2 and load them cached.
  if constexpr (!(EXACT && BM == 256)) gemm_tile<BM, FUSED, EXACT>(g, j, pos0, rows_avail, e, nvalid, BM <= 32 && units == 1);
}

template <int BM, bool FUSED>
__global__ __launch_bounds__(Tile<BM>::THREADS)
__attribute__((amdgpu_waves_per_eu(Tile<BM>::NW / 4 * Tile<BM>::WG_PER_CU, Tile<BM>::NW / 4 * Tile<BM>::WG_PER_CU)))
void grouped_gemm_kernel(GemmArgs g) {
  grouped_gemm_body<BM, FUSED, false>(g);
}

// The fused W13 GEMM with exact dots (moe_gemm_w13_silu_quant_exact).
template <int BM>
__global__ __launch_bounds__(Tile<BM>::THREADS)
__attribute__((amdgpu_waves_per_eu(Tile<BM>::NW / 4 * Tile<BM>::WG_PER_CU, Tile<BM>::NW / 4 * Tile<BM>::WG_PER_CU)))
void w13_exact_kernel(GemmArgs g) {
  grouped_gemm_body<BM, true, true>(g);
}

template <int BM, bool FUSED, bool EXACT>
static int launch_gemm(const GemmArgs& args, hipStream_t st) {
  using T = Tile<BM>;
  const void* fn;
  if constexpr (EXACT)
    fn = (const void*)w13_exact_kernel<BM>;
  else
    fn = (const void*)grouped_gemm_kernel<BM, FUSED>;
  // Set once per process (a function-local static is initialised exactly once,
  // also when several host threads make their first call together).
  static const hipError_t attr_rc =
      hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kernel_lds<BM>());
  if (attr_rc != hipSuccess) return kErrLaunch;
  // Upper bound on the tile count (the real one depends on ntpp, on the device).
  const int64_t grid = (args.max_blocks * args.n_tiles + kXcds - 1) / kXcds * kXcds;
  if (grid <= 0) return kOk;
  if constexpr (EXACT)
    hipLaunchKernelGGL((w13_exact_kernel<BM>), dim3((unsigned)grid), dim3(T::THREADS), kernel_lds<BM>(), st, args);
  else
    hipLaunchKernelGGL((grouped_gemm_kernel<BM, FUSED>), dim3((unsigned)grid), dim3(T::THREADS), kernel_lds<BM>(),
                       st, args);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

template <bool FUSED, bool EXACT = false>
static int dispatch_gemm(int TM, const GemmArgs& args, hipStream_t st) {
  switch (TM) {
    case 16: return launch_gemm<16, FUSED, EXACT>(args, st);
    case 32: return launch_gemm<32, FUSED, EXACT>(args, st);
    case 64: return launch_gemm<64, FUSED, EXACT>(args, st);
    case 128: return launch_gemm<128, FUSED, EXACT>(args, st);
    case 256: return launch_gemm<256, FUSED, EXACT>(args, st);
    default: return kErrBadBlockSize;
  }
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Rows of a workgroup tile: tile_m / BM consecutive align blocks of one expert
// share a tile.  0 picks 256 when the experts average at least 160 slots (the
// weight tile is then fetched once per 256 rows instead of once per block) and
// BM otherwise.  Returns -1 for a tile_m that is not a supported block size and
// a multiple of BM.
static int resolve_tile_m(int32_t tile_m, int32_t BM, int64_t S, int32_t E) {
  if (tile_m == 0) return S >= 160 * (int64_t)E ? 256 : BM;
  if (!block_m_ok(tile_m) || tile_m < BM || tile_m % BM != 0) return -1;
  return tile_m;
}

// 32-bit lane offsets: every A row and every expert's B block must be
// addressable with a uint32 offset from its base.
static bool offsets_fit(int64_t rows, int64_t N, int64_t K) {
  return rows * K < (int64_t)1 << 32 && N * K < (int64_t)1 << 32;
}

}  // namespace moe

using namespace moe;

// The plain grouped GEMM on dense operands; A_scale row-major by A row, or
// K-major by sorted position when scales_by_pos (A then by position too).
static int plain_gemm(const void* A, const float* A_scale, const void* B, const float* B_scale,
                      const int32_t* sorted_ids, const int32_t* expert_ids, const int32_t* ntpp,
                      const float* topk_weights, int64_t S, int32_t top_k, int32_t a_by_pos, int64_t N,
                      int64_t K, int32_t E, int32_t BM, int64_t max_padded, int32_t tile_order,
                      int32_t tile_m, bool scales_by_pos, void* C, void* stream) {
  if (S < 0 || N <= 0 || K <= 0 || max_padded < 0) return kErrBadShape;
  if (N % 128 != 0 || K % 128 != 0 || K > 128 * kMaxKB) return kErrBadShape;
  if (top_k <= 0) return kErrBadTopK;
  if (E <= 0) return kErrBadExperts;
  if (!block_m_ok(BM)) return kErrBadBlockSize;
  const int TM = resolve_tile_m(tile_m, BM, S, E);
  if (TM < 0) return kErrBadBlockSize;
  if (tile_order < 0 || tile_order > 2) return kErrBadShape;
  if (max_padded == 0 || S == 0) return kOk;
  if (!A || !A_scale || !B || !B_scale || !sorted_ids || !expert_ids || !ntpp || !C)
    return kErrNullPointer;
  if (!aligned16(A) || !aligned16(B) || !aligned16(C)) return kErrBadShape;
  const int64_t a_rows = a_by_pos ? max_padded : (S + top_k - 1) / top_k;
  if (!offsets_fit(a_rows, N, K)) return kErrBadShape;
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
  g.bma = BM;
  g.top_k = top_k;
  g.a_by_pos = a_by_pos ? 1 : 0;
  g.E = E;
  g.tile_order = tile_order;
  dense_strides(g);
  if (scales_by_pos) g.as_pos_ld = max_padded;
  return dispatch_gemm<false>(TM, g, (hipStream_t)stream);
}

extern "C" int moe_grouped_gemm_tiled(const void* A, const float* A_scale, const void* B,
                                      const float* B_scale, const int32_t* sorted_ids,
                                      const int32_t* expert_ids, const int32_t* ntpp,
                                      const float* topk_weights, int64_t S, int32_t top_k,
                                      int32_t a_by_pos, int64_t N, int64_t K, int32_t E, int32_t BM,
                                      int64_t max_padded, int32_t tile_order, int32_t tile_m,
                                      void* C, void* stream) {
  return plain_gemm(A, A_scale, B, B_scale, sorted_ids, expert_ids, ntpp, topk_weights, S, top_k, a_by_pos, N, K,
                    E, BM, max_padded, tile_order, tile_m, false, C, stream);
}

extern "C" int moe_grouped_gemm_pos(const void* A, const float* A_scale_pos, const void* B,
                                    const float* B_scale, const int32_t* sorted_ids,
                                    const int32_t* expert_ids, const int32_t* ntpp,
                                    const float* topk_weights, int64_t S, int64_t N, int64_t K, int32_t E,
                                    int32_t BM, int64_t max_padded, int32_t tile_m, void* C, void* stream) {
  return plain_gemm(A, A_scale_pos, B, B_scale, sorted_ids, expert_ids, ntpp, topk_weights, S, 1, 1, N, K, E, BM,
                    max_padded, 0, tile_m, true, C, stream);
}

extern "C" int moe_grouped_gemm_ordered(const void* A, const float* A_scale, const void* B,
                                        const float* B_scale, const int32_t* sorted_ids,
                                        const int32_t* expert_ids, const int32_t* ntpp,
                                        const float* topk_weights, int64_t S, int32_t top_k,
                                        int32_t a_by_pos, int64_t N, int64_t K, int32_t E,
                                        int32_t BM, int64_t max_padded, int32_t tile_order,
                                        void* C, void* stream) {
  return moe_grouped_gemm_tiled(A, A_scale, B, B_scale, sorted_ids, expert_ids, ntpp, topk_weights, S,
                                top_k, a_by_pos, N, K, E, BM, max_padded, tile_order, 0, C, stream);
}

extern "C" int moe_grouped_gemm(const void* A, const float* A_scale, const void* B,
                                const float* B_scale, const int32_t* sorted_ids,
                                const int32_t* expert_ids, const int32_t* ntpp,
                                const float* topk_weights, int64_t S, int32_t top_k,
                                int32_t a_by_pos, int64_t N, int64_t K, int32_t E, int32_t BM,
                                int64_t max_padded, void* C, void* stream) {
  return moe_grouped_gemm_ordered(A, A_scale, B, B_scale, sorted_ids, expert_ids, ntpp,
                                  topk_weights, S, top_k, a_by_pos, N, K, E, BM, max_padded, 0, C,
                                  stream);
}

// Shared argument checks and setup of the plain-epilogue GEMM on (possibly
// sliced) operands; the caller fills the strides and pre-offsets the bases.
static int setup_plain(GemmArgs& g, int& TM, const void* A, const float* A_scale, const void* B,
                       const float* B_scale, const int32_t* sorted_ids, const int32_t* expert_ids,
                       const int32_t* ntpp, const float* topk_weights, int64_t S, int32_t top_k,
                       int32_t a_by_pos, int64_t N, int64_t K, int32_t E, int32_t BM, int64_t max_padded,
                       void* C) {
  if (S < 0 || N <= 0 || K <= 0 || max_padded < 0) return kErrBadShape;
  if (N % 128 != 0 || K % 128 != 0 || K > 128 * kMaxKB) return kErrBadShape;
  if (top_k <= 0) return kErrBadTopK;
  if (E <= 0) return kErrBadExperts;
  if (!block_m_ok(BM)) return kErrBadBlockSize;
  TM = resolve_tile_m(0, BM, S, E);
  // nothing to compute: the caller returns before touching g (empty operands may be null)
  if (max_padded == 0 || S == 0) return kOk;
  if (!A || !A_scale || !B || !B_scale || !sorted_ids || !expert_ids || !ntpp || !C)
    return kErrNullPointer;
  g = GemmArgs{};
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
  g.max_blocks = (max_padded + BM - 1) / BM;
  g.n_tiles = (N / 128 + 1) / 2;
  g.bma = BM;
  g.top_k = top_k;
  g.a_by_pos = a_by_pos ? 1 : 0;
  g.E = E;
  dense_strides(g);
  return kOk;
}

extern "C" int moe_grouped_gemm_n_split(const void* A, const float* A_scale, const void* B,
                                        const float* B_scale, const int32_t* sorted_ids,
                                        const int32_t* expert_ids, const int32_t* ntpp,
                                        const float* topk_weights, int64_t S, int32_t top_k,
                                        int32_t a_by_pos, int64_t full_N, int64_t N_offset,
                                        int64_t N_chunk, int64_t K, int32_t E, int32_t BM,
                                        int64_t max_padded, void* C, void* stream) {
  if (full_N <= 0 || N_offset < 0 || N_chunk <= 0 || N_offset + N_chunk > full_N) return kErrBadShape;
  if (full_N % 128 != 0 || N_offset % 128 != 0) return kErrBadShape;
  GemmArgs g;
  int TM = 0;
  const int rc = setup_plain(g, TM, A, A_scale, B, B_scale, sorted_ids, expert_ids, ntpp, topk_weights, S,
                             top_k, a_by_pos, N_chunk, K, E, BM, max_padded, C);
  if (rc != kOk || max_padded == 0 || S == 0) return rc;
  const int64_t KB = K / 128;
  // B[:, N_offset:N_offset+N_chunk, :], B_scale[:, N_offset/128:, :], C[:, N_offset:]
  g.B += N_offset * K;
  g.Bs += (N_offset / 128) * KB;
  g.C += N_offset;
  g.b_es = full_N * K;
  g.bs_es = (full_N / 128) * KB;
  g.ldc = full_N;
  if (!aligned16(g.A) || !aligned16(g.B) || !aligned16(g.C)) return kErrBadShape;
  const int64_t a_rows = a_by_pos ? max_padded : (S + top_k - 1) / top_k;
  if (!offsets_fit(a_rows, full_N, K)) return kErrBadShape;
  return dispatch_gemm<false>(TM, g, (hipStream_t)stream);
}

extern "C" int moe_grouped_gemm_k_split(const void* A, const float* A_scale, int64_t A_cols,
                                        int64_t A_K_offset, const void* B, const float* B_scale,
                                        const int32_t* sorted_ids, const int32_t* expert_ids,
                                        const int32_t* ntpp, const float* topk_weights, int64_t S,
                                        int32_t top_k, int32_t a_by_pos, int64_t N, int64_t full_K,
                                        int64_t K_offset, int64_t K_chunk, int32_t E, int32_t BM,
                                        int64_t max_padded, int32_t is_first_chunk, void* C,
                                        void* stream) {
  if (full_K <= 0 || K_offset < 0 || K_chunk <= 0 || K_offset + K_chunk > full_K) return kErrBadShape;
  if (A_cols <= 0 || A_K_offset < 0 || A_K_offset + K_chunk > A_cols) return kErrBadShape;
  if (full_K % 128 != 0 || K_offset % 128 != 0 || A_cols % 128 != 0 || A_K_offset % 128 != 0)
    return kErrBadShape;
  GemmArgs g;
  int TM = 0;
  const int rc = setup_plain(g, TM, A, A_scale, B, B_scale, sorted_ids, expert_ids, ntpp, topk_weights, S,
                             top_k, a_by_pos, N, K_chunk, E, BM, max_padded, C);
  if (rc != kOk || max_padded == 0 || S == 0) return rc;
  // A[:, A_K_offset:+K_chunk] of an [rows, A_cols] tensor (scales [rows, A_cols/128]),
  // B[:, :, K_offset:+K_chunk] of [E, N, full_K] (scales [E, N/128, full_K/128]).
  g.A += A_K_offset;
  g.As += A_K_offset / 128;
  g.lda = A_cols;
  g.as_ld = A_cols / 128;
  g.B += K_offset;
  g.Bs += K_offset / 128;
  g.ldb = full_K;
  g.b_es = N * full_K;
  g.bs_ld = full_K / 128;
  g.bs_es = (N / 128) * (full_K / 128);
  g.accumulate = is_first_chunk ? 0 : 1;
  if (!aligned16(g.A) || !aligned16(g.B) || !aligned16(g.C)) return kErrBadShape;
  const int64_t a_rows = a_by_pos ? max_padded : (S + top_k - 1) / top_k;
  if (!offsets_fit(a_rows, N, full_K) || a_rows * A_cols >= ((int64_t)1 << 32)) return kErrBadShape;
  return dispatch_gemm<false>(TM, g, (hipStream_t)stream);
}

// The fused W13 GEMM; scales row-major (A_scale by token, hs by position), or
// both K-major by sorted position when scales_by_pos; exact dots on the bf16
// matrix core when exact.
static int w13_gemm(const void* Aq, const float* A_scale, const void* W13, const float* W13_scale,
                    const int32_t* sorted_ids, const int32_t* expert_ids, const int32_t* ntpp, int64_t S,
                    int32_t top_k, int64_t H, int64_t I, int32_t E, int32_t BM, int64_t max_padded,
                    int32_t tile_m, bool scales_by_pos, bool exact, void* hq, float* hs, void* stream) {
  if (S < 0 || H <= 0 || I <= 0 || max_padded < 0) return kErrBadShape;
  if (H % 128 != 0 || I % 128 != 0 || H > 128 * kMaxKB) return kErrBadShape;
  if (top_k <= 0) return kErrBadTopK;
  if (E <= 0) return kErrBadExperts;
  if (!block_m_ok(BM)) return kErrBadBlockSize;
  int TM = resolve_tile_m(tile_m, BM, S, E);
  if (TM < 0) return kErrBadBlockSize;
  // The exact-dot form runs a 256-row tile as two 128-row bodies one after the
  // other; its automatic tile is 128 rows instead (separate 128-row workgroups
  // measured 6-10 % faster on DeepSeek-V3 and Mixtral), over 256-row align
  // blocks as two virtual 128-row blocks each.  Results do not depend on the
  // tile height.
  int vshift = 0;
  if (exact && tile_m == 0 && TM == 256) {
    TM = 128;
    vshift = BM == 256 ? 1 : 0;
  }
  if (max_padded == 0 || S == 0) return kOk;
  if (!Aq || !A_scale || !W13 || !W13_scale || !sorted_ids || !expert_ids || !ntpp || !hq || !hs)
    return kErrNullPointer;
  if (!aligned16(Aq) || !aligned16(W13) || !aligned16(hq)) return kErrBadShape;
  if (!offsets_fit((S + top_k - 1) / top_k, 2 * I, H)) return kErrBadShape;
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
  g.max_blocks = (max_padded + (BM >> vshift) - 1) / (BM >> vshift);
  g.n_tiles = I / 128;
  g.bma = BM;
  g.vshift = vshift;
  g.top_k = top_k;
  g.a_by_pos = 0;
  g.E = E;
  dense_strides(g);
  if (scales_by_pos) g.as_pos_ld = g.hs_pos_ld = max_padded;
  return exact ? dispatch_gemm<true, true>(TM, g, (hipStream_t)stream) : dispatch_gemm<true>(TM, g, (hipStream_t)stream);
}

extern "C" int moe_gemm_w13_silu_quant_tiled(const void* Aq, const float* A_scale, const void* W13,
                                             const float* W13_scale, const int32_t* sorted_ids,
                                             const int32_t* expert_ids, const int32_t* ntpp, int64_t S,
                                             int32_t top_k, int64_t H, int64_t I, int32_t E, int32_t BM,
                                             int64_t max_padded, int32_t tile_m, void* hq, float* hs,
                                             void* stream) {
  return w13_gemm(Aq, A_scale, W13, W13_scale, sorted_ids, expert_ids, ntpp, S, top_k, H, I, E, BM, max_padded,
                  tile_m, false, false, hq, hs, stream);
}

extern "C" int moe_gemm_w13_silu_quant_pos(const void* Aq, const float* A_scale_pos, const void* W13,
                                           const float* W13_scale, const int32_t* sorted_ids,
                                           const int32_t* expert_ids, const int32_t* ntpp, int64_t S,
                                           int32_t top_k, int64_t H, int64_t I, int32_t E, int32_t BM,
                                           int64_t max_padded, int32_t tile_m, void* hq, float* hs_pos,
                                           void* stream) {
  return w13_gemm(Aq, A_scale_pos, W13, W13_scale, sorted_ids, expert_ids, ntpp, S, top_k, H, I, E, BM, max_padded,
                  tile_m, true, false, hq, hs_pos, stream);
}

extern "C" int moe_gemm_w13_silu_quant_exact(const void* Aq, const float* A_scale, const void* W13,
                                             const float* W13_scale, const int32_t* sorted_ids,
                                             const int32_t* expert_ids, const int32_t* ntpp, int64_t S,
                                             int32_t top_k, int64_t H, int64_t I, int32_t E, int32_t BM,
                                             int64_t max_padded, int32_t tile_m, int32_t scales_by_position,
                                             void* hq, float* hs, void* stream) {
  return w13_gemm(Aq, A_scale, W13, W13_scale, sorted_ids, expert_ids, ntpp, S, top_k, H, I, E, BM, max_padded,
                  tile_m, scales_by_position != 0, true, hq, hs, stream);
}

namespace moe {

// out[kb * max_padded + p] = scales[row(p) * groups + kb], row(p) =
// sorted[p] / top_k for the positions p < ntpp that hold a slot and row 0
// otherwise -- the A row the row-major path reads for a padding position, so
// both layouts give the same outputs at every position.
// One thread per (position, 4 K blocks), positions fastest, so each K block's
// row of out is written coalesced and every thread has one load in flight.
template <bool VEC4>
__global__ __launch_bounds__(256) void gather_scales_kernel(const float* __restrict__ scales, int64_t groups,
                                                            const int32_t* __restrict__ sorted,
                                                            const int32_t* __restrict__ ntpp, int64_t S,
                                                            int top_k, int64_t max_padded,
                                                            float* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t chunks = (groups + 3) / 4;
  if (idx >= max_padded * chunks) return;
  const int64_t c = idx / max_padded, p = idx % max_padded;
  int64_t row = 0;
  if (p < *ntpp) {
    const int32_t slot = sorted[p];
    if (slot < S) row = slot / top_k;
  }
  const int64_t kb0 = 4 * c;
  const float* src = scales + row * groups + kb0;
  if constexpr (VEC4) {
    const v4f v = *reinterpret_cast<const v4f*>(src);
#pragma unroll
    for (int q = 0; q < 4; ++q) out[(kb0 + q) * max_padded + p] = v[q];
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (kb0 + q < groups) out[(kb0 + q) * max_padded + p] = src[q];
  }
}

}  // namespace moe

extern "C" int moe_gather_scales_by_position(const float* scales, int64_t rows, int64_t groups,
                                             const int32_t* sorted_ids, const int32_t* ntpp, int64_t S,
                                             int32_t top_k, int64_t max_padded, float* out, void* stream) {
  if (rows < 0 || groups <= 0 || S < 0 || max_padded < 0) return kErrBadShape;
  if (top_k <= 0) return kErrBadTopK;
  if (max_padded == 0) return kOk;
  if (!scales || !sorted_ids || !ntpp || !out) return kErrNullPointer;
  if (rows < (S + top_k - 1) / top_k) return kErrCapacity;
  const unsigned blocks = (unsigned)((max_padded * ((groups + 3) / 4) + 255) / 256);
  if (groups % 4 == 0 && ((uintptr_t)scales & 15) == 0)
    hipLaunchKernelGGL(gather_scales_kernel<true>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, scales, groups,
                       sorted_ids, ntpp, S, (int)top_k, max_padded, out);
  else
    hipLaunchKernelGGL(gather_scales_kernel<false>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, scales, groups,
                       sorted_ids, ntpp, S, (int)top_k, max_padded, out);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

extern "C" int moe_gemm_w13_silu_quant(const void* Aq, const float* A_scale, const void* W13,
                                       const float* W13_scale, const int32_t* sorted_ids,
                                       const int32_t* expert_ids, const int32_t* ntpp, int64_t S,
                                       int32_t top_k, int64_t H, int64_t I, int32_t E,
                                       int32_t BM, int64_t max_padded, void* hq, float* hs,
                                       void* stream) {
  return moe_gemm_w13_silu_quant_tiled(Aq, A_scale, W13, W13_scale, sorted_ids, expert_ids, ntpp, S, top_k,
                                       H, I, E, BM, max_padded, 0, hq, hs, stream);
}
