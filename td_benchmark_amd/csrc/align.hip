// A3: moe_align_block_size -- sort token slots by expert and pad every
// expert's run to a multiple of the GEMM block size BM.
//
// Semantics (reference call sites overlap/overlap_forward.py:165-169, padded
// cumsum of tdx/kernels/moe_utils.py:168-217, pad value = number of valid
// slots as overlap/kernels.py:108-110 masks it):
//   c_e = #slots with expert e, p_e = ceil(c_e/BM)*BM, off_e = sum_{e'<e} p_e'
//   sorted_ids[off_e + j] = j-th slot (flat t*top_k+i, ascending) of expert e
//   sorted_ids[...]      = S at every padding position and in the tail
//   expert_ids[b]        = e for the blocks of e, -1 for blocks >= ntpp/BM
//   ntpp                 = sum_e p_e
// The within-expert order is the stable (ascending slot) order, so the result
// is deterministic and bit-exact against the CPU restatement.
//
// Small problems (S <= 1024, E <= 256) take one launch (align_small_kernel);
// otherwise three launches, none of which waits on another workgroup:
//   1. count:  1024 slots per workgroup.  Slots with equal expert inside a wave
//      are found with log2(E) ballots (a match-any built from per-bit ballots),
//      giving each slot its rank among equal-expert slots of its wave; per-wave
//      counts in LDS are prefix-summed across the 16 waves, giving each slot its
//      rank within the chunk and each chunk its per-expert count.
//   2. scan:   one workgroup scans the chunk counts per expert (column-wise,
//      from LDS), pads, scans across experts, and writes the expert offsets,
//      counts and ntpp; the chunk counts become within-expert chunk bases.
//   3. place:  a wide pass: sorted_ids[off[e] + chunk_base[chunk][e] + rank[s]]
//      = s for every slot, S at every padding position, and expert_ids for
//      every block (the expert of a position comes from a binary search over
//      the offsets held in LDS).
// Align moves well under 2 MB at every configuration, so it is latency-bound.
#include <mutex>

#include "common.hpp"

namespace moe {

constexpr int kAlignChunk = 1024;   // slots per count workgroup (16 waves)
constexpr int kAlignMaxExperts = 1024;
constexpr int64_t kAlignStageLimit = 32768;  // chunk counts staged in LDS up to 128 KiB

__global__ __launch_bounds__(kAlignChunk) void align_count_kernel(
    const int32_t* __restrict__ ids, int64_t S, int E, int nbits,
    int32_t* __restrict__ chunk_count, int32_t* __restrict__ rank) {
  extern __shared__ int32_t wcnt[];  // [16][E]
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int64_t s = (int64_t)blockIdx.x * kAlignChunk + tid;
  for (int i = tid; i < 16 * E; i += kAlignChunk) wcnt[i] = 0;
  int e = -1;
  if (s < S) e = ids[s];
  const bool valid = (e >= 0) && (e < E);
  uint64_t m = __ballot(valid);
  for (int b = 0; b < nbits; ++b) {
    const bool bit = (e >> b) & 1;
    const uint64_t bb = __ballot(bit);
    m &= bit ? bb : ~bb;
  }
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int rank_in_wave = __popcll(m & lt);
  __syncthreads();
  if (valid && rank_in_wave == 0) wcnt[wave * E + e] = __popcll(m);
  __syncthreads();
  for (int x = tid; x < E; x += kAlignChunk) {
    int run = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
      int t = wcnt[w * E + x];
      wcnt[w * E + x] = run;
      run += t;
    }
    chunk_count[(int64_t)blockIdx.x * E + x] = run;
  }
  __syncthreads();
  if (valid) rank[s] = wcnt[wave * E + e] + rank_in_wave;
}

// One workgroup: per-expert totals and the within-expert base of every chunk
// (column prefix sums of the chunk counts, staged in LDS when they fit), then
// padded sizes and their exclusive scan across experts.  Writes off[0..E]
// (off[E] = ntpp), cnt[0..E) and ntpp; every fill is left to the wide place
// kernel.
__global__ __launch_bounds__(kAlignMaxExperts) void align_scan_kernel(
    int32_t* __restrict__ chunk_count, int64_t n_chunks, int E, int BM, int use_lds,
    int32_t* __restrict__ off_out, int32_t* __restrict__ cnt_out, int32_t* __restrict__ ntpp_out) {
  extern __shared__ int32_t staged[];  // [n_chunks][E] when use_lds
  __shared__ int32_t wave_tot[kAlignMaxExperts / 64];
  const int tid = threadIdx.x;
  const int e = tid;
  if (use_lds) {
    for (int64_t i = tid; i < n_chunks * E; i += kAlignMaxExperts) staged[i] = chunk_count[i];
    __syncthreads();
  }
  int cnt = 0;
  if (e < E) {
    if (use_lds) {
      for (int64_t c = 0; c < n_chunks; ++c) {
        const int v = staged[c * E + e];
        chunk_count[c * E + e] = cnt;
        cnt += v;
      }
    } else {
      int64_t c = 0;
      for (; c + 8 <= n_chunks; c += 8) {
        int v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = chunk_count[(c + j) * E + e];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          chunk_count[(c + j) * E + e] = cnt;
          cnt += v[j];
        }
      }
      for (; c < n_chunks; ++c) {
        const int v = chunk_count[c * E + e];
        chunk_count[c * E + e] = cnt;
        cnt += v;
      }
    }
  }
  const int padded = (e < E) ? (cnt + BM - 1) / BM * BM : 0;
  // Block-wide exclusive scan of `padded` (wave inclusive scan + wave totals).
  const int lane = tid & 63, wave = tid >> 6;
  int incl = padded;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wave_tot[wave] = incl;
  __syncthreads();
  if (tid < 64) {
    // exclusive scan of the 16 wave totals by the first wave
    const int t = tid < kAlignMaxExperts / 64 ? wave_tot[tid] : 0;
    int x = t;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const int y = __shfl_up(x, o);
      if (lane >= o) x += y;
    }
    if (tid < kAlignMaxExperts / 64) wave_tot[tid] = x - t;
    if (tid == kAlignMaxExperts / 64 - 1) {
      off_out[E] = x;
      *ntpp_out = x;
    }
  }
  __syncthreads();
  if (e < E) {
    off_out[e] = wave_tot[wave] + incl - padded;
    cnt_out[e] = cnt;
  }
}

// Wide pass over max(S, max_padded) indices: slot i goes to
// off[e] + chunk_base[chunk][e] + rank[i]; position i is set to S when it is
// padding (inside an expert's run past its count, or past ntpp), and the first
// position of every block writes that block's expert (-1 past ntpp).  Valid
// and padding positions are disjoint, so no two threads write one element.
__global__ __launch_bounds__(256) void align_place_kernel(
    const int32_t* __restrict__ ids, int64_t S, int E, int BM, const int32_t* __restrict__ chunk_base,
    const int32_t* __restrict__ rank, const int32_t* __restrict__ off, const int32_t* __restrict__ cnt,
    const int32_t* __restrict__ expert_map, int32_t* __restrict__ sorted_ids,
    int32_t* __restrict__ expert_ids, int64_t max_padded) {
  __shared__ int32_t s_off[kAlignMaxExperts + 1];
  __shared__ int32_t s_cnt[kAlignMaxExperts];
  for (int i = threadIdx.x; i <= E; i += 256) s_off[i] = off[i];
  for (int i = threadIdx.x; i < E; i += 256) s_cnt[i] = cnt[i];
  __syncthreads();
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < S) {
    const int e = ids[i];
    if (e >= 0 && e < E) {
      const int64_t chunk = i / kAlignChunk;
      sorted_ids[s_off[e] + chunk_base[chunk * E + e] + rank[i]] = (int32_t)i;
    }
  }
  if (i < max_padded) {
    const int total = s_off[E];
    int e = -1;
    bool pad = true;
    if (i < total) {
      int lo = 0, hi = E - 1;  // largest e with off[e] <= i
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_off[mid] <= i) lo = mid;
        else hi = mid - 1;
      }
      e = lo;
      pad = (i - s_off[e]) >= s_cnt[e];
    }
    if (pad) sorted_ids[i] = (int32_t)S;
    // With an expert map (global -> local id, -1 = not on this device) the
    // block's expert is reported as its local id.
    if (i % BM == 0) expert_ids[i / BM] = (expert_map && e >= 0) ? expert_map[e] : e;
  }
}

// Small problems (S <= 1024 slots, E <= 256 experts) in one launch: one
// workgroup walks the slots 1024 at a time, keeping running per-expert counts
// in LDS so every slot gets its rank within its expert (the same stable order
// as the three-kernel path), then scans, places and fills like the wide pass.
// Measured on MI355X: faster than the three launches for one chunk of slots
// (and half the launches when the host issues them), slower from ~2 chunks on,
// where the serial chunk loop outweighs the saved launches.
constexpr int64_t kAlignSmallSlots = 1024;
constexpr int kAlignSmallExperts = 256;

__global__ __launch_bounds__(kAlignChunk) void align_small_kernel(
    const int32_t* __restrict__ ids, int64_t S, int E, int nbits, int BM,
    const int32_t* __restrict__ expert_map, int32_t* __restrict__ sorted_ids,
    int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntpp_out, int64_t max_padded) {
  extern __shared__ int32_t lds[];
  int32_t* wcnt = lds;                         // [16][E]
  int32_t* base = wcnt + 16 * E;               // [E] running counts
  int32_t* s_off = base + E;                   // [E + 1]
  int32_t* s_e = s_off + E + 1;                // [S] expert of each slot (-1 = dropped)
  int32_t* s_rank = s_e + S;                   // [S] rank of the slot within its expert
  __shared__ int32_t wave_tot[kAlignChunk / 64];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  for (int i = tid; i < E; i += kAlignChunk) base[i] = 0;
  for (int64_t c0 = 0; c0 < S; c0 += kAlignChunk) {
    for (int i = tid; i < 16 * E; i += kAlignChunk) wcnt[i] = 0;
    const int64_t sl = c0 + tid;
    int e = -1;
    if (sl < S) e = ids[sl];
    const bool valid = (e >= 0) && (e < E);
    uint64_t m = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (e >> b) & 1;
      const uint64_t bb = __ballot(bit);
      m &= bit ? bb : ~bb;
    }
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const int rank_in_wave = __popcll(m & lt);
    __syncthreads();
    if (valid && rank_in_wave == 0) wcnt[wave * E + e] = __popcll(m);
    __syncthreads();
    for (int x = tid; x < E; x += kAlignChunk) {
      int run = base[x];
#pragma unroll
      for (int w = 0; w < 16; ++w) {
        const int t = wcnt[w * E + x];
        wcnt[w * E + x] = run;
        run += t;
      }
      base[x] = run;
    }
    __syncthreads();
    if (sl < S) {
      s_e[sl] = valid ? e : -1;
      s_rank[sl] = valid ? wcnt[wave * E + e] + rank_in_wave : 0;
    }
    __syncthreads();
  }
  // padded sizes and their exclusive scan across experts (E <= 256 < 1024 threads)
  const int cnt = tid < E ? base[tid] : 0;
  const int padded = (cnt + BM - 1) / BM * BM;
  int incl = padded;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wave_tot[wave] = incl;
  __syncthreads();
  if (tid < 64) {
    const int t = tid < kAlignChunk / 64 ? wave_tot[tid] : 0;
    int x = t;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const int y = __shfl_up(x, o);
      if (lane >= o) x += y;
    }
    if (tid < kAlignChunk / 64) wave_tot[tid] = x - t;
    if (tid == kAlignChunk / 64 - 1) {
      s_off[E] = x;
      *ntpp_out = x;
    }
  }
  __syncthreads();
  if (tid < E) s_off[tid] = wave_tot[wave] + incl - padded;
  __syncthreads();
  for (int64_t sl = tid; sl < S; sl += kAlignChunk) {
    const int e = s_e[sl];
    if (e >= 0) sorted_ids[s_off[e] + s_rank[sl]] = (int32_t)sl;
  }
  const int total = s_off[E];
  for (int64_t i = tid; i < max_padded; i += kAlignChunk) {
    int e = -1;
    bool pad = true;
    if (i < total) {
      int lo = 0, hi = E - 1;  // largest e with off[e] <= i
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_off[mid] <= i) lo = mid;
        else hi = mid - 1;
      }
      e = lo;
      pad = (i - s_off[e]) >= base[e];
    }
    if (pad) sorted_ids[i] = (int32_t)S;
    if (i % BM == 0) expert_ids[i / BM] = (expert_map && e >= 0) ? expert_map[e] : e;
  }
}

}  // namespace moe

using namespace moe;

extern "C" int64_t moe_align_max_padded(int64_t S, int32_t E, int32_t BM) {
  if (S < 0 || E <= 0 || BM <= 0) return -1;
  int64_t m = S + (int64_t)E * (BM - 1);
  if (S < E) m = (S * BM < m) ? S * BM : m;
  return m;
}

extern "C" int64_t moe_align_workspace_bytes(int64_t S, int32_t E) {
  if (S < 0 || E <= 0) return -1;
  const int64_t n_chunks = (S + kAlignChunk - 1) / kAlignChunk;
  // chunk counts [n_chunks][E], rank [S], off [E+1], cnt [E]
  return 4 * (n_chunks * E + S + 2 * (int64_t)E + 1) + 256;
}

// Every argument check of an align call, before any device work; the
// workspace pointer is checked only when the caller supplies one.
static int align_args(const int32_t* topk_ids, int64_t S, int32_t E, int32_t BM, int32_t* sorted_ids,
                      int32_t* expert_ids, int32_t* ntpp, int64_t max_padded, bool need_ws, const void* workspace) {
  if (S < 0) return kErrBadShape;
  if (E <= 0 || E > kAlignMaxExperts) return kErrBadExperts;
  if (!block_m_ok(BM)) return kErrBadBlockSize;
  if (!sorted_ids || !expert_ids || !ntpp || (need_ws && !workspace) || (S > 0 && !topk_ids))
    return kErrNullPointer;
  if (max_padded < moe_align_max_padded(S, E, BM)) return kErrCapacity;
  if (S > 0x7FFFFFFF - 1 || max_padded > 0x7FFFFFFF) return kErrBadShape;
  return kOk;
}

static int align_impl(const int32_t* topk_ids, int64_t S, int32_t E, int32_t BM, const int32_t* expert_map,
                      int32_t* sorted_ids, int32_t* expert_ids, int32_t* ntpp, int64_t max_padded,
                      void* workspace, void* stream) {
  const int arg_rc = align_args(topk_ids, S, E, BM, sorted_ids, expert_ids, ntpp, max_padded, true, workspace);
  if (arg_rc != kOk) return arg_rc;
  hipStream_t st = (hipStream_t)stream;
  int nbits0 = 0;
  while ((1 << nbits0) < E) ++nbits0;
  if (S > 0 && S <= kAlignSmallSlots && E <= kAlignSmallExperts) {
    const size_t lds = (size_t)(16 * E + E + E + 1 + 2 * S) * sizeof(int32_t);
    hipLaunchKernelGGL(align_small_kernel, dim3(1), dim3(kAlignChunk), lds, st, topk_ids, S, (int)E, nbits0,
                       (int)BM, expert_map, sorted_ids, expert_ids, ntpp, max_padded);
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
  }
  const int64_t n_chunks = (S + kAlignChunk - 1) / kAlignChunk;
  int32_t* chunk_count = (int32_t*)workspace;
  int32_t* rank = chunk_count + n_chunks * E;
  int32_t* off = rank + S;
  int32_t* cnt = off + E + 1;
  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  if (n_chunks > 0) {
    hipLaunchKernelGGL(align_count_kernel, dim3((unsigned)n_chunks), dim3(kAlignChunk),
                       16 * E * sizeof(int32_t), st, topk_ids, S, (int)E, nbits, chunk_count,
                       rank);
  }
  // Stage the chunk counts in LDS when they fit (128 KiB of the 160 KiB).
  // Set once per process (thread-safe initialisation of a function-local static).
  static const hipError_t lds_attr_rc = hipFuncSetAttribute(
      (const void*)align_scan_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
      (int)(kAlignStageLimit * sizeof(int32_t)));
  if (lds_attr_rc != hipSuccess) return kErrLaunch;
  const int use_lds = n_chunks * E <= kAlignStageLimit ? 1 : 0;
  hipLaunchKernelGGL(align_scan_kernel, dim3(1), dim3(kAlignMaxExperts),
                     use_lds ? (size_t)(n_chunks * E * sizeof(int32_t)) : 0, st, chunk_count, n_chunks,
                     (int)E, (int)BM, use_lds, off, cnt, ntpp);
  const int64_t wide = S > max_padded ? S : max_padded;
  if (wide > 0) {
    hipLaunchKernelGGL(align_place_kernel, dim3((unsigned)((wide + 255) / 256)), dim3(256), 0, st,
                       topk_ids, S, (int)E, (int)BM, chunk_count, rank, off, cnt, expert_map,
                       sorted_ids, expert_ids, max_padded);
  }
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

extern "C" int moe_align_block_size(const int32_t* topk_ids, int64_t S, int32_t E, int32_t BM,
                                    int32_t* sorted_ids, int32_t* expert_ids, int32_t* ntpp,
                                    int64_t max_padded, void* workspace, void* stream) {
  return align_impl(topk_ids, S, E, BM, nullptr, sorted_ids, expert_ids, ntpp, max_padded, workspace, stream);
}

extern "C" int moe_align_block_size_mapped(const int32_t* topk_ids, int64_t S, int32_t E, int32_t BM,
                                           const int32_t* expert_map, int32_t* sorted_ids,
                                           int32_t* expert_ids, int32_t* ntpp, int64_t max_padded,
                                           void* workspace, void* stream) {
  if (!expert_map) return kErrNullPointer;
  return align_impl(topk_ids, S, E, BM, expert_map, sorted_ids, expert_ids, ntpp, max_padded, workspace,
                    stream);
}

// ---------------------------------------------------------------------------
// Allocation-free align: the same three kernels with their workspace in a
// file-scope device array instead of caller memory, for callers that cannot
// allocate (code under graph capture, tight serving loops).  Each GPU holds
// its own copy of the array until the process ends; every call on a GPU
// shares it, so calls that overlap on one GPU race.  Nothing in the workspace
// needs clearing: every call writes each chunk count, rank, offset and count
// that it later reads.

namespace moe {

constexpr int64_t kNoAllocScratchBytes = MOE_ALIGN_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

// The array's device address on the current GPU, looked up once per device
// with that device current (the host-side name is only a stand-in).
static int scratch_for_current_device(void** out) {
  static std::mutex mu;
  static void* ptr[kMaxDevices] = {};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return kErrLaunch;
  std::lock_guard<std::mutex> lock(mu);
  if (!ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return kErrLaunch;
    ptr[dev] = p;
  }
  *out = ptr[dev];
  return kOk;
}

}  // namespace moe

extern "C" int moe_align_block_size_noalloc(const int32_t* topk_ids, int64_t S, int32_t E, int32_t BM,
                                            int32_t* sorted_ids, int32_t* expert_ids, int32_t* ntpp,
                                            int64_t max_padded, void* stream) {
  // every argument is checked before the device is touched (symbol lookup)
  const int arg_rc = align_args(topk_ids, S, E, BM, sorted_ids, expert_ids, ntpp, max_padded, false, nullptr);
  if (arg_rc != kOk) return arg_rc;
  if (moe_align_workspace_bytes(S, E) > kNoAllocScratchBytes) return kErrCapacity;
  void* ws = nullptr;
  const int rc = scratch_for_current_device(&ws);
  if (rc != kOk) return rc;
  return align_impl(topk_ids, S, E, BM, nullptr, sorted_ids, expert_ids, ntpp, max_padded, ws, stream);
}
