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
// Three launches, none of which waits on another workgroup:
//   1. count:  1024 slots per workgroup.  Slots with equal expert inside a wave
//      are found with log2(E) ballots (a match-any built from per-bit ballots),
//      giving each slot its rank among equal-expert slots of its wave; per-wave
//      counts in LDS are prefix-summed across the 16 waves, giving each slot its
//      rank within the chunk and each chunk its per-expert count.
//   2. scan:   one workgroup scans the chunk counts per expert (column-wise),
//      pads, scans across experts, writes expert_ids / ntpp / pad fill, and
//      turns the chunk counts into chunk base positions.
//   3. place:  sorted_ids[chunk_base[chunk][e] + rank[s]] = s.
// Align moves well under 2 MB at every configuration, so it is latency-bound.
#include "common.hpp"

namespace moe {

constexpr int kAlignChunk = 1024;   // slots per count workgroup (16 waves)
constexpr int kAlignMaxExperts = 1024;

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

__global__ __launch_bounds__(kAlignMaxExperts) void align_scan_kernel(
    int32_t* __restrict__ chunk_count, int64_t n_chunks, int E, int BM, int64_t S,
    int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
    int32_t* __restrict__ ntpp_out, int64_t max_padded) {
  __shared__ int32_t pad_scan[kAlignMaxExperts];
  __shared__ int32_t wave_tot[kAlignMaxExperts / 64];
  const int tid = threadIdx.x;
  const int e = tid;
  int cnt = 0;
  if (e < E) {
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
      int v = chunk_count[c * E + e];
      chunk_count[c * E + e] = cnt;
      cnt += v;
    }
  }
  const int padded = (e < E) ? (cnt + BM - 1) / BM * BM : 0;
  // Block-wide exclusive scan of `padded` (wave inclusive scan + wave totals).
  const int lane = tid & 63, wave = tid >> 6;
  int incl = padded;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wave_tot[wave] = incl;
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int w = 0; w < kAlignMaxExperts / 64; ++w) {
      int t = wave_tot[w];
      wave_tot[w] = run;
      run += t;
    }
    pad_scan[0] = run;  // total, read below after the barrier
  }
  __syncthreads();
  const int total = pad_scan[0];
  const int off = wave_tot[wave] + incl - padded;
  if (e < E) {
    for (int64_t c = 0; c < n_chunks; ++c) chunk_count[c * E + e] += off;
    for (int b = off / BM; b < (off + padded) / BM; ++b) expert_ids[b] = e;
    for (int p = off + cnt; p < off + padded; ++p) sorted_ids[p] = (int32_t)S;
  }
  const int64_t max_blocks = (max_padded + BM - 1) / BM;
  for (int64_t b = total / BM + tid; b < max_blocks; b += kAlignMaxExperts) expert_ids[b] = -1;
  for (int64_t p = total + tid; p < max_padded; p += kAlignMaxExperts) sorted_ids[p] = (int32_t)S;
  if (tid == 0) *ntpp_out = total;
}

__global__ __launch_bounds__(256) void align_place_kernel(
    const int32_t* __restrict__ ids, int64_t S, int E, const int32_t* __restrict__ chunk_base,
    const int32_t* __restrict__ rank, int32_t* __restrict__ sorted_ids) {
  const int64_t s = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (s >= S) return;
  const int e = ids[s];
  if (e < 0 || e >= E) return;
  const int64_t chunk = s / kAlignChunk;
  sorted_ids[chunk_base[chunk * E + e] + rank[s]] = (int32_t)s;
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
  return 4 * (n_chunks * E + S) + 256;
}

extern "C" int moe_align_block_size(const int32_t* topk_ids, int64_t S, int32_t E, int32_t BM,
                                    int32_t* sorted_ids, int32_t* expert_ids, int32_t* ntpp,
                                    int64_t max_padded, void* workspace, void* stream) {
  if (S < 0) return kErrBadShape;
  if (E <= 0 || E > kAlignMaxExperts) return kErrBadExperts;
  if (BM != 16 && BM != 32 && BM != 64 && BM != 128) return kErrBadBlockSize;
  if (!sorted_ids || !expert_ids || !ntpp || !workspace || (S > 0 && !topk_ids))
    return kErrNullPointer;
  if (max_padded < moe_align_max_padded(S, E, BM)) return kErrCapacity;
  if (S > 0x7FFFFFFF - 1 || max_padded > 0x7FFFFFFF) return kErrBadShape;
  hipStream_t st = (hipStream_t)stream;
  const int64_t n_chunks = (S + kAlignChunk - 1) / kAlignChunk;
  int32_t* chunk_count = (int32_t*)workspace;
  int32_t* rank = chunk_count + n_chunks * E;
  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  if (n_chunks > 0) {
    hipLaunchKernelGGL(align_count_kernel, dim3((unsigned)n_chunks), dim3(kAlignChunk),
                       16 * E * sizeof(int32_t), st, topk_ids, S, (int)E, nbits, chunk_count,
                       rank);
  }
  hipLaunchKernelGGL(align_scan_kernel, dim3(1), dim3(kAlignMaxExperts), 0, st, chunk_count,
                     n_chunks, (int)E, (int)BM, S, sorted_ids, expert_ids, ntpp, max_padded);
  if (S > 0) {
    hipLaunchKernelGGL(align_place_kernel, dim3((unsigned)((S + 255) / 256)), dim3(256), 0, st,
                       topk_ids, S, (int)E, chunk_count, rank, sorted_ids);
  }
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}
