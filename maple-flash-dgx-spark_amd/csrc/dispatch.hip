// Token-to-expert dispatch: per-expert lists of (token, slot) pairs (gfx950).
//
// There is no reference function (the reference grids over pairs,
// src/maple_run/kernels/ternary_expert.py:210,443); the definition is the
// stable counting sort of pairs p = t * top_k + j by expert id:
//   counts[e], offsets[e] = exclusive scan (offsets[E] = n_pairs),
//   pair_ids = pairs in (expert, p) order, inverse[pair_ids[i]] = i.
//
// One 1024-thread workgroup.  Each of the 16 waves owns a contiguous range of
// pairs and walks it 64 at a time.  Lanes holding the same expert find each
// other with ballots over the bits of the id (a match-any), the lowest such
// lane is the group's leader, and a lane's rank inside the group is the
// popcount of the group mask below it.  Pass 1 counts per (wave, expert);
// a scan turns the counts into per-(wave, expert) bases; pass 2 writes every
// pair at base + rank, so the order inside an expert is the pair order.
#include "common.h"

namespace ma {

constexpr int kDispatchWaves = 16;
constexpr int kDispatchMaxExperts = 512;  // 32 KB of LDS counters

// Mask of the lanes whose (valid) expert id equals this lane's.
__device__ __forceinline__ uint64_t match_any(int e, int bits, bool valid) {
  uint64_t m = __ballot(valid);
  for (int b = 0; b < bits; ++b) {
    const uint64_t set = __ballot(valid && ((e >> b) & 1));
    m &= ((e >> b) & 1) ? set : ~set;
  }
  return valid ? m : 0ull;
}

__global__ __launch_bounds__(1024) void k_dispatch(const void* __restrict__ ids, int ids64,
                                                   int64_t n_pairs, int n_exp, int bits,
                                                   int32_t* __restrict__ counts,
                                                   int32_t* __restrict__ offsets,
                                                   int32_t* __restrict__ pair_ids,
                                                   int32_t* __restrict__ inverse) {
  // base[w][e]: pass 1 counts, then running write positions.
  __shared__ int32_t base[kDispatchWaves][kDispatchMaxExperts];
  __shared__ int32_t wave_tot[kDispatchWaves];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wv = tid >> 6;
  for (int i = tid; i < kDispatchWaves * n_exp; i += 1024) base[i / n_exp][i % n_exp] = 0;
  __syncthreads();

  const int64_t chunk = ((n_pairs + kDispatchWaves - 1) / kDispatchWaves + 63) / 64 * 64;
  const int64_t p0 = wv * chunk;
  const int64_t p1 = p0 + chunk < n_pairs ? p0 + chunk : n_pairs;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));

  // Pass 1: per-wave counts.
  for (int64_t p = p0; p < p1; p += 64) {
    const int64_t q = p + lane;
    const bool valid = q < p1;
    int e = valid ? static_cast<int>(ld_id(ids, ids64, q)) : 0;
    e = e < 0 ? 0 : (e >= n_exp ? n_exp - 1 : e);
    const uint64_t m = match_any(e, bits, valid);
    if (valid && (m & below) == 0) base[wv][e] += __popcll(m);
  }
  __syncthreads();

  // Scan: expert totals, exclusive offsets, per-wave bases.
  int32_t tot = 0;
  const int e = tid;
  if (e < n_exp)
    for (int w = 0; w < kDispatchWaves; ++w) tot += base[w][e];
  // block-wide exclusive scan of tot over e (1024 threads)
  int32_t incl = tot;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int32_t v = __shfl_up(incl, off, 64);
    if (lane >= off) incl += v;
  }
  if (lane == 63) wave_tot[wv] = incl;
  __syncthreads();
  int32_t wave_base = 0;
  for (int w = 0; w < wv; ++w) wave_base += wave_tot[w];
  const int32_t excl = wave_base + incl - tot;
  if (e < n_exp) {
    counts[e] = tot;
    offsets[e] = excl;
    int32_t run = excl;
    for (int w = 0; w < kDispatchWaves; ++w) {
      const int32_t c = base[w][e];
      base[w][e] = run;
      run += c;
    }
  }
  if (tid == 0) offsets[n_exp] = static_cast<int32_t>(n_pairs);
  __syncthreads();

  // Pass 2: stable placement.
  for (int64_t p = p0; p < p1; p += 64) {
    const int64_t q = p + lane;
    const bool valid = q < p1;
    int ee = valid ? static_cast<int>(ld_id(ids, ids64, q)) : 0;
    ee = ee < 0 ? 0 : (ee >= n_exp ? n_exp - 1 : ee);
    const uint64_t m = match_any(ee, bits, valid);
    int32_t pos = 0;
    if (valid) {
      pos = base[wv][ee] + __popcll(m & below);
      pair_ids[pos] = static_cast<int32_t>(q);
      inverse[q] = pos;
    }
    __builtin_amdgcn_wave_barrier();
    if (valid && (m & below) == 0) base[wv][ee] += __popcll(m);
    __builtin_amdgcn_wave_barrier();
  }
}

}  // namespace ma

using namespace ma;

extern "C" int ma_moe_dispatch(const void* ids, int ids_is_int64, int64_t n_pairs, int n_experts,
                               int32_t* counts, int32_t* offsets, int32_t* pair_ids,
                               int32_t* inverse, void* stream) {
  if (n_pairs < 0 || n_pairs > 0x7fffffff) return fail(MA_EVALUE, "moe_dispatch: bad n_pairs");
  if (n_experts < 1 || n_experts > kDispatchMaxExperts)
    return fail(MA_EVALUE, "moe_dispatch: n_experts must be in [1, %d]", kDispatchMaxExperts);
  int bits = 0;
  while ((1 << bits) < n_experts) ++bits;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), 0, s, ids, ids_is_int64, n_pairs,
                     n_experts, bits, counts, offsets, pair_ids, inverse);
  return check_launch("moe_dispatch");
}
