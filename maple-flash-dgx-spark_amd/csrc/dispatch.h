// Stable counting sort of (token, slot) pairs by expert id, run by one
// workgroup of NW waves (the dispatch lists of the grouped MoE path).
//
// There is no reference function (the reference grids over pairs,
// src/maple_run/kernels/ternary_expert.py:210,443); the definition is the
// stable counting sort of pairs p = t * top_k + j by expert id:
//   counts[e], offsets[e] = exclusive scan (offsets[E] = n_pairs),
//   pair_ids = pairs in (expert, p) order, inverse[pair_ids[i]] = i.
//
// Each of the NW waves owns a contiguous range of pairs and walks it 64 at a
// time.  Lanes holding the same expert find each other with ballots over the
// bits of the id (a match-any), the lowest such lane is the group's leader,
// and a lane's rank inside the group is the popcount of the group mask below
// it.  Pass 1 counts per (wave, expert) with LDS atomic adds (integers: the
// order does not matter); a scan turns the counts into
// per-(wave, expert) bases; pass 2 writes every pair at base + rank, so the
// order inside an expert is the pair order.
#pragma once

#include "common.h"

namespace ma {

constexpr int kIdBatch = 8;  // rows of 64 pairs whose ids a wave loads at once

// Mask of the lanes whose (valid) expert id equals this lane's.
__device__ __forceinline__ uint64_t match_any(int e, int bits, bool valid) {
  uint64_t m = __ballot(valid);
  for (int b = 0; b < bits; ++b) {
    const uint64_t set = __ballot(valid && ((e >> b) & 1));
    m &= ((e >> b) & 1) ? set : ~set;
  }
  return valid ? m : 0ull;
}

// n_exp <= 64 * NW and <= MAXE; load_id(q) returns pair q's expert id.
// base: LDS [NW][MAXE], wave_tot: LDS [NW].  All NW * 64 threads call this.
template <int NW, int MAXE, typename LoadId>
__device__ __forceinline__ void dispatch_block(LoadId load_id, int64_t n_pairs, int n_exp,
                                               int bits, int32_t (*base)[MAXE],
                                               int32_t* wave_tot, int32_t* __restrict__ counts,
                                               int32_t* __restrict__ offsets,
                                               int32_t* __restrict__ pair_ids,
                                               int32_t* __restrict__ inverse) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wv = tid >> 6;
  for (int i = tid; i < NW * n_exp; i += 64 * NW) base[i / n_exp][i % n_exp] = 0;
  __syncthreads();

  const int64_t chunk = ((n_pairs + NW - 1) / NW + 63) / 64 * 64;
  const int64_t p0 = wv * chunk;
  const int64_t p1 = p0 + chunk < n_pairs ? p0 + chunk : n_pairs;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));

  // Pass 1: per-wave counts.  The ids of kIdBatch rows of 64 pairs are
  // loaded together, so a wave waits for memory once per batch.
  for (int64_t pb = p0; pb < p1; pb += 64 * kIdBatch) {
    int eb[kIdBatch];
#pragma unroll
    for (int u = 0; u < kIdBatch; ++u) {  // unconditional loads (clamped index): no wait between them
      const int64_t q = pb + 64 * u + lane;
      eb[u] = load_id(q < p1 ? q : p1 - 1);
    }
#pragma unroll
    for (int u = 0; u < kIdBatch; ++u) {
      if (pb + 64 * u >= p1) break;  // (wave-uniform) rows past the range
      const int e = eb[u] < 0 ? 0 : (eb[u] >= n_exp ? n_exp - 1 : eb[u]);
      if (pb + 64 * u + lane < p1) atomicAdd(&base[wv][e], 1);  // integer counts: any order
    }
  }
  __syncthreads();

  // Scan: expert totals, exclusive offsets, per-wave bases.
  int32_t tot = 0;
  const int e = tid;
  if (e < n_exp)
    for (int w = 0; w < NW; ++w) tot += base[w][e];
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
    for (int w = 0; w < NW; ++w) {
      const int32_t c = base[w][e];
      base[w][e] = run;
      run += c;
    }
  }
  if (tid == 0) offsets[n_exp] = static_cast<int32_t>(n_pairs);
  __syncthreads();

  // Pass 2: stable placement (ids batched as in pass 1).
  for (int64_t pb = p0; pb < p1; pb += 64 * kIdBatch) {
    int eb[kIdBatch];
#pragma unroll
    for (int u = 0; u < kIdBatch; ++u) {  // unconditional loads (clamped index): no wait between them
      const int64_t q = pb + 64 * u + lane;
      eb[u] = load_id(q < p1 ? q : p1 - 1);
    }
#pragma unroll
    for (int u = 0; u < kIdBatch; ++u) {
      if (pb + 64 * u >= p1) break;  // (wave-uniform) rows past the range
      const int64_t q = pb + 64 * u + lane;
      const bool valid = q < p1;
      const int ee = eb[u] < 0 ? 0 : (eb[u] >= n_exp ? n_exp - 1 : eb[u]);
      const uint64_t m = match_any(ee, bits, valid);
      if (valid) {
        const int32_t pos = base[wv][ee] + __popcll(m & below);
        pair_ids[pos] = static_cast<int32_t>(q);
        inverse[q] = pos;
      }
      __builtin_amdgcn_wave_barrier();
      if (valid && (m & below) == 0) base[wv][ee] += __popcll(m);
      __builtin_amdgcn_wave_barrier();
    }
  }
}

}  // namespace ma
