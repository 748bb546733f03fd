// Token-to-expert dispatch: per-expert lists of (token, slot) pairs (gfx950).
// Up to kDispatchOneWg pairs, one 1024-thread workgroup runs the stable
// counting sort of dispatch.h; beyond, k_dispatch_multi spreads the placement
// over several workgroups (one launch, no workspace).
#include "dispatch.h"

namespace ma {

constexpr int kDispatchWaves = 16;
constexpr int kDispatchMaxExperts = 512;  // 32 KB of LDS counters

__global__ __launch_bounds__(1024) void k_dispatch(const void* __restrict__ ids, int ids64,
                                                   int64_t n_pairs, int n_exp, int bits,
                                                   int32_t* __restrict__ counts,
                                                   int32_t* __restrict__ offsets,
                                                   int32_t* __restrict__ pair_ids,
                                                   int32_t* __restrict__ inverse) {
  // base[w][e]: pass 1 counts, then running write positions.
  __shared__ int32_t base[kDispatchWaves][kDispatchMaxExperts];
  __shared__ int32_t wave_tot[kDispatchWaves];
  const int32_t* const id32 = static_cast<const int32_t*>(ids);  // an id's low 32 bits
  dispatch_block<kDispatchWaves, kDispatchMaxExperts>(
      [&](int64_t q) { return id32[q << ids64]; }, n_pairs, n_exp, bits,
      base, wave_tot, counts, offsets, pair_ids, inverse);
}

constexpr int64_t kDispatchOneWg = 4096;     // pairs: one workgroup up to here
constexpr int kDispatchMultiMaxExperts = 256;
constexpr int64_t kDispatchChunk = 1024;     // pairs placed per workgroup of k_dispatch_multi (2048: 8.25 against 7.7 us at 16384 pairs)

// Many pairs: workgroup c places pairs [c * chunk, (c + 1) * chunk).  It
// first counts every pair (its 16 waves take contiguous ranges, kIdBatch rows
// of 64 ids loaded at once): per expert the total, and how many of its pairs
// come before the chunk.  The exclusive scan of the totals gives offsets; the
// chunk's pairs of expert e then start at offsets[e] + (those before), and
// inside the chunk they are placed as dispatch_block places them (per-wave
// counts, wave bases, rank by match-any) -- so the lists are the one stable
// counting sort whatever the number of workgroups.  Workgroup 0 writes
// counts and offsets.
__global__ __launch_bounds__(1024) void k_dispatch_multi(const void* __restrict__ ids, int ids64,
                                                         int64_t n_pairs, int n_exp, int bits,
                                                         int32_t* __restrict__ counts,
                                                         int32_t* __restrict__ offsets,
                                                         int32_t* __restrict__ pair_ids,
                                                         int32_t* __restrict__ inverse) {
  constexpr int NW = kDispatchWaves, MAXE = kDispatchMultiMaxExperts;
  __shared__ int32_t tot[MAXE], bef[MAXE], base[NW][MAXE];
  __shared__ int32_t wave_tot[NW];
  __shared__ int32_t start[MAXE];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * kDispatchChunk;
  const int64_t c1 = c0 + kDispatchChunk < n_pairs ? c0 + kDispatchChunk : n_pairs;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int i = tid; i < NW * n_exp; i += 64 * NW) base[i / n_exp][i % n_exp] = 0;
  if (tid < n_exp) {
    tot[tid] = 0;
    bef[tid] = 0;
  }
  __syncthreads();
  // An id is its low 32 bits (int32 ids, or the low word of int64 ones: the
  // same value as the int64 id cast to int), clamped to [0, n_exp).
  const int32_t* const id32 = static_cast<const int32_t*>(ids);

  // This wave's rows of the chunk (contiguous, in order), loaded first.
  constexpr int RPW = kDispatchChunk / (64 * NW);
  static_assert(RPW * 64 * NW == kDispatchChunk, "chunk rows per wave");
  const int64_t q0 = c0 + static_cast<int64_t>(wv) * 64 * RPW;
  int ec[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t q = q0 + 64 * r + lane;
    ec[r] = id32[(q < c1 ? q : c1 - 1) << ids64];
  }
  // Count every pair: totals and those before this chunk (no ranks needed
  // here, so LDS atomics count them; match-any ranks only the chunk's own).
  {
    const int64_t cw = ((n_pairs + NW - 1) / NW + 63) / 64 * 64;
    const int64_t p0 = wv * cw, p1 = p0 + cw < n_pairs ? p0 + cw : n_pairs;
    for (int64_t pb = p0; pb < p1; pb += 64 * kIdBatch) {
      int eb[kIdBatch];
#pragma unroll
      for (int u = 0; u < kIdBatch; ++u) {  // unconditional loads (clamped index): no wait between them
        const int64_t q = pb + 64 * u + lane;
        eb[u] = id32[(q < p1 ? q : p1 - 1) << ids64];
      }
#pragma unroll
      for (int u = 0; u < kIdBatch; ++u) eb[u] = eb[u] < 0 ? 0 : (eb[u] >= n_exp ? n_exp - 1 : eb[u]);
#pragma unroll
      for (int u = 0; u < kIdBatch; ++u) {
        if (pb + 64 * u >= p1) break;  // (wave-uniform) rows past the range
        const int64_t q = pb + 64 * u + lane;
        if (q < p1) {  // counts only: LDS atomic adds (integers, so any order gives the same)
          atomicAdd(&tot[eb[u]], 1);
          if (q < c0) atomicAdd(&bef[eb[u]], 1);
        }
      }
    }
  }
  __syncthreads();
  // Scan of the totals (n_exp <= 256: the first four waves).
  const int e = tid;
  const int32_t tot_e = e < n_exp ? tot[e] : 0;
  int32_t incl = tot_e;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int32_t v = __shfl_up(incl, off, 64);
    if (lane >= off) incl += v;
  }
  if (lane == 63) wave_tot[wv] = incl;
  __syncthreads();
  int32_t wave_base = 0;
  for (int w = 0; w < wv; ++w) wave_base += wave_tot[w];
  const int32_t excl = wave_base + incl - tot_e;
  if (e < n_exp) {
    start[e] = excl + bef[e];
    if (blockIdx.x == 0) {
      counts[e] = tot_e;
      offsets[e] = excl;
    }
  }
  if (blockIdx.x == 0 && tid == 0) offsets[n_exp] = static_cast<int32_t>(n_pairs);

  // This chunk: per-wave counts of its rows, then bases.
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    ec[r] = ec[r] < 0 ? 0 : (ec[r] >= n_exp ? n_exp - 1 : ec[r]);
    if (q0 + 64 * r + lane < c1) atomicAdd(&base[wv][ec[r]], 1);
  }
  __syncthreads();
  if (e < n_exp) {
    int32_t run = start[e];
    for (int w = 0; w < NW; ++w) {
      const int32_t c = base[w][e];
      base[w][e] = run;
      run += c;
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t q = q0 + 64 * r + lane;
    const bool valid = q < c1;
    const int ee = ec[r];
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
  if (n_pairs > kDispatchOneWg && n_experts <= kDispatchMultiMaxExperts)
    hipLaunchKernelGGL(k_dispatch_multi, dim3(static_cast<unsigned>(cdiv(n_pairs, kDispatchChunk))),
                       dim3(1024), 0, s, ids, ids_is_int64, n_pairs, n_experts, bits, counts, offsets,
                       pair_ids, inverse);
  else
    hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), 0, s, ids, ids_is_int64, n_pairs,
                       n_experts, bits, counts, offsets, pair_ids, inverse);
  return check_launch("moe_dispatch");
}
