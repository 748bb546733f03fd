// Softmax + top-k over one wave's logits (router semantics of reference
// src/maple_run/kernels/router.py:78-126).
#pragma once

#include "common.h"

namespace ma {

// Softmax over the wave-held logits p[i] (expert lane + 64 i), then top-k by
// rank: the rank of an expert is the number of experts with a larger
// probability, or an equal one at a lower index, so rank order is the
// reference's descending order with ties to the lowest index.  Ranks come
// from v_readlane broadcasts (no LDS round trips).  One full wave runs this.
// COH: ids and weights are stored with the device-coherent policy (read by
// another workgroup of the same launch).
template <int PER, bool COH = false>
__device__ __forceinline__ void softmax_topk(float (&p)[PER], int64_t n_exp, int top_k,
                                             int32_t* __restrict__ ids,
                                             float* __restrict__ wts) {
  const int lane = threadIdx.x & 63;
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < PER; ++i) m = fmaxf(m, p[i]);
  m = wave_max(m);
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t e = lane + 64 * i;
    p[i] = e < n_exp ? expf(p[i] - m) : 0.f;
    sum += p[i];
  }
  sum = group_sum<64>(sum);
  const float inv_sum = 1.0f / sum;
  int rank[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t e = lane + 64 * i;
    p[i] = e < n_exp ? p[i] * inv_sum : -INFINITY;
    rank[i] = 0;
  }
#pragma unroll
  for (int im = 0; im < PER; ++im) {
    for (int src = 0; src < 64; ++src) {
      const float q = lane_bcast(p[im], src);
      const int em = src + 64 * im;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int e = lane + 64 * i;
        rank[i] += (q > p[i]) || (q == p[i] && em < e);
      }
    }
  }
  float sel = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) sel += rank[i] < top_k ? p[i] : 0.f;
  const float inv_total = 1.0f / (group_sum<64>(sel) + 1e-20f);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    if (e < n_exp && rank[i] < top_k) {
      if constexpr (COH) {
        __hip_atomic_store(&ids[rank[i]], e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&wts[rank[i]], p[i] * inv_total, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      } else {
        ids[rank[i]] = e;
        wts[rank[i]] = p[i] * inv_total;
      }
    }
  }
}

}  // namespace ma
