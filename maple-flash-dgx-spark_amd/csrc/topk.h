// Softmax + top-k over one wave's logits (router semantics of reference
// src/maple_run/kernels/router.py:78-126).
#pragma once

#include "common.h"

namespace ma {

// Softmax over the wave-held logits p[i] (expert lane + 64 i), then top-k:
// slot s takes the largest probability left, the lowest expert index among
// equal ones (the reference's descending order with ties to the lowest
// index).  Probabilities are >= 0, so their bits order as integers: a slot is
// one wave-wide integer max (DPP steps into lane 63, read back as a scalar;
// no LDS round trip) and one ballot.  top_k <= 64; lane s keeps slot s.  One
// full wave runs this.
// COH: ids and weights are stored with the device-coherent policy (read by
// another workgroup of the same launch).
template <int PER, bool COH = false>
__device__ __forceinline__ void softmax_topk(float (&p)[PER], int64_t n_exp, int top_k,
                                             int32_t* __restrict__ ids,
                                             float* __restrict__ wts) {
  const int lane = threadIdx.x & 63;
  int mk = INT_MIN;
#pragma unroll
  for (int i = 0; i < PER; ++i) mk = max(mk, float_order_key(p[i]));
  const float m = float_from_order_key(wave_max_ui(mk));
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t e = lane + 64 * i;
    p[i] = e < n_exp ? expf(p[i] - m) : 0.f;
    sum += p[i];
  }
  const float inv_sum = 1.0f / wave_sum_u(sum);
  // experts past E get -1 (below every probability), chosen ones INT_MIN
  int key[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) key[i] = lane + 64 * i < n_exp ? __float_as_int(p[i] * inv_sum) : -1;
  int my_e = 0;
  float my_p = 0.f, sel = 0.f;
  for (int s = 0; s < top_k; ++s) {
    int lk = key[0];
#pragma unroll
    for (int i = 1; i < PER; ++i) lk = max(lk, key[i]);
    const int mx = wave_max_ui(lk);
    int e_s = 0;
#pragma unroll
    for (int i = PER - 1; i >= 0; --i) {  // the lowest i with a hit wins: the lowest index
      const uint64_t hit = __ballot(key[i] == mx);
      if (hit) e_s = __builtin_ctzll(hit) + 64 * i;
    }
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (lane + 64 * i == e_s) key[i] = INT_MIN;
    const float p_s = __int_as_float(mx);
    sel += p_s;
    if (lane == s) {
      my_e = e_s;
      my_p = p_s;
    }
  }
  const float inv_total = 1.0f / (sel + 1e-20f);
  if (lane < top_k) {
    if constexpr (COH) {
      __hip_atomic_store(&ids[lane], my_e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&wts[lane], my_p * inv_total, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      ids[lane] = my_e;
      wts[lane] = my_p * inv_total;
    }
  }
}

}  // namespace ma
