// MoE router: logits GEMV, softmax, top-k, renormalisation (gfx950).
//
// Semantics of reference src/maple_run/kernels/router.py:39-126: float32
// logits (+ this build's optional bias), p = exp(l - max) / sum, k passes of
// argmax with the winner masked out (descending; ties to the lowest index),
// w_j = p_j / (sum p_top + 1e-20).
//
// Two launches like the reference: one wave per (token, expert) logit with
// bf16 x bf16 products summed by v_dot2_f32_bf16 (exact products, float32
// accumulation), then one wave per token for softmax and top-k.
#include "common.h"

namespace ma {

__global__ __launch_bounds__(256) void k_router_logits(
    const void* __restrict__ x, int x_dt, int64_t ldx, const void* __restrict__ w, int w_dt,
    int64_t n_exp, int64_t k_in, const float* __restrict__ bias, float* __restrict__ logits,
    int fast) {
  const int lane = threadIdx.x & 63;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t t = blockIdx.y;
  if (e >= n_exp) return;  // uniform per wave
  float a0 = 0.f, a1 = 0.f;
  if (fast) {
    const uint4* xp = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + t * ldx);
    const uint4* wp = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(w) + e * k_in);
    const int64_t n8 = k_in / 8;
#pragma unroll 4
    for (int64_t i = lane; i < n8; i += 64) {
      const uint4 a = xp[i], b = wp[i];
      a0 = dot2(a.x, b.x, a0);
      a1 = dot2(a.y, b.y, a1);
      a0 = dot2(a.z, b.z, a0);
      a1 = dot2(a.w, b.w, a1);
    }
  } else {
    for (int64_t k = lane; k < k_in; k += 64)
      a0 += ld_f(x, x_dt, t * ldx + k) * ld_f(w, w_dt, e * k_in + k);
  }
  const float s = group_sum<64>(a0 + a1);
  if (lane == 0) logits[t * n_exp + e] = s + (bias ? bias[e] : 0.f);
}

// Wave arg-max of (value, index): larger value wins, ties to the lower index.
__device__ __forceinline__ void wave_argmax(float& v, int& idx) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(v, off, 64);
    const int oi = __shfl_xor(idx, off, 64);
    if (ov > v || (ov == v && oi < idx)) {
      v = ov;
      idx = oi;
    }
  }
}

constexpr int kRouterMaxPerLane = 16;  // up to 1024 experts

__global__ __launch_bounds__(64) void k_router_topk(const float* __restrict__ logits,
                                                    int64_t n_exp, int top_k,
                                                    int32_t* __restrict__ ids,
                                                    float* __restrict__ wts) {
  const int lane = threadIdx.x;
  const int64_t t = blockIdx.x;
  const float* l = logits + t * n_exp;
  float p[kRouterMaxPerLane];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < kRouterMaxPerLane; ++i) {
    const int64_t e = lane + 64 * i;
    p[i] = e < n_exp ? l[e] : -INFINITY;
    m = fmaxf(m, p[i]);
  }
  m = wave_max(m);
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < kRouterMaxPerLane; ++i) {
    const int64_t e = lane + 64 * i;
    p[i] = e < n_exp ? expf(p[i] - m) : 0.f;
    sum += p[i];
  }
  sum = group_sum<64>(sum);
  const float inv_sum = 1.0f / sum;
#pragma unroll
  for (int i = 0; i < kRouterMaxPerLane; ++i) {
    const int64_t e = lane + 64 * i;
    p[i] = e < n_exp ? p[i] * inv_sum : -INFINITY;
  }
  float total = 0.f;
  float mine = 0.f;  // lane j < top_k keeps the j-th pick
  int mine_id = 0;
  for (int j = 0; j < top_k; ++j) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < kRouterMaxPerLane; ++i) {
      const int e = lane + 64 * i;
      if (p[i] > bv) {
        bv = p[i];
        bi = e;
      }
    }
    wave_argmax(bv, bi);
    total += bv;
    if (lane == j) {
      mine = bv;
      mine_id = bi;
    }
#pragma unroll
    for (int i = 0; i < kRouterMaxPerLane; ++i)
      if (lane + 64 * i == bi) p[i] = -INFINITY;
  }
  if (lane < top_k) {
    ids[t * top_k + lane] = mine_id;
    wts[t * top_k + lane] = mine * (1.0f / (total + 1e-20f));
  }
}

}  // namespace ma

using namespace ma;

extern "C" size_t ma_router_workspace_bytes(int64_t tokens, int64_t n_experts) {
  return static_cast<size_t>(tokens > 0 ? tokens : 0) * static_cast<size_t>(n_experts > 0 ? n_experts : 0) * sizeof(float);
}

extern "C" int ma_router_topk(const void* x, int x_dtype, int64_t tokens, int64_t ldx,
                              const void* gate_weight, int w_dtype, int64_t n_experts,
                              int64_t k_in, const float* bias, int top_k, int32_t* ids,
                              float* weights, void* workspace, size_t workspace_bytes,
                              void* stream) {
  if (tokens < 0 || n_experts < 1 || k_in < 1)
    return fail(MA_EVALUE, "router_topk: bad sizes");
  if (top_k < 1 || top_k > n_experts || top_k > 64)
    return fail(MA_EVALUE, "top_k=%d must be in [1, min(n_experts=%lld, 64)].", top_k,
                (long long)n_experts);
  if (n_experts > 64 * kRouterMaxPerLane)
    return fail(MA_EVALUE, "router_topk supports at most %d experts", 64 * kRouterMaxPerLane);
  if (tokens == 0) return MA_OK;
  if (workspace_bytes < ma_router_workspace_bytes(tokens, n_experts))
    return fail(MA_EVALUE, "router_topk: workspace too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* logits = static_cast<float*>(workspace);
  const int fast = x_dtype == MA_BF16 && w_dtype == MA_BF16 && (k_in % 8) == 0 &&
                   (ldx % 8) == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(gate_weight)) & 15u) == 0;
  dim3 g1(static_cast<unsigned>(cdiv(n_experts, 4)), static_cast<unsigned>(tokens));
  hipLaunchKernelGGL(k_router_logits, g1, dim3(256), 0, s, x, x_dtype, ldx, gate_weight, w_dtype,
                     n_experts, k_in, bias, logits, fast);
  hipLaunchKernelGGL(k_router_topk, dim3(static_cast<unsigned>(tokens)), dim3(64), 0, s, logits,
                     n_experts, top_k, ids, weights);
  return check_launch("router_topk");
}
