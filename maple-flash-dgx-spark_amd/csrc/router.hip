// MoE router: logits GEMV, softmax, top-k, renormalisation (gfx950).
//
// Semantics of reference src/maple_run/kernels/router.py:39-126: float32
// logits (+ an optional additive bias), p = exp(l - max) / sum, k passes of
// argmax with the winner masked out (descending; ties to the lowest index),
// w_j = p_j / (sum p_top + 1e-20).  Products are bf16 x bf16 summed by
// v_dot2_f32_bf16: exact products, float32 accumulation.
//
// Decode (tokens <= kFusedMaxTokens, bf16): ONE launch.  Workgroup (e, t)
// computes logit e of token t and publishes it as a 64-bit (value, tag = 1)
// word; workgroup (0, t) waits for the E tagged words of its token, clears
// them back to 0 and runs softmax + top-k.  The workspace therefore starts
// and ends every call all-zero (it must be zero-filled once when allocated),
// no atomic read-modify-write is used, and calls sharing a workspace must not
// overlap.  The wait is bounded (about 0.2 s): on timeout the kernel records
// an error in the workspace instead of hanging.
//
// Otherwise: two launches, like the reference (logits kernel, then top-k);
// prefill-sized batches take the logits as a GEMM on MFMA.
#include "mfma.h"
#include "topk.h"

namespace ma {

constexpr int kRouterMaxPerLane = 16;  // up to 1024 experts
constexpr int64_t kFusedMaxTokens = 16;
constexpr int64_t kFusedMaxExperts = 256;

// Workspace layout of the fused path (uint32 words):
//   [1]      error flag (1 = a wait timed out)
//   [64 ...] tagged logits, uint64 [tokens][E]: (1 << 32) | float bits
constexpr size_t kWsHeader = 64 * sizeof(uint32_t);

__device__ __forceinline__ float router_dot(const uint16_t* __restrict__ x,
                                            const uint16_t* __restrict__ w, int64_t k_in,
                                            int tid, int nthreads) {
  const uint4* xp = reinterpret_cast<const uint4*>(x);
  const uint4* wp = reinterpret_cast<const uint4*>(w);
  const int64_t n8 = k_in / 8;
  float a0 = 0.f, a1 = 0.f;
  for (int64_t i = tid; i < n8; i += nthreads) {
    const uint4 a = xp[i], b = wp[i];
    a0 = dot2(a.x, b.x, a0);
    a1 = dot2(a.y, b.y, a1);
    a0 = dot2(a.z, b.z, a0);
    a1 = dot2(a.w, b.w, a1);
  }
  return a0 + a1;
}

template <int PER>
__global__ __launch_bounds__(256) void k_router_fused(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ w,
    int64_t n_exp, int64_t k_in, const float* __restrict__ bias, int top_k,
    int32_t* __restrict__ ids, float* __restrict__ wts, uint32_t* __restrict__ ws) {
  __shared__ float red[4];
  const int64_t e = blockIdx.x, t = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  uint64_t* tagged = reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(ws) + kWsHeader);

  float s = router_dot(x + t * ldx, w + e * k_in, k_in, tid, 256);
  s = group_sum<64>(s);
  if (lane == 0) red[wv] = s;
  __syncthreads();
  if (tid == 0) {
    const float logit = (red[0] + red[1]) + (red[2] + red[3]) + (bias ? bias[e] : 0.f);
    const uint64_t word = (1ull << 32) | __float_as_uint(logit);
    __hip_atomic_store(&tagged[t * n_exp + e], word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (e != 0 || wv != 0) return;

  // Workgroup (0, t), wave 0: gather the E tagged logits of token t.
  float p[PER];
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  bool timed_out = false;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t ee = lane + 64 * i;
    p[i] = -INFINITY;
    if (ee < n_exp) {
      uint64_t v = __hip_atomic_load(&tagged[t * n_exp + ee], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      while ((v >> 32) != 1ull && !timed_out) {
        __builtin_amdgcn_s_sleep(2);
        v = __hip_atomic_load(&tagged[t * n_exp + ee], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        timed_out = (__builtin_amdgcn_s_memrealtime() - t0) > 20000000ull;  // 0.2 s at 100 MHz
      }
      p[i] = __uint_as_float(static_cast<uint32_t>(v));
      __hip_atomic_store(&tagged[t * n_exp + ee], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (__ballot(timed_out) && lane == 0)
    __hip_atomic_store(&ws[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  softmax_topk<PER>(p, n_exp, top_k, ids + t * top_k, wts + t * top_k);
}

__global__ __launch_bounds__(256) void k_router_logits(
    const void* __restrict__ x, int x_dt, int64_t ldx, const void* __restrict__ w, int w_dt,
    int64_t n_exp, int64_t k_in, const float* __restrict__ bias, float* __restrict__ logits,
    int fast) {
  const int lane = threadIdx.x & 63;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t t = blockIdx.y;
  if (e >= n_exp) return;  // uniform per wave
  float a = 0.f;
  if (fast) {
    a = router_dot(static_cast<const uint16_t*>(x) + t * ldx,
                   static_cast<const uint16_t*>(w) + e * k_in, k_in, lane, 64);
  } else {
    for (int64_t k = lane; k < k_in; k += 64)
      a += ld_f(x, x_dt, t * ldx + k) * ld_f(w, w_dt, e * k_in + k);
  }
  const float s = group_sum<64>(a);
  if (lane == 0) logits[t * n_exp + e] = s + (bias ? bias[e] : 0.f);
}

// The logits of prefill-sized batches as a GEMM on v_mfma_f32_16x16x32_bf16
// (A = 16 tokens, B = 16 experts, both straight from memory): a workgroup
// takes 16 tokens x 32 experts (at 2048 tokens and 64 experts, 256
// workgroups: one per CU; with 64 experts each, half the CUs idled and the
// launch took 11.6 against 7.9 us), its 8 waves each a K range of K / 8, walked
// in steps of kRgStep 32-wide k-slices whose operands are all loaded before
// the step's MFMAs; the waves' partial tiles are then added through LDS in
// wave order (the same bits on every run).  bf16 x bf16 products are exact;
// the sums are float32 (in another order than the dot-product kernel's).
constexpr int kRgWaves = 8, kRgExperts = 32, kRgStep = 4;

__global__ __launch_bounds__(64 * kRgWaves) void k_router_gemm(
    const uint16_t* __restrict__ x, int64_t ldx, int64_t tokens, const uint16_t* __restrict__ w,
    int64_t k_in, const float* __restrict__ bias, float* __restrict__ logits, int64_t n_exp) {
  __shared__ float part[kRgWaves][16][kRgExperts + 1];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * 16;
  const int64_t e0 = static_cast<int64_t>(blockIdx.y) * kRgExperts;
  const int64_t t = t0 + r16 < tokens ? t0 + r16 : tokens - 1;
  const uint16_t* const xr = x + t * ldx + 8 * g;
  constexpr int NBE = kRgExperts / 16;  // 16-expert blocks per workgroup
  const uint16_t* wr[NBE];
#pragma unroll
  for (int nb = 0; nb < NBE; ++nb) wr[nb] = w + (e0 + 16 * nb + r16) * k_in + 8 * g;
  const int64_t kw = k_in / kRgWaves;
  f32x4d_t acc[NBE];
#pragma unroll
  for (int nb = 0; nb < NBE; ++nb) acc[nb] = f32x4d_t{0.f, 0.f, 0.f, 0.f};
  for (int64_t k0 = wv * kw; k0 < (wv + 1) * kw; k0 += 32 * kRgStep) {
    u32x4v_t a[kRgStep], b[kRgStep][NBE];
#pragma unroll
    for (int s = 0; s < kRgStep; ++s) {
      a[s] = *reinterpret_cast<const u32x4v_t*>(xr + k0 + 32 * s);
#pragma unroll
      for (int nb = 0; nb < NBE; ++nb) b[s][nb] = *reinterpret_cast<const u32x4v_t*>(wr[nb] + k0 + 32 * s);
    }
    mfma_block_begin();
#pragma unroll
    for (int s = 0; s < kRgStep; ++s)
#pragma unroll
      for (int nb = 0; nb < NBE; ++nb) mfma_acc(acc[nb], a[s], b[s][nb]);
    mfma_block_end();
    keep_b(a, acc);
#pragma unroll
    for (int s = 0; s < kRgStep; ++s) keep_b(b[s], acc);
  }
  // lane (r16, g) holds tokens 4 g .. 4 g + 3 of expert 16 nb + r16
#pragma unroll
  for (int nb = 0; nb < NBE; ++nb)
#pragma unroll
    for (int i = 0; i < 4; ++i) part[wv][4 * g + i][16 * nb + r16] = acc[nb][i];
  __syncthreads();
  for (int o = tid; o < 16 * kRgExperts; o += 64 * kRgWaves) {
    const int tr = o / kRgExperts, ec = o % kRgExperts;
    float v = part[0][tr][ec];
#pragma unroll
    for (int ww = 1; ww < kRgWaves; ++ww) v += part[ww][tr][ec];
    const int64_t e = e0 + ec;
    if (t0 + tr < tokens) logits[(t0 + tr) * n_exp + e] = v + (bias ? bias[e] : 0.f);
  }
}

// The GEMM form pays off from kRgMinTokens tokens (below, its few
// workgroups leave most of the GPU idle and the dot-product kernel is faster).
constexpr int64_t kRgMinTokens = 256;

static bool gemm_ok(int x_dtype, int w_dtype, int64_t tokens, int64_t n_exp, int64_t k_in, int64_t ldx,
                    const void* x, const void* w) {
  return x_dtype == MA_BF16 && w_dtype == MA_BF16 && tokens >= kRgMinTokens && n_exp % kRgExperts == 0 &&
         k_in % (32 * kRgStep * kRgWaves) == 0 && (ldx % 8) == 0 &&
         ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15u) == 0;
}

template <int PER>
// Top-k of token t's logits.  With xp set, the same wave also writes token
// t's x' pairs (the grouped experts' B operands: xp [T, nwords * 8]) and its
// correction xc[t] = sum (f + 1) x, with the arithmetic and summation order
// of the grouped GEMMs' own x' launch (whose two waves' words lane and
// lane + 64, every 128th, are this lane's two sums), so the experts give the
// same bits either way and that launch is not needed.
__global__ __launch_bounds__(64) void k_router_topk(const float* __restrict__ logits,
                                                    int64_t n_exp, int top_k,
                                                    int32_t* __restrict__ ids,
                                                    float* __restrict__ wts,
                                                    const uint16_t* __restrict__ x, int64_t ldx,
                                                    int64_t nwords, uint32_t* __restrict__ xp,
                                                    float* __restrict__ xc) {
  const int lane = threadIdx.x;
  const int64_t t = blockIdx.x;
  float p[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t e = lane + 64 * i;
    p[i] = e < n_exp ? logits[t * n_exp + e] : -INFINITY;
  }
  if (xp) {  // the same in every lane
    float c[2] = {0.f, 0.f};
    for (int64_t w0 = 0; w0 < nwords; w0 += 128) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int64_t wd = w0 + lane + 64 * h;
        if (wd < nwords) {
          const uint4* src = reinterpret_cast<const uint4*>(x + t * ldx + wd * 16);
          uint32_t pr[8];
          c[h] += x16_to_pairs(src[0], src[1], pr);
          uint4* dst = reinterpret_cast<uint4*>(xp + (t * nwords + wd) * 8);
          dst[0] = make_uint4(pr[0], pr[1], pr[2], pr[3]);
          dst[1] = make_uint4(pr[4], pr[5], pr[6], pr[7]);
        }
      }
    }
    const float c0 = group_sum<64>(c[0]), c1 = group_sum<64>(c[1]);
    if (lane == 0) xc[t] = c0 + c1;
  }
  softmax_topk<PER>(p, n_exp, top_k, ids + t * top_k, wts + t * top_k);
}

static bool fused_ok(int x_dtype, int w_dtype, int64_t tokens, int64_t n_exp, int64_t k_in,
                     int64_t ldx, const void* x, const void* w) {
  return x_dtype == MA_BF16 && w_dtype == MA_BF16 && tokens <= kFusedMaxTokens &&
         n_exp <= kFusedMaxExperts && (k_in % 8) == 0 && (ldx % 8) == 0 &&
         ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15u) == 0;
}

}  // namespace ma

using namespace ma;

extern "C" size_t ma_router_workspace_bytes(int64_t tokens, int64_t n_experts) {
  const size_t t = static_cast<size_t>(tokens > 0 ? tokens : 0);
  const size_t e = static_cast<size_t>(n_experts > 0 ? n_experts : 0);
  // The fused path's tagged region comes first (it must stay zero between
  // calls); the two-pass path's float32 logits follow it.
  const size_t fused = kWsHeader + kFusedMaxTokens * kFusedMaxExperts * sizeof(uint64_t);
  return fused + t * e * sizeof(float);
}

// router_topk, and with x_pairs / x_corr set also the grouped experts' x'
// pairs of x (then always through the logits and the per-token top-k
// launch, which writes them).
static int router_topk_impl(const void* x, int x_dtype, int64_t tokens, int64_t ldx,
                            const void* gate_weight, int w_dtype, int64_t n_experts,
                            int64_t k_in, const float* bias, int top_k, int32_t* ids,
                            float* weights, uint32_t* x_pairs, float* x_corr, void* workspace,
                            size_t workspace_bytes, void* stream) {
  if (tokens < 0 || n_experts < 1 || k_in < 1)
    return fail(MA_EVALUE, "router_topk: bad sizes");
  if (top_k < 1 || top_k > n_experts || top_k > 64)
    return fail(MA_EVALUE, "top_k=%d must be in [1, min(n_experts=%lld, 64)].", top_k,
                (long long)n_experts);
  if (n_experts > 64 * kRouterMaxPerLane)
    return fail(MA_EVALUE, "router_topk supports at most %d experts", 64 * kRouterMaxPerLane);
  if (tokens == 0) return MA_OK;
  if (!workspace || workspace_bytes < ma_router_workspace_bytes(tokens, n_experts))
    return fail(MA_EVALUE, "router_topk: workspace too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!x_pairs && fused_ok(x_dtype, w_dtype, tokens, n_experts, k_in, ldx, x, gate_weight)) {
    dim3 grid(static_cast<unsigned>(n_experts), static_cast<unsigned>(tokens));
    const auto* xb = static_cast<const uint16_t*>(x);
    const auto* wb = static_cast<const uint16_t*>(gate_weight);
    auto* wsp = static_cast<uint32_t*>(workspace);
    if (n_experts <= 64)
      hipLaunchKernelGGL(k_router_fused<1>, grid, dim3(256), 0, s, xb, ldx, wb, n_experts, k_in,
                         bias, top_k, ids, weights, wsp);
    else
      hipLaunchKernelGGL(k_router_fused<4>, grid, dim3(256), 0, s, xb, ldx, wb, n_experts, k_in,
                         bias, top_k, ids, weights, wsp);
    return check_launch("router_topk");
  }
  float* logits = reinterpret_cast<float*>(static_cast<char*>(workspace) + kWsHeader +
                                           kFusedMaxTokens * kFusedMaxExperts * sizeof(uint64_t));
  const int fast = x_dtype == MA_BF16 && w_dtype == MA_BF16 && (k_in % 8) == 0 &&
                   (ldx % 8) == 0 &&
                   ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(gate_weight)) & 15u) == 0;
  if (gemm_ok(x_dtype, w_dtype, tokens, n_experts, k_in, ldx, x, gate_weight)) {
    dim3 gg(static_cast<unsigned>(cdiv(tokens, 16)), static_cast<unsigned>(n_experts / kRgExperts));
    hipLaunchKernelGGL(k_router_gemm, gg, dim3(64 * kRgWaves), 0, s, static_cast<const uint16_t*>(x), ldx,
                       tokens, static_cast<const uint16_t*>(gate_weight), k_in, bias, logits, n_experts);
  } else {
    dim3 g1(static_cast<unsigned>(cdiv(n_experts, 4)), static_cast<unsigned>(tokens));
    hipLaunchKernelGGL(k_router_logits, g1, dim3(256), 0, s, x, x_dtype, ldx, gate_weight, w_dtype,
                       n_experts, k_in, bias, logits, fast);
  }
  const dim3 gt(static_cast<unsigned>(tokens));
  const auto* xb = static_cast<const uint16_t*>(x);
  const int64_t nwords = k_in / 16;
  if (n_experts <= 64)
    hipLaunchKernelGGL(k_router_topk<1>, gt, dim3(64), 0, s, logits, n_experts, top_k, ids, weights, xb, ldx,
                       nwords, x_pairs, x_corr);
  else if (n_experts <= 256)
    hipLaunchKernelGGL(k_router_topk<4>, gt, dim3(64), 0, s, logits, n_experts, top_k, ids, weights, xb, ldx,
                       nwords, x_pairs, x_corr);
  else
    hipLaunchKernelGGL(k_router_topk<kRouterMaxPerLane>, gt, dim3(64), 0, s, logits, n_experts,
                       top_k, ids, weights, xb, ldx, nwords, x_pairs, x_corr);
  return check_launch("router_topk");
}

extern "C" int ma_router_topk(const void* x, int x_dtype, int64_t tokens, int64_t ldx,
                              const void* gate_weight, int w_dtype, int64_t n_experts,
                              int64_t k_in, const float* bias, int top_k, int32_t* ids,
                              float* weights, void* workspace, size_t workspace_bytes,
                              void* stream) {
  return router_topk_impl(x, x_dtype, tokens, ldx, gate_weight, w_dtype, n_experts, k_in, bias, top_k, ids,
                          weights, nullptr, nullptr, workspace, workspace_bytes, stream);
}

extern "C" int ma_router_topk_pairs(const void* x, int x_dtype, int64_t tokens, int64_t ldx,
                                    const void* gate_weight, int w_dtype, int64_t n_experts,
                                    int64_t k_in, const float* bias, int top_k, int32_t* ids,
                                    float* weights, uint32_t* x_pairs, float* x_corr, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  if (x_dtype != MA_BF16 || k_in % 16 || ldx % 8 || !x_pairs || !x_corr ||
      ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(x_pairs)) & 15u))
    return fail(MA_EVALUE, "router_topk_pairs: x must be bfloat16 with 16-byte aligned rows, hidden a "
                "multiple of 16, and x_pairs / x_corr given (x_pairs 16-byte aligned)");
  return router_topk_impl(x, x_dtype, tokens, ldx, gate_weight, w_dtype, n_experts, k_in, bias, top_k, ids,
                          weights, x_pairs, x_corr, workspace, workspace_bytes, stream);
}
