// Batched MoE routing in one launch (gfx950): residual add + RMSNorm, router
// logits (+ optional bias), softmax + top-k, and the per-expert dispatch lists
// of the grouped expert GEMMs.
//
// Composes, with the arithmetic of this library's own kernels for each step
// (so the outputs equal those of the separate launches bit for bit):
//   add_rms_norm   reference src/maple_run/kernels/fused_norm.py:31-56
//                  (k_norm_fast: float32 x + y, h rounded to bf16, xn = bf16(
//                  v * rsqrt(mean(v^2) + eps) * w))
//   router_topk    reference src/maple_run/kernels/router.py:39-126
//                  (one wave per expert over xn, lane stride 64, v_dot2_f32_bf16)
//   dispatch       stable counting sort of (token, slot) pairs by expert
//                  (dispatch.h; the reference grids over pairs instead,
//                  src/maple_run/kernels/ternary_expert.py:210,443)
//
// Workgroup (b, t) normalises token t (every workgroup of the token does, from
// the same loads, so the norm is not a hand-off) and computes the logits of
// experts 4b .. 4b+3, one per wave, published as tagged 64-bit words
// (1 << 32 | float bits).  Workgroup (0, t) also writes h and xn, gathers its
// token's tagged logits (clearing them back to zero), runs softmax + top-k and
// stores ids / weights with the device-coherent policy; then it takes a
// ticket.  The workgroup that takes the last ticket resets the counter and
// builds the dispatch lists from every token's ids.  The workspace therefore
// starts and ends every call all-zero (zero-fill it once when allocating it);
// calls sharing a workspace must not overlap.  Waits are bounded (about 0.2
// s); a timeout sets the error word instead of hanging.
#include "dispatch.h"
#include "grid_sync.h"
#include "topk.h"

namespace ma {

constexpr int kRouteMaxExperts = 256;
constexpr int64_t kRouteMaxTokens = 1024;
// Workspace layout (uint32 words): [0] ticket counter, [64] error flag,
// then from byte kRouteHeader the tagged logits, uint64 [tokens][E].
constexpr size_t kRouteHeader = 512;

template <int CH, int WDT, int PER, bool ADD>
__global__ __launch_bounds__(256) void k_moe_route(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ add, int64_t hidden,
    const void* __restrict__ nw, float eps, const uint16_t* __restrict__ gate,
    const float* __restrict__ bias, int64_t n_exp, int top_k, int64_t tokens, int bits,
    uint16_t* __restrict__ h_out, uint16_t* __restrict__ xn_out, uint32_t* __restrict__ xn_pairs,
    float* __restrict__ xn_corr, int32_t* __restrict__ ids, float* __restrict__ wts,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets, int32_t* __restrict__ pair_ids,
    int32_t* __restrict__ inverse, uint32_t* __restrict__ ws) {
  __shared__ float red[4];
  __shared__ uint4 xs[256 * CH];  // xn of token t, packed bf16
  __shared__ int32_t base[4][kRouteMaxExperts];
  __shared__ int32_t wave_tot[4];
  __shared__ int last;
  const int64_t t = blockIdx.y;
  const int64_t eb = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t e = eb * 4 + wv;
  const int nch = static_cast<int>(hidden >> 3);
  uint64_t* tagged = reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(ws) + kRouteHeader);

  // ---- add + RMSNorm (k_norm_fast's arithmetic) --------------------------
  uint4 xv[CH], yv[CH];
  float wgt[CH][8];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = tid + 256 * c;
    const int cc = ch < nch ? ch : nch - 1;
    xv[c] = reinterpret_cast<const uint4*>(x + t * hidden)[cc];
    if constexpr (ADD) yv[c] = reinterpret_cast<const uint4*>(add + t * hidden)[cc];
#pragma unroll
    for (int k = 0; k < 8; ++k) wgt[c][k] = ld_t<WDT>(nw, cc * 8 + k);
  }
  // this wave's gate row, loaded with the activations (lane stride 64)
  const int64_t er = e < n_exp ? e : n_exp - 1;
  const uint4* grow = reinterpret_cast<const uint4*>(gate + er * hidden);
  uint4 gv[4 * CH];
#pragma unroll
  for (int j = 0; j < 4 * CH; ++j) {
    const int i = lane + 64 * j;
    gv[j] = grow[i < nch ? i : nch - 1];
  }
  MA_ISSUE_FENCE();
  float v[CH][8], ss = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const bool live = tid + 256 * c < nch;
    const uint32_t* xw = reinterpret_cast<const uint32_t*>(&xv[c]);
    const uint32_t* yw = reinterpret_cast<const uint32_t*>(&yv[c]);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float lo = __uint_as_float(xw[k] << 16), hi = __uint_as_float(xw[k] & 0xffff0000u);
      if constexpr (ADD) {
        lo += __uint_as_float(yw[k] << 16);
        hi += __uint_as_float(yw[k] & 0xffff0000u);
      }
      v[c][2 * k] = lo;
      v[c][2 * k + 1] = hi;
      if (live) ss += lo * lo + hi * hi;
    }
  }
  const float rstd = rsqrtf(block_sum256(ss, red) / static_cast<float>(hidden) + eps);
  const bool pairs = eb == 0 && xn_pairs != nullptr;
  float cpart = 0.f;  // sum (f + 1) xn over this thread's elements (pairs only)
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = tid + 256 * c;
    uint4 o, r;
    uint32_t* ow = reinterpret_cast<uint32_t*>(&o);
    uint32_t* rw = reinterpret_cast<uint32_t*>(&r);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      ow[k] = pack_bf16x2_rn(v[c][2 * k] * rstd * wgt[c][2 * k],
                             v[c][2 * k + 1] * rstd * wgt[c][2 * k + 1]);
      if constexpr (ADD) rw[k] = pack_bf16x2_rn(v[c][2 * k], v[c][2 * k + 1]);
    }
    if (pairs) {
      // x' pairs of word ch / 2: pair j = (f_j xn_j, f_j xn_{j+8}); this
      // thread holds elements 8 (ch & 1) .. +7 of the word, its partner
      // (lane ^ 1) the other half.
      uint32_t hv[4];  // f_j xn_j as bf16 bits, two per dword (exact)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float x0 = __uint_as_float(ow[k] << 16), x1 = __uint_as_float(ow[k] & 0xffff0000u);
        const float f0 = pair_scale(2 * k), f1 = pair_scale(2 * k + 1);
        hv[k] = pack_bf16x2(f0 * x0, f1 * x1);
        if (ch < nch) cpart += (f0 + 1.0f) * x0 + (f1 + 1.0f) * x1;
      }
      uint32_t ov[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) ov[k] = __shfl_xor(hv[k], 1, 64);
      if ((ch & 1) == 0 && ch < nch) {
        uint4 p0, p1;  // dword j: lo = own f_j xn_j, hi = partner's
        p0.x = (hv[0] & 0xffffu) | (ov[0] << 16);
        p0.y = (hv[0] >> 16) | (ov[0] & 0xffff0000u);
        p0.z = (hv[1] & 0xffffu) | (ov[1] << 16);
        p0.w = (hv[1] >> 16) | (ov[1] & 0xffff0000u);
        p1.x = (hv[2] & 0xffffu) | (ov[2] << 16);
        p1.y = (hv[2] >> 16) | (ov[2] & 0xffff0000u);
        p1.z = (hv[3] & 0xffffu) | (ov[3] << 16);
        p1.w = (hv[3] >> 16) | (ov[3] & 0xffff0000u);
        uint4* dst = reinterpret_cast<uint4*>(xn_pairs + t * (hidden / 2) + (ch >> 1) * 8);
        dst[0] = p0;
        dst[1] = p1;
      }
    }
    if (ch >= nch) continue;
    xs[ch] = o;
    if (eb == 0) {
      reinterpret_cast<uint4*>(xn_out + t * hidden)[ch] = o;
      if constexpr (ADD) reinterpret_cast<uint4*>(h_out + t * hidden)[ch] = r;
    }
  }
  if (pairs) {  // uniform per workgroup
    const float csum = block_sum256(cpart, red);
    if (tid == 0) xn_corr[t] = csum;
  }
  __syncthreads();

  // ---- logit of expert e (k_router_logits' arithmetic) -------------------
  if (e < n_exp) {
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int j = 0; j < 4 * CH; ++j) {
      const int i = lane + 64 * j;
      if (i < nch) {
        const uint4 a = xs[i], b = gv[j];
        a0 = dot2(a.x, b.x, a0);
        a1 = dot2(a.y, b.y, a1);
        a0 = dot2(a.z, b.z, a0);
        a1 = dot2(a.w, b.w, a1);
      }
    }
    const float s = group_sum<64>(a0 + a1);
    if (lane == 0) {
      const float logit = s + (bias ? bias[e] : 0.f);
      st_coh64(&tagged[t * n_exp + e], (1ull << 32) | __float_as_uint(logit));
    }
  }
  if (eb != 0) return;

  // ---- workgroup (0, t): softmax + top-k, ticket -------------------------
  if (wv == 0) {
    float p[PER];
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    bool timed_out = false;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int64_t ee = lane + 64 * i;
      p[i] = -INFINITY;
      if (ee < n_exp) {
        uint64_t w = ld_coh64(&tagged[t * n_exp + ee]);
        while ((w >> 32) != 1ull && !timed_out) {
          __builtin_amdgcn_s_sleep(2);
          w = ld_coh64(&tagged[t * n_exp + ee]);
          timed_out = (__builtin_amdgcn_s_memrealtime() - t0) > kGridSpin;
        }
        p[i] = __uint_as_float(static_cast<uint32_t>(w));
        st_coh64(&tagged[t * n_exp + ee], 0ull);
      }
    }
    if (__ballot(timed_out) && lane == 0) st_coh32(&ws[64], 1u);
    softmax_topk<PER, true>(p, n_exp, top_k, ids + t * top_k, wts + t * top_k);
    __builtin_amdgcn_s_waitcnt(0);  // this token's ids / weights have completed
    int is_last = 0;
    if (lane == 0) {
      is_last = atomicAdd(&ws[0], 1u) == static_cast<uint32_t>(tokens - 1);
      if (is_last) st_coh32(&ws[0], 0u);
      last = is_last;
    }
  }
  __syncthreads();
  if (!last) return;

  // ---- the last token's workgroup: dispatch lists of all tokens ----------
  const uint32_t* idu = reinterpret_cast<const uint32_t*>(ids);
  dispatch_block<4, kRouteMaxExperts>(
      [&](int64_t q) { return static_cast<int>(ld_coh32(idu + q)); }, tokens * top_k,
      static_cast<int>(n_exp), bits, base, wave_tot, counts, offsets, pair_ids, inverse);
}

}  // namespace ma

using namespace ma;

extern "C" size_t ma_moe_route_workspace_bytes(int64_t tokens, int64_t n_experts) {
  const size_t t = static_cast<size_t>(tokens > 0 ? tokens : 0);
  const size_t e = static_cast<size_t>(n_experts > 0 ? n_experts : 0);
  return kRouteHeader + t * e * sizeof(uint64_t);
}

extern "C" int ma_moe_route(const void* x, const void* x_add, int64_t tokens, int64_t hidden,
                            const void* norm_weight, int norm_dtype, float eps,
                            const void* gate_weight, const float* router_bias,
                            int64_t n_experts, int top_k, void* h_out, void* xn_out,
                            uint32_t* xn_pairs, float* xn_corr,
                            int32_t* topk_ids, float* topk_weight, int32_t* counts,
                            int32_t* offsets, int32_t* pair_ids, int32_t* inverse,
                            void* workspace, size_t workspace_bytes, void* stream) {
  if (tokens < 0 || tokens > kRouteMaxTokens || hidden < 8 || hidden % 8 || hidden > 4096)
    return fail(MA_EVALUE, "moe_route: tokens must be in [0, %lld] and hidden a multiple of 8 "
                "up to 4096 (got %lld, %lld)", (long long)kRouteMaxTokens, (long long)tokens,
                (long long)hidden);
  if (n_experts < 1 || n_experts > kRouteMaxExperts)
    return fail(MA_EVALUE, "moe_route: n_experts must be in [1, %d]", kRouteMaxExperts);
  if (top_k < 1 || top_k > n_experts || top_k > 64)
    return fail(MA_EVALUE, "top_k=%d must be in [1, min(n_experts=%lld, 64)].", top_k,
                (long long)n_experts);
  if (norm_dtype != MA_F32 && norm_dtype != MA_BF16)
    return fail(MA_ETYPE, "moe_route: norm weight must be float32 or bfloat16");
  if (tokens == 0) return MA_OK;
  if (!x || !norm_weight || !gate_weight || !xn_out || !topk_ids || !topk_weight || !counts ||
      !offsets || !pair_ids || !inverse || (x_add && !h_out) || (!xn_pairs != !xn_corr))
    return fail(MA_EVALUE, "moe_route: null pointer");
  if (xn_pairs && (hidden % 16 || (reinterpret_cast<uintptr_t>(xn_pairs) & 15)))
    return fail(MA_EVALUE, "moe_route: x' pairs need hidden %% 16 == 0 and 16-byte alignment");
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (!a16(x) || !a16(gate_weight) || !a16(xn_out) || (x_add && (!a16(x_add) || !a16(h_out))))
    return fail(MA_EVALUE, "moe_route: rows must be 16-byte aligned");
  if (!workspace || workspace_bytes < ma_moe_route_workspace_bytes(tokens, n_experts) ||
      (reinterpret_cast<uintptr_t>(workspace) & 255))
    return fail(MA_EVALUE, "moe_route: workspace too small or not 256-byte aligned");
  int bits = 0;
  while ((1 << bits) < n_experts) ++bits;
  const int ch = hidden <= 2048 ? 1 : 2;
  const int per = n_experts <= 64 ? 1 : 4;
  dim3 grid(static_cast<unsigned>(cdiv(n_experts, 4)), static_cast<unsigned>(tokens));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* xb = static_cast<const uint16_t*>(x);
  const auto* ab = static_cast<const uint16_t*>(x_add);
  const auto* gb = static_cast<const uint16_t*>(gate_weight);
  auto* hb = static_cast<uint16_t*>(h_out);
  auto* nb = static_cast<uint16_t*>(xn_out);
  auto* wsp = static_cast<uint32_t*>(workspace);
#define MA_RT(CH, WDT, PER, ADD)                                                                \
  hipLaunchKernelGGL((k_moe_route<CH, WDT, PER, ADD>), grid, dim3(256), 0, s, xb, ab, hidden, \
                     norm_weight, eps, gb, router_bias, n_experts, top_k, tokens, bits, hb, nb, \
                     xn_pairs, xn_corr, topk_ids, topk_weight, counts, offsets, pair_ids, inverse, \
                     wsp)
#define MA_RT_A(CH, WDT, PER) \
  if (x_add) { MA_RT(CH, WDT, PER, true); } else { MA_RT(CH, WDT, PER, false); }
#define MA_RT_P(CH, WDT) \
  if (per == 1) { MA_RT_A(CH, WDT, 1) } else { MA_RT_A(CH, WDT, 4) }
#define MA_RT_W(CH) \
  if (norm_dtype == MA_F32) { MA_RT_P(CH, MA_F32) } else { MA_RT_P(CH, MA_BF16) }
  if (ch == 1) { MA_RT_W(1) } else { MA_RT_W(2) }
#undef MA_RT_W
#undef MA_RT_P
#undef MA_RT_A
#undef MA_RT
  return check_launch("moe_route");
}
