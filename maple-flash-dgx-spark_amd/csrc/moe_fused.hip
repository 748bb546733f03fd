// One-launch MoE FFN layer for one token (decode batch 1), gfx950.
//
// Semantics: MapleSparseMoeBlock.__call__ (reference src/maple_run/model.py:
// 448-474) at T = 1: router_topk (kernels/router.py:39-126), the expert SwiGLU
// (kernels/ternary_expert.py:240-319, h stored bf16), each slot's down
// projection rounded to bf16 (ternary_expert.py:58-122), and the top-k
// weighted float32 combine with the residual (fused_norm.py:59-96), y stored
// bf16.  Optionally the add + RMSNorm ahead
// of it (kernels/fused_norm.py:31-56): s = a + b in float32, residual =
// bf16(s), x = bf16(s * rsqrt(mean(s^2) + eps) * w).
//
// A persistent grid of G workgroups (all resident) runs four phases; the one
// hand-off between workgroups goes through the workspace with
// device-coherent stores and a monotonic counter (no grid barrier, nothing to
// clear between calls):
//   1. every workgroup stages x (after the optional add + RMSNorm);
//   2. every workgroup computes all E router logits itself (the router is
//      small and L2-resident) and the softmax + top-k;
//   3. it issues its down-projection weight loads (known once the ids are),
//      computes its slice of the 8 x I SwiGLU outputs, publishes them and
//      counts itself in;
//   4. it waits until all G have, stages h and finishes its rows of y.
// The last workgroup to finish (a ticket) advances the counter base.  Every
// wait is bounded (about 0.2 s); on timeout the workspace error word is set
// and the kernel finishes with wrong values instead of hanging.
#include "ternary_engine.h"
#include "topk.h"

namespace ma {

constexpr int kFusedWaves = 4;
constexpr uint64_t kFusedSpin = 20000000ull;  // 0.2 s of the 100 MHz realtime counter

// Workspace layout (uint32 words, then bytes):
//   [1] end ticket   [2] error   [3] h-done counter (+1 per workgroup per call)
//   [4] the counter's value when this call started (advanced by G by the
//       last workgroup out, so the goal is base + G whatever the grid size)
//   [256 bytes ...)  h, bf16 [TK * I]
constexpr size_t kMoeWsHeader = 256;

__device__ __forceinline__ uint32_t ld_coh32(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_coh64(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh16(uint16_t* p, uint16_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Shapes: H = 16 * KWH * LPRH (SwiGLU rows split over LPRH lanes), I = 16 *
// KWI * LPRI (down rows over LPRI lanes), US SwiGLU iterations and UD down
// row iterations per wave, TK experts per token, PER = ceil(E / 64).
template <int KWH, int LPRH, int US, int KWI, int LPRI, int UD, int TK, int PER>
__global__ __launch_bounds__(64 * kFusedWaves) void k_moe_fused(
    const uint16_t* __restrict__ xa, const uint16_t* __restrict__ xb,
    const void* __restrict__ norm_w, int norm_dt, float eps, const uint16_t* __restrict__ residual,
    const uint16_t* __restrict__ gate_w, const float* __restrict__ bias, int n_exp,
    const uint32_t* __restrict__ ug, const uint16_t* __restrict__ ug_alpha,
    const uint32_t* __restrict__ dn, const uint16_t* __restrict__ dn_alpha,
    uint16_t* __restrict__ y, int32_t* __restrict__ ids_out, float* __restrict__ wts_out,
    uint32_t* __restrict__ ws) {
  constexpr int NWH = KWH * LPRH, H = 16 * NWH;
  constexpr int NWI = KWI * LPRI, I = 16 * NWI;
  constexpr int RPIH = 64 / LPRH, PPI = RPIH / 2;      // SwiGLU: up/gate pairs per wave pass
  constexpr int UNITS_WG = kFusedWaves * US * PPI;     // h outputs per workgroup
  constexpr int RPID = 64 / LPRI;                      // down rows per wave pass
  constexpr int RPB = RPID * UD;                       // y rows per workgroup
  constexpr int SPW = TK >= kFusedWaves ? TK / kFusedWaves : 1;
  static_assert(TK % kFusedWaves == 0 || TK < kFusedWaves, "top-k split over waves");
  static_assert(H % 8 == 0 && H / 8 <= 64 * kFusedWaves * 4, "router staging");

  __shared__ __align__(16) uint32_t xs[NWH][8];
  __shared__ float cw[NWH];
  __shared__ __align__(16) uint16_t xr[H];         // bf16 x for the router
  __shared__ __align__(16) uint32_t hs[TK][NWI][8];
  __shared__ float hc[TK][NWI];
  __shared__ float s_logit[64 * PER];
  __shared__ int32_t s_ids[TK];
  __shared__ float s_wts[TK];
  __shared__ float red[kFusedWaves];
  __shared__ float part[kFusedWaves][RPB];
  __shared__ int s_last;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = gridDim.x, wg = blockIdx.x;
  // h-done counter value at the start of this call (written only by the
  // previous call's last workgroup, so every workgroup reads the same value)
  const uint32_t base = ld_coh32(&ws[4]);
  uint16_t* hbuf = reinterpret_cast<uint16_t*>(reinterpret_cast<char*>(ws) + kMoeWsHeader);
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  bool timed_out = false;

  // ---- 1. x (optionally add + RMSNorm), staged as raw bf16 and as x' pairs
  {
    // thread t owns words t, t + 256, ... (16 values each)
    constexpr int WPT = (NWH + 255) / 256;
    float v[WPT][16];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      const int w = tid + 256 * i;
      const int wc = w < NWH ? w : NWH - 1;
      const uint4 a0 = reinterpret_cast<const uint4*>(xa + wc * 16)[0];
      const uint4 a1 = reinterpret_cast<const uint4*>(xa + wc * 16)[1];
      const uint32_t u[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        v[i][2 * q] = __uint_as_float(u[q] << 16);
        v[i][2 * q + 1] = __uint_as_float(u[q] & 0xffff0000u);
      }
      if (xb) {
        const uint4 b0 = reinterpret_cast<const uint4*>(xb + wc * 16)[0];
        const uint4 b1 = reinterpret_cast<const uint4*>(xb + wc * 16)[1];
        const uint32_t ub[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          v[i][2 * q] += __uint_as_float(ub[q] << 16);
          v[i][2 * q + 1] += __uint_as_float(ub[q] & 0xffff0000u);
        }
      }
      if (w < NWH) {
#pragma unroll
        for (int q = 0; q < 16; ++q) ss += v[i][q] * v[i][q];
      }
    }
    if (xb) {
      ss = group_sum<64>(ss);
      if (lane == 0) red[wv] = ss;
      __syncthreads();
      const float rstd = rsqrtf((red[0] + red[1] + red[2] + red[3]) / static_cast<float>(H) + eps);
#pragma unroll
      for (int i = 0; i < WPT; ++i) {
        const int w = tid + 256 * i;
        const int wc = w < NWH ? w : NWH - 1;
#pragma unroll
        for (int q = 0; q < 16; ++q)
          v[i][q] = bf16_to_f32(f32_to_bf16(v[i][q] * rstd * ld_f(norm_w, norm_dt, wc * 16 + q)));
      }
    }
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      const int w = tid + 256 * i;
      if (w < NWH) {
        uint32_t pr[8];
        cw[w] = prep_word_pairs(v[i], pr);
#pragma unroll
        for (int j = 0; j < 8; ++j) xs[w][j] = pr[j];
        uint4 r0, r1;
        r0.x = pack_bf16x2(v[i][0], v[i][1]);   r0.y = pack_bf16x2(v[i][2], v[i][3]);
        r0.z = pack_bf16x2(v[i][4], v[i][5]);   r0.w = pack_bf16x2(v[i][6], v[i][7]);
        r1.x = pack_bf16x2(v[i][8], v[i][9]);   r1.y = pack_bf16x2(v[i][10], v[i][11]);
        r1.z = pack_bf16x2(v[i][12], v[i][13]); r1.w = pack_bf16x2(v[i][14], v[i][15]);
        reinterpret_cast<uint4*>(xr + w * 16)[0] = r0;
        reinterpret_cast<uint4*>(xr + w * 16)[1] = r1;
      }
    }
  }
  __syncthreads();

  // ---- 2. router: every workgroup computes all E logits itself (the router
  // weights are L2-resident after the first workgroup of an XCD reads them),
  // so no workgroup waits for another to learn the expert ids.  Wave w takes
  // experts w, w + 4, ...; lane l holds x[32 l, 32 l + 32) for H = 2048.
  {
    constexpr int XU = H / 8 / 64;  // uint4 of x (and of a router row) per lane
    static_assert(H % 512 == 0 || H == 256, "router lane split");
    constexpr int XUL = XU > 0 ? XU : 1;
    uint4 xl[XUL];
#pragma unroll
    for (int i = 0; i < XUL; ++i) {
      const int idx = lane * XUL + i;
      xl[i] = idx < H / 8 ? reinterpret_cast<const uint4*>(xr)[idx] : make_uint4(0, 0, 0, 0);
    }
    constexpr int EB = 4;  // experts per batch of loads
    for (int e0 = wv * EB; e0 < n_exp; e0 += kFusedWaves * EB) {
      uint4 wr[EB][XUL];
#pragma unroll
      for (int b = 0; b < EB; ++b) {
        const int e = e0 + b < n_exp ? e0 + b : n_exp - 1;
        const uint4* wp = reinterpret_cast<const uint4*>(gate_w + static_cast<int64_t>(e) * H);
#pragma unroll
        for (int i = 0; i < XUL; ++i) {
          const int idx = lane * XUL + i;
          wr[b][i] = idx < H / 8 ? wp[idx] : make_uint4(0, 0, 0, 0);
        }
      }
#pragma unroll
      for (int b = 0; b < EB; ++b) {
        float a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int i = 0; i < XUL; ++i) {
          a0 = dot2(xl[i].x, wr[b][i].x, a0);
          a1 = dot2(xl[i].y, wr[b][i].y, a1);
          a0 = dot2(xl[i].z, wr[b][i].z, a0);
          a1 = dot2(xl[i].w, wr[b][i].w, a1);
        }
        const float sum = group_sum<64>(a0 + a1);
        if (lane == 0 && e0 + b < n_exp) s_logit[e0 + b] = sum + (bias ? bias[e0 + b] : 0.f);
      }
    }
  }
  __syncthreads();
  if (wv == 0) {
    float p[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = lane + 64 * i;
      p[i] = e < n_exp ? s_logit[e] : -INFINITY;
    }
    softmax_topk<PER>(p, n_exp, TK, s_ids, s_wts);
  }
  __syncthreads();
  if (wg == 0 && tid < TK) {
    ids_out[tid] = s_ids[tid];
    wts_out[tid] = s_wts[tid];
  }

  // ---- 3. weights: SwiGLU rows of this workgroup's h outputs, then the down
  // rows of its y rows (every load issued before any arithmetic)
  const int klh = lane % LPRH, subh = lane / LPRH, half = subh / PPI, pi = subh % PPI;
  uint32_t wu[US][KWH];
  float au[US];
#pragma unroll
  for (int u = 0; u < US; ++u) {
    int ug_i = (wg * kFusedWaves + wv) * (US * PPI) + u * PPI + pi;
    ug_i = ug_i < TK * I ? ug_i : TK * I - 1;
    const int s = ug_i / I, j = ug_i % I;
    const int64_t e = clamp_id(s_ids[s], n_exp);
    const int64_t row = e * (2 * I) + j + half * I;
    load_words_v<KWH>(ug + row * NWH + klh * KWH, wu[u]);
    au[u] = bf16_to_f32(ug_alpha[row]);
  }
  const int kld = lane % LPRI, subd = lane / LPRI;
  const int rbase = wg * RPB;
  uint32_t wd[SPW][UD][KWI];
  float ad[SPW][UD], wj[SPW];
#pragma unroll
  for (int q = 0; q < SPW; ++q) {
    const int js = wv + kFusedWaves * q;
    const int jj = js < TK ? js : 0;  // idle waves (TK < waves) read slot 0 and add nothing
    const int64_t e = clamp_id(s_ids[jj], n_exp);
    wj[q] = js < TK ? s_wts[jj] : 0.f;
#pragma unroll
    for (int u = 0; u < UD; ++u) {
      int r = rbase + u * RPID + subd;
      r = r < H ? r : H - 1;
      load_words_v<KWI>(dn + (e * H + r) * NWI + kld * KWI, wd[q][u]);
      ad[q][u] = bf16_to_f32(dn_alpha[e * H + r]);
    }
  }
  float resv = 0.f;
  const int ro = rbase + tid;
  if (tid < RPB && ro < H) {
    if (xb)
      resv = bf16_to_f32(f32_to_bf16(bf16_to_f32(xa[ro]) + bf16_to_f32(xb[ro])));
    else if (residual)
      resv = bf16_to_f32(residual[ro]);
  }
  MA_ISSUE_FENCE();

  // SwiGLU outputs of this workgroup
  {
    XSlice<KWH> xsl;
    slice_from_lds<KWH>(xs, cw, klh, xsl);
    const ExpandConsts kc;
#pragma unroll
    for (int u = 0; u < US; ++u) {
      const float v = group_sum<LPRH>(slice_dot<KWH>(wu[u], xsl, kc) * au[u]);
      const float g = __shfl(v, lane + PPI * LPRH, 64);
      const int ug_i = (wg * kFusedWaves + wv) * (US * PPI) + u * PPI + pi;
      if (half == 0 && klh == 0 && ug_i < TK * I) st_coh16(&hbuf[ug_i], f32_to_bf16(swiglu_act(v, g)));
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // this workgroup's h stores have completed
  __syncthreads();
  // ---- 4. count this workgroup in, wait until all G are (one lane polls a
  // single monotonic counter: it reads base + G once this call's h is out)
  if (tid == 0) {
    atomicAdd(&ws[3], 1u);
    const uint32_t goal = base + static_cast<uint32_t>(G);
    while (static_cast<int32_t>(ld_coh32(&ws[3]) - goal) < 0 && !timed_out) {
      __builtin_amdgcn_s_sleep(2);
      timed_out = (__builtin_amdgcn_s_memrealtime() - t0) > kFusedSpin;
    }
  }
  __syncthreads();
  for (int wi = tid; wi < TK * NWI; wi += 256) {
    const int s = wi / NWI, w = wi % NWI;
    const uint64_t* src = reinterpret_cast<const uint64_t*>(hbuf + s * I + w * 16);
    uint32_t u[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint64_t d = ld_coh64(src + q);
      u[2 * q] = static_cast<uint32_t>(d);
      u[2 * q + 1] = static_cast<uint32_t>(d >> 32);
    }
    float vv[16];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      vv[2 * q] = __uint_as_float(u[q] << 16);
      vv[2 * q + 1] = __uint_as_float(u[q] & 0xffff0000u);
    }
    uint32_t pr[8];
    hc[s][w] = prep_word_pairs(vv, pr);
#pragma unroll
    for (int j = 0; j < 8; ++j) hs[s][w][j] = pr[j];
  }
  __syncthreads();

  // down rows + weighted combine + residual
  {
    const ExpandConsts kc;
    float acc[UD];
#pragma unroll
    for (int u = 0; u < UD; ++u) acc[u] = 0.f;
#pragma unroll
    for (int q = 0; q < SPW; ++q) {
      const int js = wv + kFusedWaves * q;
      const int jj = js < TK ? js : 0;
      XSlice<KWI> hsl;
      slice_from_lds<KWI>(hs[jj], hc[jj], kld, hsl);
#pragma unroll
      for (int u = 0; u < UD; ++u) {
        // each slot's down output is rounded to bf16 before the weighted sum,
        // as the reference's ternary_expert_gemv -> moe_reduce_add chain stores it
        const float eo = group_sum<LPRI>(slice_dot<KWI>(wd[q][u], hsl, kc) * ad[q][u]);
        acc[u] += wj[q] * bf16_to_f32(f32_to_bf16(eo));
      }
    }
#pragma unroll
    for (int u = 0; u < UD; ++u)
      if (kld == 0) part[wv][u * RPID + subd] = acc[u];
  }
  __syncthreads();
  if (tid < RPB && ro < H) {
    float v = resv;
#pragma unroll
    for (int ww = 0; ww < kFusedWaves; ++ww) v += part[ww][tid];
    y[ro] = f32_to_bf16(v);
  }
  if (__ballot(timed_out) && lane == 0) st_coh32(&ws[2], 1u);

  // ---- the last workgroup out advances the counter base
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(&ws[1], 1u) == static_cast<uint32_t>(G - 1);
  __syncthreads();
  if (s_last && tid == 0) {
    st_coh32(&ws[1], 0u);
    st_coh32(&ws[4], base + static_cast<uint32_t>(G));
  }
}

}  // namespace ma

using namespace ma;

namespace {

// Supported (hidden, intermediate, top_k) shapes and their grid.
struct FusedShape {
  int hidden, inter, top_k, grid;
};
// (2048, 768, 8): SwiGLU 24 outputs and down 8 rows per workgroup -> 256 groups.
// (256, 128, 2): SwiGLU 16 outputs, down 8 rows per workgroup -> 32 groups.
constexpr FusedShape kShapes[] = {{2048, 768, 8, 256}, {256, 128, 2, 32}};

const FusedShape* find_shape(int64_t hidden, int64_t inter, int64_t top_k) {
  for (const auto& s : kShapes)
    if (s.hidden == hidden && s.inter == inter && s.top_k == top_k) return &s;
  return nullptr;
}

size_t ws_bytes(int64_t, int, int64_t inter, int64_t top_k) {
  return kMoeWsHeader + static_cast<size_t>(top_k * inter) * 2;
}

}  // namespace

extern "C" size_t ma_moe_fused_workspace_bytes(int64_t n_experts, int64_t hidden, int64_t inter,
                                               int64_t top_k) {
  const FusedShape* s = find_shape(hidden, inter, top_k);
  if (!s || n_experts < 1) return 0;
  return ws_bytes(n_experts, s->grid, inter, top_k);
}

extern "C" int ma_moe_fused(const void* x, const void* x_add, const void* norm_weight,
                            int norm_dtype, float eps, const void* residual,
                            const void* gate_weight, const float* router_bias, int64_t n_experts,
                            int64_t hidden, int64_t inter, int64_t top_k,
                            const uint32_t* up_gate, const void* up_gate_alpha,
                            const uint32_t* down, const void* down_alpha, void* y,
                            int32_t* topk_ids, float* topk_weight, void* workspace,
                            size_t workspace_bytes, void* stream) {
  const FusedShape* s = find_shape(hidden, inter, top_k);
  if (!s)
    return fail(MA_EVALUE, "moe_fused: shape (hidden %lld, inter %lld, top_k %lld) not built",
                static_cast<long long>(hidden), static_cast<long long>(inter),
                static_cast<long long>(top_k));
  if (n_experts < top_k || n_experts > 256 || n_experts > static_cast<int64_t>(s->grid) * 64)
    return fail(MA_EVALUE, "moe_fused: %lld experts unsupported", static_cast<long long>(n_experts));
  if (x_add && !norm_weight) return fail(MA_EVALUE, "moe_fused: add without norm weight");
  if (norm_weight && norm_dtype != MA_F32 && norm_dtype != MA_BF16)
    return fail(MA_ETYPE, "moe_fused: norm weight dtype %d", norm_dtype);
  if (!workspace || workspace_bytes < ws_bytes(n_experts, s->grid, inter, top_k))
    return fail(MA_EVALUE, "moe_fused: workspace too small");
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (!a16(x) || (x_add && !a16(x_add)) || !a16(gate_weight) || !a16(up_gate) || !a16(workspace))
    return fail(MA_EVALUE, "moe_fused: x, x_add, weights and workspace must be 16-byte aligned");
  const int per = n_experts <= 64 ? 1 : 4;
  hipStream_t st = static_cast<hipStream_t>(stream);
#define MA_FUSED_ARGS                                                                            \
  static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(x_add), norm_weight, norm_dtype, \
      eps, static_cast<const uint16_t*>(residual), static_cast<const uint16_t*>(gate_weight),    \
      router_bias, static_cast<int>(n_experts), up_gate,                                         \
      static_cast<const uint16_t*>(up_gate_alpha), down, static_cast<const uint16_t*>(down_alpha), \
      static_cast<uint16_t*>(y), topk_ids, topk_weight, static_cast<uint32_t*>(workspace)
  if (hidden == 2048) {
    if (per == 1)
      hipLaunchKernelGGL((k_moe_fused<4, 32, 6, 3, 16, 2, 8, 1>), dim3(s->grid), dim3(256), 0, st, MA_FUSED_ARGS);
    else
      hipLaunchKernelGGL((k_moe_fused<4, 32, 6, 3, 16, 2, 8, 4>), dim3(s->grid), dim3(256), 0, st, MA_FUSED_ARGS);
  } else {
    hipLaunchKernelGGL((k_moe_fused<1, 16, 2, 1, 8, 1, 2, 1>), dim3(s->grid), dim3(256), 0, st, MA_FUSED_ARGS);
  }
#undef MA_FUSED_ARGS
  return check_launch("moe_fused");
}

extern "C" int ma_moe_fused_timed_out(const void* workspace, int* out, void* stream) {
  // Copies the error word (1 if a wait timed out since the workspace was
  // zeroed) to host memory ``out``; synchronises the stream.
  if (!workspace || !out) return fail(MA_EVALUE, "moe_fused_timed_out: null pointer");
  uint32_t v = 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (hipMemcpyAsync(&v, static_cast<const char*>(workspace) + 8, 4, hipMemcpyDeviceToHost, st) !=
          hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess)
    return fail(MA_ERUNTIME, "moe_fused_timed_out: copy failed");
  *out = static_cast<int>(v);
  return MA_OK;
}
