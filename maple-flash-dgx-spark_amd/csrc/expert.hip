// Indexed stacked-expert ternary kernels (gfx950).
//
// Semantics follow reference src/maple_run/kernels/ternary_expert.py:
//   expert_gemv     :58-122   y[s] = alpha_e * (T_e . x_s), e = ids[s]
//   expert_swiglu   :240-319  rows [up; gate]; clamp(up,+-7) * g * sigmoid(g), g = min(gate, 7)
//   expert_down_sum :322-400  y[t] = sum_j w[t,j] * alpha_e (T_e . x[t,j]) (+ residual)
// Fast kernels: bf16 activations, [E, N, K/16] codes, nwords = KW * LPR; each
// one-wave workgroup handles U row-iterations of one slot (or token), with
// every weight load of the wave issued before the activations are prepared.
// Generic kernels: any dtype / layout, one wave per output row.
#include "ternary_engine.h"

namespace ma {


// Expert id of a slot, clamped into [0, n_exp): an id outside the stack would
// otherwise address memory outside the weights (no host-side check is possible
// without a device sync).
__device__ __forceinline__ int64_t expert_id(const void* ids, int ids64, int64_t s, int64_t n_exp) {
  const int64_t e = ld_id(ids, ids64, s);
  return e < 0 ? 0 : (e >= n_exp ? n_exp - 1 : e);
}

constexpr int kMaxStageWords = 256;  // K <= 4096 for the LDS-staged kernels

// ---------------------------------------------------------------------------
// Fast SwiGLU: the waves of a workgroup share the staged x of one token.  In a
// wave, lanes of sub-group [0, PPI) compute up rows and [PPI, 2*PPI) the
// matching gate rows; the gate value is fetched across the wave.
// ---------------------------------------------------------------------------
constexpr int kSwigluWaves = 8;

template <int KW, int LPR, int U, int ADT>
__global__ __launch_bounds__(64 * kSwigluWaves) void k_swiglu_fast(
    const uint16_t* __restrict__ x, int64_t ldx, int64_t topk,
    const uint32_t* __restrict__ w, int64_t n_half,
    const void* __restrict__ alpha, const int32_t* __restrict__ ids, int64_t n_exp,
    uint16_t* __restrict__ h, int64_t ldh) {
  constexpr int NW = KW * LPR;
  constexpr int RPI = 64 / LPR;
  constexpr int PPI = RPI / 2;
  __shared__ __align__(16) uint32_t xs[NW][8];
  __shared__ float cw[NW];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int kl = lane % LPR, sub = lane / LPR;
  const int half = sub / PPI, pi = sub % PPI;
  const int64_t slot = blockIdx.y;
  const int64_t e = clamp_id(ids[slot], n_exp);
  const uint32_t* we = w + e * (2 * n_half) * NW;
  const int64_t a_off = e * (2 * n_half);
  const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * kSwigluWaves + wv) * (PPI * U);

  uint32_t wv_[U][KW];
  float a[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    int64_t i = i0 + u * PPI + pi;
    i = i < n_half ? i : n_half - 1;
    const int64_t row = i + half * n_half;
    load_words_v<KW>(we + row * NW + kl * KW, wv_[u]);
    a[u] = ld_t<ADT>(alpha, a_off + row);
  }
  MA_ISSUE_FENCE();
  stage_row(x + (slot / topk) * ldx, NW, xs, cw);
  __syncthreads();
  XSlice<KW> xsl;
  slice_from_lds<KW>(xs, cw, kl, xsl);
  const ExpandConsts kc;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const float v = group_sum<LPR>(slice_dot<KW>(wv_[u], xsl, kc) * a[u]);
    const float g = __shfl(v, lane + PPI * LPR, 64);
    const int64_t i = i0 + u * PPI + pi;
    if (half == 0 && kl == 0 && i < n_half) h[slot * ldh + i] = f32_to_bf16(swiglu_act(v, g));
  }
}

// ---------------------------------------------------------------------------
// Fast expert GEMV: rows i0 + u*RPI + sub of expert ids[slot].
// ---------------------------------------------------------------------------
template <int KW, int LPR, int U, int ADT>
__global__ __launch_bounds__(64) void k_egemv_fast(
    const uint16_t* __restrict__ x, int64_t ldx, int64_t x_div,
    const uint32_t* __restrict__ w, int64_t n_out,
    const void* __restrict__ alpha, const int32_t* __restrict__ ids, int64_t n_exp,
    uint16_t* __restrict__ y, int64_t ldy) {
  constexpr int NW = KW * LPR;
  constexpr int RPI = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int kl = lane % LPR, sub = lane / LPR;
  const int64_t slot = blockIdx.y;
  const int64_t e = clamp_id(ids[slot], n_exp);
  const uint32_t* we = w + e * n_out * NW;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * (RPI * U);
  uint32_t wv[U][KW];
  float a[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    int64_t r = r0 + u * RPI + sub;
    r = r < n_out ? r : n_out - 1;
    load_words_v<KW>(we + r * NW + kl * KW, wv[u]);
    a[u] = ld_t<ADT>(alpha, e * n_out + r);
  }
  XSlice<KW> xs;
  xs.load(x + (slot / x_div) * ldx, kl);
  MA_ISSUE_FENCE();
  xs.finish();
  const ExpandConsts kc;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const float v = group_sum<LPR>(slice_dot<KW>(wv[u], xs, kc) * a[u]);
    const int64_t r = r0 + u * RPI + sub;
    if (kl == 0 && r < n_out) y[slot * ldy + r] = f32_to_bf16(v);
  }
}

// ---------------------------------------------------------------------------
// Fast down projection + top-k weighted combine (+ residual), float32 until
// the single store.  A workgroup owns RPI output rows of one token; its 4
// waves split the TK slots (wave w takes slots w, w + 4, ...), every lane
// loads its own K slice of each slot's activations and weights up front, and
// the waves' partial sums meet in LDS.
// ---------------------------------------------------------------------------
constexpr int kDownWaves = 8;

// ROUND (the MoE block's composition, ternary_expert_gemv then moe_reduce_add,
// model.py:470-473): each slot's output alpha * (T h) is rounded to bf16
// (with k_egemv_fast's arithmetic), then weighted and summed in slot order
// with k_moe_reduce's fused multiply-adds, the residual last
// (fused_norm.py:83-96) -- the two launches' bits; otherwise
// ternary_expert_down_sum's float32 sum.
template <int KW, int LPR, int TK, int U, int ADT, bool ROUND>
__global__ __launch_bounds__(64 * kDownWaves) void k_down_sum_fast(
    const uint16_t* __restrict__ x, int64_t ldx,
    const uint32_t* __restrict__ w, int64_t n_out,
    const void* __restrict__ alpha, const int32_t* __restrict__ ids, int64_t n_exp,
    const float* __restrict__ wts, const void* __restrict__ res, int res_dt,
    uint16_t* __restrict__ y, int64_t ldy) {
  constexpr int NW = KW * LPR;
  constexpr int RPI = 64 / LPR;
  constexpr int SPW = TK >= kDownWaves ? TK / kDownWaves : 1;  // slots per wave
  constexpr int RPB = RPI * U;                                  // rows per workgroup
  static_assert(!ROUND || SPW == 1, "per-slot rounding: one slot per wave");
  __shared__ float part[kDownWaves][RPB];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kl = lane % LPR, sub = lane / LPR;
  const int64_t t = blockIdx.y;
  const int64_t rbase = static_cast<int64_t>(blockIdx.x) * RPB;
  uint32_t wd[SPW][U][KW];
  float a[SPW][U], wj[SPW];
  XSlice<KW> xs[SPW];
#pragma unroll
  for (int q = 0; q < SPW; ++q) {
    const int j = wv + kDownWaves * q;
    const int jj = j < TK ? j : 0;  // idle waves (TK < waves) read slot 0 and add nothing
    const int64_t e = clamp_id(ids[t * TK + jj], n_exp);
    wj[q] = j < TK ? wts[t * TK + jj] : 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int64_t r = rbase + u * RPI + sub;
      r = r < n_out ? r : n_out - 1;
      load_words_v<KW>(w + (e * n_out + r) * NW + kl * KW, wd[q][u]);
      a[q][u] = ld_t<ADT>(alpha, e * n_out + r);
    }
    xs[q].load(x + (t * TK + jj) * ldx, kl);
  }
  const int64_t ro = rbase + threadIdx.x;
  float resv = 0.f;
  if (res && threadIdx.x < RPB && ro < n_out) resv = ld_f(res, res_dt, t * n_out + ro);
  MA_ISSUE_FENCE();
  const ExpandConsts kc;
  float acc[U];
#pragma unroll
  for (int u = 0; u < U; ++u) acc[u] = 0.f;
#pragma unroll
  for (int q = 0; q < SPW; ++q) {
    xs[q].finish();
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if constexpr (ROUND)
        acc[u] += slice_dot<KW>(wd[q][u], xs[q], kc) * a[q][u];
      else
        acc[u] += slice_dot<KW>(wd[q][u], xs[q], kc) * (wj[q] * a[q][u]);
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float v = group_sum<LPR>(acc[u]);
    if constexpr (ROUND) v = bf16_to_f32(f32_to_bf16(v));  // the slot's output, as stored
    if (kl == 0) part[wv][u * RPI + sub] = v;
  }
  __syncthreads();
  if (threadIdx.x < RPB && ro < n_out) {
    float v;
    if constexpr (ROUND) {
      v = 0.f;
#pragma unroll
      for (int j = 0; j < (TK < kDownWaves ? TK : kDownWaves); ++j) v = fmaf(wts[t * TK + j], part[j][threadIdx.x], v);
      v += resv;
    } else {
      v = resv;
#pragma unroll
      for (int ww = 0; ww < kDownWaves; ++ww) v += part[ww][threadIdx.x];
    }
    y[t * ldy + ro] = f32_to_bf16(v);
  }
}

// ---------------------------------------------------------------------------
// Generic kernels: one wave per (slot, row); any float dtype, either layout.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float row_dot_generic(const void* x, int x_dt, int64_t xoff,
                                                 const uint32_t* w, int64_t e, int64_t row,
                                                 int64_t n_rows, int64_t nwords, int kn,
                                                 int lane) {
  float acc = 0.f;
  const uint32_t* we = w + e * n_rows * nwords;
  for (int64_t wi = lane; wi < nwords; wi += 64) {
    const uint32_t word = kn ? we[wi * n_rows + row] : we[row * nwords + wi];
#pragma unroll 4
    for (int i = 0; i < 16; ++i) {
      const float v = static_cast<float>((word >> (2 * i)) & 3u) - 1.0f;
      acc += v * ld_f(x, x_dt, xoff + wi * 16 + i);
    }
  }
  return group_sum<64>(acc);
}

// mode 0: gemv, 1: swiglu (row = up row, gate row = row + n_half)
__global__ __launch_bounds__(256) void k_expert_generic(
    const void* __restrict__ x, int x_dt, int64_t ldx, int64_t x_div,
    const uint32_t* __restrict__ w, int64_t n_rows, int64_t n_out, int64_t nwords, int kn,
    const void* __restrict__ alpha, int a_dt, const void* __restrict__ ids, int ids64,
    int64_t n_exp, int mode, void* __restrict__ y, int y_dt, int64_t ldy) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= n_out) return;
  const int64_t slot = blockIdx.y;
  const int64_t e = expert_id(ids, ids64, slot, n_exp);
  const int64_t xoff = (slot / x_div) * ldx;
  const float v = row_dot_generic(x, x_dt, xoff, w, e, row, n_rows, nwords, kn, lane) *
                  ld_f(alpha, a_dt, e * n_rows + row);
  float out = v;
  if (mode == 1) {
    const int64_t grow = row + n_out;
    const float g = row_dot_generic(x, x_dt, xoff, w, e, grow, n_rows, nwords, kn, lane) *
                    ld_f(alpha, a_dt, e * n_rows + grow);
    out = swiglu_act(v, g);
  }
  if (lane == 0) st_f(y, y_dt, slot * ldy + row, out);
}

__global__ __launch_bounds__(256) void k_down_sum_generic(
    const void* __restrict__ x, int x_dt, int64_t ldx,
    const uint32_t* __restrict__ w, int64_t n_out, int64_t nwords, int kn,
    const void* __restrict__ alpha, int a_dt, const void* __restrict__ ids, int ids64,
    int64_t n_exp, const float* __restrict__ wts, const void* __restrict__ res, int res_dt, int64_t topk,
    void* __restrict__ y, int64_t ldy, int round_slots) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= n_out) return;
  const int64_t t = blockIdx.y;
  float acc = 0.f;
  for (int64_t j = 0; j < topk; ++j) {
    const int64_t s = t * topk + j;
    const int64_t e = expert_id(ids, ids64, s, n_exp);
    const float v = row_dot_generic(x, x_dt, s * ldx, w, e, row, n_out, nwords, kn, lane);
    float eo = v * ld_f(alpha, a_dt, e * n_out + row);
    // round_slots: each slot's output in the activation dtype first (the block's composition)
    if (round_slots) eo = x_dt == MA_BF16 ? bf16_to_f32(f32_to_bf16(eo))
                          : x_dt == MA_F16 ? static_cast<float>(static_cast<_Float16>(eo)) : eo;
    acc += wts[s] * eo;
  }
  if (lane == 0) {
    if (res) acc += ld_f(res, res_dt, t * n_out + row);
    st_f(y, x_dt, t * ldy + row, acc);
  }
}

// ---------------------------------------------------------------------------
// Host dispatch.
// ---------------------------------------------------------------------------
#define MA_EXPERT_SHAPES(X) X(32, 4) X(32, 8) X(32, 2) X(32, 1) X(32, 3) X(32, 5) X(16, 3) X(16, 1) X(8, 1)
// down projections: K = intermediate size (768 -> 48 words; 512 -> 32; 128 -> 8)
#define MA_DOWN_SHAPES(X) X(16, 3) X(32, 1) X(16, 1) X(8, 1) X(32, 2)

static bool fast_shape(int64_t nwords, int& lpr, int& kw) {
#define MA_PICK(L, K) \
  if (nwords == (L) * (K)) { lpr = L; kw = K; return true; }
  MA_EXPERT_SHAPES(MA_PICK)
#undef MA_PICK
  return false;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

static bool fast_ok(const void* x, int x_dt, int64_t ldx, const uint32_t* w, int64_t nwords,
                    int kn, int a_dt, int ids64, int& lpr, int& kw) {
  if (x_dt != MA_BF16 || kn || ids64 || (a_dt != MA_BF16 && a_dt != MA_F32)) return false;
  if (!fast_shape(nwords, lpr, kw)) return false;
  const uintptr_t wa = (kw % 4 == 0) ? 16 : (kw % 2 == 0) ? 8 : 4;
  return aligned16(x) && (ldx % 8) == 0 && (reinterpret_cast<uintptr_t>(w) % wa) == 0;
}

}  // namespace ma

using namespace ma;

extern "C" int ma_ternary_expert_swiglu(const void* x, int x_dtype, int64_t ldx, int64_t tokens,
                                        int64_t top_k, const uint32_t* packed,
                                        int64_t n_experts, int64_t n_rows, int64_t nwords,
                                        int packed_kn, const void* row_alpha, int alpha_dtype,
                                        const void* ids, int ids_is_int64, void* h, int64_t ldh,
                                        void* stream) {
  if (tokens < 0 || top_k < 1 || n_rows < 0 || (n_rows % 2) || nwords < 1 || n_experts < 1)
    return fail(MA_EVALUE, "ternary_expert_swiglu: bad sizes");
  const int64_t slots = tokens * top_k, n_half = n_rows / 2;
  if (slots == 0 || n_half == 0) return MA_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int lpr = 0, kw = 0;
  if (fast_ok(x, x_dtype, ldx, packed, nwords, packed_kn, alpha_dtype, ids_is_int64, lpr, kw) &&
      nwords <= kMaxStageWords) {
    constexpr int U = 3;
#define MA_LAUNCH(L, K)                                                                        \
  if (lpr == L && kw == K) {                                                                   \
    constexpr int PPI = (64 / L) / 2;                                                          \
    dim3 grid(static_cast<unsigned>(cdiv(n_half, kSwigluWaves * PPI * U)),                     \
              static_cast<unsigned>(slots));                                                   \
    if (alpha_dtype == MA_BF16)                                                                \
      hipLaunchKernelGGL((k_swiglu_fast<K, L, U, MA_BF16>), grid, dim3(64 * kSwigluWaves), 0, s, \
                         static_cast<const uint16_t*>(x), ldx, top_k, packed, n_half,          \
                         row_alpha, static_cast<const int32_t*>(ids), n_experts, static_cast<uint16_t*>(h), ldh);        \
    else                                                                                       \
      hipLaunchKernelGGL((k_swiglu_fast<K, L, U, MA_F32>), grid, dim3(64 * kSwigluWaves), 0, s, \
                         static_cast<const uint16_t*>(x), ldx, top_k, packed, n_half,          \
                         row_alpha, static_cast<const int32_t*>(ids), n_experts, static_cast<uint16_t*>(h), ldh);        \
    return check_launch("ternary_expert_swiglu");                                             \
  }
    MA_EXPERT_SHAPES(MA_LAUNCH)
#undef MA_LAUNCH
  }
  dim3 grid(static_cast<unsigned>(cdiv(n_half, 4)), static_cast<unsigned>(slots));
  hipLaunchKernelGGL(k_expert_generic, grid, dim3(256), 0, s, x, x_dtype, ldx, top_k, packed,
                     n_rows, n_half, nwords, packed_kn, row_alpha, alpha_dtype, ids,
                     ids_is_int64, n_experts, 1, h, x_dtype, ldh);
  return check_launch("ternary_expert_swiglu");
}

extern "C" int ma_ternary_expert_gemv(const void* x, int x_dtype, int64_t ldx, int64_t x_div,
                                      const uint32_t* packed, int64_t n_experts, int64_t n_out,
                                      int64_t nwords, int packed_kn, const void* row_alpha,
                                      int alpha_dtype, const void* ids, int ids_is_int64,
                                      int64_t n_slots, void* y, int64_t ldy, void* stream) {
  if (n_slots < 0 || n_out < 0 || nwords < 1 || x_div < 1 || n_experts < 1)
    return fail(MA_EVALUE, "ternary_expert_gemv: bad sizes");
  if (n_slots == 0 || n_out == 0) return MA_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int lpr = 0, kw = 0;
  if (fast_ok(x, x_dtype, ldx, packed, nwords, packed_kn, alpha_dtype, ids_is_int64, lpr, kw)) {
    constexpr int U = 2;
#define MA_LAUNCH(L, K)                                                                        \
  if (lpr == L && kw == K) {                                                                   \
    dim3 grid(static_cast<unsigned>(cdiv(n_out, (64 / L) * U)), static_cast<unsigned>(n_slots)); \
    if (alpha_dtype == MA_BF16)                                                                \
      hipLaunchKernelGGL((k_egemv_fast<K, L, U, MA_BF16>), grid, dim3(64), 0, s,               \
                         static_cast<const uint16_t*>(x), ldx, x_div, packed, n_out,           \
                         row_alpha, static_cast<const int32_t*>(ids), n_experts, static_cast<uint16_t*>(y), ldy);        \
    else                                                                                       \
      hipLaunchKernelGGL((k_egemv_fast<K, L, U, MA_F32>), grid, dim3(64), 0, s,                \
                         static_cast<const uint16_t*>(x), ldx, x_div, packed, n_out,           \
                         row_alpha, static_cast<const int32_t*>(ids), n_experts, static_cast<uint16_t*>(y), ldy);        \
    return check_launch("ternary_expert_gemv");                                               \
  }
    MA_EXPERT_SHAPES(MA_LAUNCH)
#undef MA_LAUNCH
  }
  dim3 grid(static_cast<unsigned>(cdiv(n_out, 4)), static_cast<unsigned>(n_slots));
  hipLaunchKernelGGL(k_expert_generic, grid, dim3(256), 0, s, x, x_dtype, ldx, x_div, packed,
                     n_out, n_out, nwords, packed_kn, row_alpha, alpha_dtype, ids,
                     ids_is_int64, n_experts, 0, y, x_dtype, ldy);
  return check_launch("ternary_expert_gemv");
}

template <bool ROUND>
static int down_sum_impl(const void* x, int x_dtype, int64_t ldx, const uint32_t* packed, int64_t n_experts,
                         int64_t n_out, int64_t nwords, int packed_kn, const void* row_alpha, int alpha_dtype,
                         const void* ids, int ids_is_int64, const float* topk_weight, const void* residual,
                         int residual_dtype, int64_t tokens, int64_t top_k, void* y, int64_t ldy, void* stream) {
  if (tokens < 0 || top_k < 1 || n_out < 0 || nwords < 1 || n_experts < 1)
    return fail(MA_EVALUE, "ternary_expert_down_sum: bad sizes");
  if (tokens == 0 || n_out == 0) return MA_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int lpr = 0, kw = 0;
  const bool tk_ok = top_k == 8 || top_k == 4 || top_k == 2 || top_k == 1;
  if (tk_ok && fast_ok(x, x_dtype, ldx, packed, nwords, packed_kn, alpha_dtype, ids_is_int64, lpr, kw)) {
#define MA_LAUNCH_TK(L, K, TK)                                                                 \
  if (lpr == L && kw == K && top_k == TK) {                                                    \
    constexpr int U = 2;                                                                       \
    dim3 grid(static_cast<unsigned>(cdiv(n_out, (64 / L) * U)), static_cast<unsigned>(tokens)); \
    const auto* xb = static_cast<const uint16_t*>(x);                                          \
    const auto* ib = static_cast<const int32_t*>(ids);                                         \
    auto* yb = static_cast<uint16_t*>(y);                                                      \
    if (alpha_dtype == MA_BF16)                                                                \
      hipLaunchKernelGGL((k_down_sum_fast<K, L, TK, U, MA_BF16, ROUND>), grid, dim3(64 * kDownWaves), 0, s, xb, ldx, \
                         packed, n_out, row_alpha, ib, n_experts, topk_weight, residual,       \
                         residual_dtype, yb, ldy);                                             \
    else                                                                                       \
      hipLaunchKernelGGL((k_down_sum_fast<K, L, TK, U, MA_F32, ROUND>), grid, dim3(64 * kDownWaves), 0, s, xb, ldx, \
                         packed, n_out, row_alpha, ib, n_experts, topk_weight, residual,       \
                         residual_dtype, yb, ldy);                                             \
    return check_launch("ternary_expert_down_sum");                                           \
  }
#define MA_LAUNCH(L, K) MA_LAUNCH_TK(L, K, 8) MA_LAUNCH_TK(L, K, 4) MA_LAUNCH_TK(L, K, 2) MA_LAUNCH_TK(L, K, 1)
    MA_DOWN_SHAPES(MA_LAUNCH)
#undef MA_LAUNCH
#undef MA_LAUNCH_TK
  }
  dim3 grid(static_cast<unsigned>(cdiv(n_out, 4)), static_cast<unsigned>(tokens));
  hipLaunchKernelGGL(k_down_sum_generic, grid, dim3(256), 0, s, x, x_dtype, ldx, packed, n_out,
                     nwords, packed_kn, row_alpha, alpha_dtype, ids, ids_is_int64, n_experts, topk_weight,
                     residual, residual_dtype, top_k, y, ldy, ROUND ? 1 : 0);
  return check_launch("ternary_expert_down_sum");
}

extern "C" int ma_ternary_expert_down_sum(const void* x, int x_dtype, int64_t ldx,
                                          const uint32_t* packed, int64_t n_experts,
                                          int64_t n_out, int64_t nwords, int packed_kn,
                                          const void* row_alpha, int alpha_dtype,
                                          const void* ids, int ids_is_int64,
                                          const float* topk_weight, const void* residual,
                                          int residual_dtype, int64_t tokens, int64_t top_k,
                                          void* y, int64_t ldy, void* stream) {
  return down_sum_impl<false>(x, x_dtype, ldx, packed, n_experts, n_out, nwords, packed_kn, row_alpha,
                              alpha_dtype, ids, ids_is_int64, topk_weight, residual, residual_dtype, tokens,
                              top_k, y, ldy, stream);
}

// The MoE block's down projection and combine (ternary_expert_gemv, then
// moe_reduce_add) in one launch: each slot's output rounded to the
// activation dtype before the float32 weighted sum, the residual last.
extern "C" int ma_ternary_expert_down_combine(const void* x, int x_dtype, int64_t ldx,
                                              const uint32_t* packed, int64_t n_experts,
                                              int64_t n_out, int64_t nwords, int packed_kn,
                                              const void* row_alpha, int alpha_dtype,
                                              const void* ids, int ids_is_int64,
                                              const float* topk_weight, const void* residual,
                                              int residual_dtype, int64_t tokens, int64_t top_k,
                                              void* y, int64_t ldy, void* stream) {
  return down_sum_impl<true>(x, x_dtype, ldx, packed, n_experts, n_out, nwords, packed_kn, row_alpha,
                             alpha_dtype, ids, ids_is_int64, topk_weight, residual, residual_dtype, tokens,
                             top_k, y, ldy, stream);
}
