// Fast packed-ternary GEMV kernel template (bf16 activations, [N, K/16] codes).
//
// A row is split over LPR lanes, each owning KW consecutive words (one 16-byte
// load for KW = 4), so a one-wave workgroup streams RPI = 64 / LPR whole rows
// with fully coalesced loads, issued before anything else the wave does.  Each lane keeps the x' pairs of its K slice in
// registers for the whole kernel; a word costs 4 shifts + 8 and/or + 8
// v_dot2_f32_bf16 (expand_word in common.h).  Up to BT activation rows share
// every expanded word, so the codes are read once per BT tokens.  With RMS the
// input RMSNorm is folded in (reference kernels/ternary_gemv.py:110-146) and
// x * w_rms is carried as a hi + lo bf16 pair to keep float32 precision.
#pragma once

#include "common.h"

namespace ma {

template <int KW>
__device__ __forceinline__ void load_words(const uint32_t* __restrict__ p, uint32_t out[KW]) {
  if constexpr (KW % 4 == 0) {
#pragma unroll
    for (int i = 0; i < KW / 4; ++i) {
      const uint4 v = reinterpret_cast<const uint4*>(p)[i];
      out[4 * i + 0] = v.x;
      out[4 * i + 1] = v.y;
      out[4 * i + 2] = v.z;
      out[4 * i + 3] = v.w;
    }
  } else if constexpr (KW % 2 == 0) {
#pragma unroll
    for (int i = 0; i < KW / 2; ++i) {
      const uint2 v = reinterpret_cast<const uint2*>(p)[i];
      out[2 * i + 0] = v.x;
      out[2 * i + 1] = v.y;
    }
  } else {
#pragma unroll
    for (int i = 0; i < KW; ++i) out[i] = p[i];
  }
}

// 16 bf16 activations starting at p (16-byte aligned) widened to float.
__device__ __forceinline__ void load_x16_bf16(const uint16_t* __restrict__ p, float xs[16]) {
  const uint4 a = reinterpret_cast<const uint4*>(p)[0];
  const uint4 b = reinterpret_cast<const uint4*>(p)[1];
  const uint32_t u[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    xs[2 * i] = __uint_as_float(u[i] << 16);
    xs[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
  }
}

// hi/lo bf16 split of f * v for the fused-RMS path: hi + lo carries v to
// ~16 mantissa bits.  Returns the value the pair actually represents.
__device__ __forceinline__ float split_hi_lo(float fv, uint16_t& hi, uint16_t& lo) {
  hi = f32_to_bf16(fv);
  const float r = fv - bf16_to_f32(hi);
  lo = f32_to_bf16(r);
  return bf16_to_f32(hi) + bf16_to_f32(lo);
}

template <int KW, int LPR, int BT, bool RMS, int ADT>
__global__ __launch_bounds__(64) void k_tgemv_fast(
    const uint16_t* __restrict__ x, int64_t batch, int64_t ldx,
    const uint32_t* __restrict__ w, int64_t n_out,
    const void* __restrict__ alpha,
    const float* __restrict__ rms_w, float eps,
    uint16_t* __restrict__ y, int64_t ldy) {
  constexpr int NW = KW * LPR;   // words per row
  constexpr int RPI = 64 / LPR;  // rows per wave
  const int lane = threadIdx.x & 63;
  const int kl = lane % LPR;
  const int sub = lane / LPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPI + sub;
  const bool ok = row < n_out;
  const int64_t rrow = ok ? row : n_out - 1;  // clamped: every load stays in bounds
  const int64_t b0 = static_cast<int64_t>(blockIdx.y) * BT;

  // Weight words and alpha first, so their latency overlaps the x' set-up.
  uint32_t wv[KW];
  load_words<KW>(w + rrow * NW + kl * KW, wv);
  const float a = ld_t<ADT>(alpha, rrow);

  uint32_t xh[BT][KW][8];
  uint32_t xl[RMS ? BT : 1][KW][8];
  float cst[BT];
  float rstd[BT];
  // Raw activations for every (row, word) first: all x loads in one batch.
  uint4 xr[BT][KW][2];
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) {
    const int64_t b = b0 + bt;
    const int64_t rb = b < batch ? b : batch - 1;
#pragma unroll
    for (int i = 0; i < KW; ++i) {
      const uint4* px = reinterpret_cast<const uint4*>(x + rb * ldx + static_cast<int64_t>(kl * KW + i) * 16);
      xr[bt][i][0] = px[0];
      xr[bt][i][1] = px[1];
    }
  }
  float rmsv[RMS ? KW : 1][RMS ? 16 : 1];
  if constexpr (RMS) {
#pragma unroll
    for (int i = 0; i < KW; ++i)
#pragma unroll
      for (int q = 0; q < 16; ++q) rmsv[i][q] = rms_w[static_cast<int64_t>(kl * KW + i) * 16 + q];
  }
  MA_ISSUE_FENCE();

#pragma unroll
  for (int bt = 0; bt < BT; ++bt) {
    const bool valid = b0 + bt < batch;
    float c = 0.f, ss = 0.f;
#pragma unroll
    for (int i = 0; i < KW; ++i) {
      float xs[16];
      const uint32_t u[8] = {xr[bt][i][0].x, xr[bt][i][0].y, xr[bt][i][0].z, xr[bt][i][0].w,
                             xr[bt][i][1].x, xr[bt][i][1].y, xr[bt][i][1].z, xr[bt][i][1].w};
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        xs[2 * q] = valid ? __uint_as_float(u[q] << 16) : 0.f;
        xs[2 * q + 1] = valid ? __uint_as_float(u[q] & 0xffff0000u) : 0.f;
      }
      if constexpr (RMS) {
        // per word: the sums over its halves (values 0..7 and 8..15; pairs
        // 0..3 and 4..7) each in order, then added, then the words in order
        // -- an order the fused next projection reproduces from per-half
        // partial sums
        float s2[2] = {0.f, 0.f}, ch[2] = {0.f, 0.f};
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          s2[q >> 3] += xs[q] * xs[q];
          xs[q] *= rmsv[i][q];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float f = pair_scale(j);
          uint16_t ha, la, hb, lb;
          const float ra = split_hi_lo(f * xs[j], ha, la);
          const float rb2 = split_hi_lo(f * xs[j + 8], hb, lb);
          xh[bt][i][j] = static_cast<uint32_t>(ha) | (static_cast<uint32_t>(hb) << 16);
          xl[bt][i][j] = static_cast<uint32_t>(la) | (static_cast<uint32_t>(lb) << 16);
          ch[j >> 2] += ((f + 1.0f) / f) * (ra + rb2);
        }
        ss += s2[0] + s2[1];
        c += ch[0] + ch[1];
      } else {
        c += prep_word_pairs(xs, xh[bt][i]);
      }
    }
    cst[bt] = c;
    if constexpr (RMS) {
      ss = group_sum<LPR>(ss);
      rstd[bt] = rsqrtf(ss / static_cast<float>(NW * 16) + eps);
    } else {
      rstd[bt] = 1.f;
    }
  }

  // Two accumulators per activation row break the v_dot2 dependency chain.
  const ExpandConsts kc;
  float acc[BT][2];
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) acc[bt][0] = acc[bt][1] = 0.f;
#pragma unroll
  for (int i = 0; i < KW; ++i) {
    uint32_t e[8];
    expand_word(wv[i], e, kc);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int bt = 0; bt < BT; ++bt) {
        acc[bt][j & 1] = dot2(e[j], xh[bt][i][j], acc[bt][j & 1]);
        if constexpr (RMS) acc[bt][j & 1] = dot2(e[j], xl[bt][i][j], acc[bt][j & 1]);
      }
    }
  }
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) {
    // alpha is uniform over the row's lanes: scaling before the reduction
    // keeps its (early) load off the tail of the kernel.
    const float d = group_sum<LPR>(((acc[bt][0] + acc[bt][1]) - cst[bt]) * (a * rstd[bt]));
    const int64_t b = b0 + bt;
    if (ok && kl == 0 && b < batch) y[b * ldy + row] = f32_to_bf16(d);
  }
}

// (LPR, KW) shapes with a fast kernel: nwords = LPR * KW.
#define MA_TGEMV_SHAPES(X) \
  X(32, 1) X(32, 2) X(32, 3) X(32, 4) X(32, 5) X(32, 8) X(16, 1) X(16, 3) X(8, 1)

template <int KW, int LPR, int BT, bool RMS>
void launch_tgemv_fast(const void* x, int64_t batch, int64_t ldx, const uint32_t* w,
                       int64_t n_out, const void* alpha, int alpha_dt, const void* rms_w,
                       int rms_dt, float eps, void* y, int64_t ldy, hipStream_t s) {
  (void)rms_dt;  // the fast path takes float32 RMS weights only
  constexpr int RPI = 64 / LPR;
  dim3 grid(static_cast<unsigned>(cdiv(n_out, RPI)), static_cast<unsigned>(cdiv(batch, BT)));
  const auto* xb = static_cast<const uint16_t*>(x);
  const auto* rw = static_cast<const float*>(rms_w);
  auto* yb = static_cast<uint16_t*>(y);
  if (alpha_dt == MA_BF16)
    hipLaunchKernelGGL((k_tgemv_fast<KW, LPR, BT, RMS, MA_BF16>), grid, dim3(64), 0, s, xb,
                       batch, ldx, w, n_out, alpha, rw, eps, yb, ldy);
  else
    hipLaunchKernelGGL((k_tgemv_fast<KW, LPR, BT, RMS, MA_F32>), grid, dim3(64), 0, s, xb,
                       batch, ldx, w, n_out, alpha, rw, eps, yb, ldy);
}

// Launch the (lpr, kw) instance for one (BT, RMS) variant; false if absent.
template <int BT, bool RMS>
bool tgemv_fast_variant(int lpr, int kw, const void* x, int64_t batch, int64_t ldx,
                        const uint32_t* w, int64_t n_out, const void* alpha, int alpha_dt,
                        const void* rms_w, int rms_dt, float eps, void* y, int64_t ldy,
                        hipStream_t s) {
#define MA_TGEMV_CASE(L, K)                                                                 \
  if (lpr == L && kw == K) {                                                                \
    launch_tgemv_fast<K, L, BT, RMS>(x, batch, ldx, w, n_out, alpha, alpha_dt, rms_w, rms_dt, \
                                     eps, y, ldy, s);                                        \
    return true;                                                                            \
  }
  MA_TGEMV_SHAPES(MA_TGEMV_CASE)
#undef MA_TGEMV_CASE
  return false;
}

// Per-variant entry points, one translation unit each (parallel compile).
#define MA_TGEMV_VARIANT_DECL(NAME)                                                         \
  bool NAME(int lpr, int kw, const void* x, int64_t batch, int64_t ldx, const uint32_t* w, \
            int64_t n_out, const void* alpha, int alpha_dt, const void* rms_w, int rms_dt,   \
            float eps, void* y, int64_t ldy, hipStream_t s);
MA_TGEMV_VARIANT_DECL(tgemv_fast_b1)
MA_TGEMV_VARIANT_DECL(tgemv_fast_b2)
MA_TGEMV_VARIANT_DECL(tgemv_fast_b4)
MA_TGEMV_VARIANT_DECL(tgemv_fast_rms1)
MA_TGEMV_VARIANT_DECL(tgemv_fast_rms2)

// True when (nwords) has a fast shape; sets lpr / kw.
inline bool tgemv_fast_shape(int64_t nwords, int& lpr, int& kw) {
#define MA_TGEMV_PICK(L, K) \
  if (nwords == (L) * (K)) { lpr = L; kw = K; return true; }
  MA_TGEMV_SHAPES(MA_TGEMV_PICK)
#undef MA_TGEMV_PICK
  return false;
}

}  // namespace ma
