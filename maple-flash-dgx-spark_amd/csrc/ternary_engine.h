// Per-lane building blocks of the bf16 fast ternary kernels (expert GEMV,
// SwiGLU, down + combine).  A row of NW = KW * LPR words is split over LPR
// lanes; lane kl owns words [kl*KW, kl*KW + KW) and the matching 16*KW
// activations, held as x' pairs (see expand_word in common.h).
#pragma once

#include "common.h"

namespace ma {

template <int KW>
__device__ __forceinline__ void load_words_v(const uint32_t* __restrict__ p, uint32_t out[KW]) {
  if constexpr (KW % 4 == 0) {
#pragma unroll
    for (int i = 0; i < KW / 4; ++i) {
      const uint4 v = reinterpret_cast<const uint4*>(p)[i];
      out[4 * i + 0] = v.x;
      out[4 * i + 1] = v.y;
      out[4 * i + 2] = v.z;
      out[4 * i + 3] = v.w;
    }
  } else if constexpr (KW == 3) {  // one 12-byte load (global_load_dwordx3) instead of three
    typedef uint32_t u32x3_t __attribute__((ext_vector_type(3)));
    const u32x3_t v = *reinterpret_cast<const u32x3_t*>(p);
    out[0] = v.x;
    out[1] = v.y;
    out[2] = v.z;
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

// x' pairs and the cancelling constant of one lane's K slice of one bf16 row.
template <int KW>
struct XSlice {
  uint32_t xp[KW][8];
  float c;

  // Raw loads only (issue early); finish() converts.
  uint4 raw[KW][2];
  __device__ __forceinline__ void load(const uint16_t* __restrict__ row, int kl) {
#pragma unroll
    for (int i = 0; i < KW; ++i) {
      const uint4* p = reinterpret_cast<const uint4*>(row + static_cast<int64_t>(kl * KW + i) * 16);
      raw[i][0] = p[0];
      raw[i][1] = p[1];
    }
  }
  __device__ __forceinline__ void finish() {
    c = 0.f;
#pragma unroll
    for (int i = 0; i < KW; ++i) {
      const uint32_t u[8] = {raw[i][0].x, raw[i][0].y, raw[i][0].z, raw[i][0].w,
                             raw[i][1].x, raw[i][1].y, raw[i][1].z, raw[i][1].w};
      float xs[16];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        xs[2 * q] = __uint_as_float(u[q] << 16);
        xs[2 * q + 1] = __uint_as_float(u[q] & 0xffff0000u);
      }
      c += prep_word_pairs(xs, xp[i]);
    }
  }
};

// sum_k (code_k - 1) x_k over the lane's slice (before the cross-lane sum).
template <int KW>
__device__ __forceinline__ float slice_dot(const uint32_t wv[KW], const XSlice<KW>& xs,
                                           const ExpandConsts& kc) {
  float a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int i = 0; i < KW; ++i) {
    uint32_t e[8];
    expand_word(wv[i], e, kc);
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      a0 = dot2(e[j], xs.xp[i][j], a0);
      a1 = dot2(e[j + 1], xs.xp[i][j + 1], a1);
    }
  }
  return (a0 + a1) - xs.c;
}

// The fast kernels take int32 ids only (one scalar load, no dtype branch).
__device__ __forceinline__ int64_t clamp_id(int32_t e, int64_t n_exp) {
  return e < 0 ? 0 : (e >= n_exp ? n_exp - 1 : e);
}


// ---------------------------------------------------------------------------
// x' staging in LDS: one workgroup prepares the pairs of one bf16 activation
// row once (thread t -> word t), so its waves do not each reload and
// re-convert x.  xs[w][j] = pair j of word w, cw[w] = sum (f_j + 1) x over w.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void stage_row(const uint16_t* __restrict__ row, int64_t nwords,
                                          uint32_t (*xs)[8], float* cw) {
  for (int64_t wi = threadIdx.x; wi < nwords; wi += blockDim.x) {
    const uint4 a = reinterpret_cast<const uint4*>(row + wi * 16)[0];
    const uint4 b = reinterpret_cast<const uint4*>(row + wi * 16)[1];
    const uint32_t u[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    float v[16];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      v[2 * q] = __uint_as_float(u[q] << 16);
      v[2 * q + 1] = __uint_as_float(u[q] & 0xffff0000u);
    }
    uint32_t pr[8];
    cw[wi] = prep_word_pairs(v, pr);
#pragma unroll
    for (int j = 0; j < 8; ++j) xs[wi][j] = pr[j];
  }
}

template <int KW>
__device__ __forceinline__ void slice_from_lds(const uint32_t (*xs)[8], const float* cw, int kl,
                                               XSlice<KW>& out) {
  out.c = 0.f;
#pragma unroll
  for (int i = 0; i < KW; ++i) {
    const int w = kl * KW + i;
    const uint4 lo = *reinterpret_cast<const uint4*>(&xs[w][0]);
    const uint4 hi = *reinterpret_cast<const uint4*>(&xs[w][4]);
    out.xp[i][0] = lo.x; out.xp[i][1] = lo.y; out.xp[i][2] = lo.z; out.xp[i][3] = lo.w;
    out.xp[i][4] = hi.x; out.xp[i][5] = hi.y; out.xp[i][6] = hi.z; out.xp[i][7] = hi.w;
    out.c += cw[w];
  }
}

}  // namespace ma
