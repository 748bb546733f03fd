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

}  // namespace ma
