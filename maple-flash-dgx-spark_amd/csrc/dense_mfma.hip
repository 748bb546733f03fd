// Batched dense GEMMs on MFMA for the decode step at batch > 4 (gfx950):
// the packed ternary projection (reference _ternary_gemm_kernel,
// src/maple_run/kernels/ternary_gemv.py:156-258, with the optional fused input
// RMSNorm kept as the x_hi + x_lo bf16 split of :241-248) and the 4-bit RTN
// lm_head (_rtn4_gemm_kernel, src/maple_run/kernels/rtn4.py:170-282, in the
// factored per-group form s_g (q.x)_g + b_g sum_g x of :197-208).
//
// y[t, n] for a tile of rows (4 waves x MB blocks of 16; the ternary GEMM uses
// MB = 1, the RTN4 one MB = 2) and 16*NB tokens, K walked in chunks of 16
// words with the next chunk's weights and activations loaded ahead.  v_mfma_f32_16x16x32_bf16 layouts (checked
// on the device): A lane l holds row l%16, k 8(l/16)..+8; B col l%16, k
// 8(l/16)..+8; C col l%16, rows 4(l/16)..+4.
//
// Ternary: a lane expands one 16-code word into 8 bf16x2 dwords of 1 + c/f
// (expand_word) = two MFMA k-slices; B holds the matching x' = f x pairs from
// LDS, so C accumulates sum (f + c) x and y = alpha (C - sum (f + 1) x).
// RTN4: a word's 8 codes expand to 4 dwords of 1 + q/16 = one k-slice against
// x' = 16 x pairs; after each RTN group C is folded into the output as
// s_g (C - 16 X_g) + b_g X_g (X_g = sum of x over the group) and cleared.
#include "common.h"

namespace ma {

typedef __bf16 bf16x8d_t __attribute__((ext_vector_type(8)));
typedef float f32x4d_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4d_t mfma16(uint4 a, uint4 b, f32x4d_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8d_t, a),
                                                 __builtin_bit_cast(bf16x8d_t, b), c, 0, 0, 0);
}

constexpr int kDenseChunk = 16;  // words of K per step
constexpr int kDenseRows = 128;  // rows per workgroup (4 waves x 2 x 16)
constexpr int kRmsMaxK = 8192;   // K of the RMS-folded ternary GEMM, at most
constexpr uint32_t kMaskQ4d = 0x00780078u;

// ---------------------------------------------------------------------------
// Ternary: y = alpha (.) (T x_hat) [* rsqrt(mean(x^2) + eps) with RMS], where
// x_hat = x * w_rms split as hi + lo bf16 when RMS.
// ---------------------------------------------------------------------------
// 16 weights of the input RMSNorm (float32 or bf16) for K positions 16 wd ..
__device__ __forceinline__ void load_rms16(const void* p, int rdt, int64_t wd, float out[16]) {
  if (rdt == MA_F32) {
    const uint4* q = reinterpret_cast<const uint4*>(static_cast<const float*>(p) + wd * 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 v = q[i];
      out[4 * i] = __uint_as_float(v.x);
      out[4 * i + 1] = __uint_as_float(v.y);
      out[4 * i + 2] = __uint_as_float(v.z);
      out[4 * i + 3] = __uint_as_float(v.w);
    }
  } else {
    const uint4* q = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + wd * 16);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint4 v = q[i];
      const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        out[8 * i + 2 * j] = __uint_as_float(u[j] << 16);
        out[8 * i + 2 * j + 1] = __uint_as_float(u[j] & 0xffff0000u);
      }
    }
  }
}

template <int NB, int MB, bool RMS, int ADT>
__global__ __launch_bounds__(256) void k_tgemm_mfma(
    const uint16_t* __restrict__ x, int64_t batch, int64_t ldx, const uint32_t* __restrict__ w,
    int64_t n_out, int64_t nwords, const void* __restrict__ alpha,
    const void* __restrict__ rms_w, int rms_dt, float rms_eps, uint16_t* __restrict__ y,
    int64_t ldy) {
  constexpr int NT = 16 * NB, NV = RMS ? 2 : 1, ROWS = 64 * MB;
  // x' pairs, word-major: a B fragment read by 16 lanes (16 tokens) is one
  // contiguous 256-byte run, so the reads are free of bank conflicts.
  __shared__ __align__(16) uint32_t xs[NV][kDenseChunk][2][NT][4];
  __shared__ float cst[NT], ssq[NT];
  // RMS weights of all of K, staged once (kRmsMaxK positions at most)
  __shared__ __align__(16) float rws[RMS ? kRmsMaxK : 1];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int64_t t0 = static_cast<int64_t>(blockIdx.y) * NT;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * ROWS + 16 * MB * wv;
  if (tid < NT) {
    cst[tid] = 0.f;
    ssq[tid] = 0.f;
  }
  const uint32_t* rowp[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    int64_t r = row0 + 16 * mb + r16;
    r = r < n_out ? r : n_out - 1;
    rowp[mb] = w + r * nwords + 4 * g;
  }
  f32x4d_t acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x4d_t{0.f, 0.f, 0.f, 0.f};
  const ExpandConsts kc;
  // x (and RMS weight) loads of chunk c0 for this thread's staging items.
  auto load_x = [&](int64_t c0, uint4 (&xa)[NB], uint4 (&xb)[NB]) {
#pragma unroll
    for (int it = 0; it < NB; ++it) {
      const int item = tid + 256 * it;
      const int col = item % NT, wd = item / NT;
      int64_t t = t0 + col;
      t = t < batch ? t : batch - 1;
      const uint4* src = reinterpret_cast<const uint4*>(x + t * ldx + (c0 + wd) * 16);
      xa[it] = src[0];
      xb[it] = src[1];
    }
  };
  uint4 wq[MB], xa[NB], xb[NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) wq[mb] = *reinterpret_cast<const uint4*>(rowp[mb]);
  load_x(0, xa, xb);
  if constexpr (RMS) {
    for (int64_t wd = tid; wd < nwords; wd += 256) {
      float r[16];
      load_rms16(rms_w, rms_dt, wd, r);
#pragma unroll
      for (int q = 0; q < 16; ++q) rws[wd * 16 + q] = r[q];
    }
  }
  // A thread stages the same token column in every chunk, so its share of the
  // token's correction (and squares) accumulates in registers; one reduction
  // over the column's threads at the end.
  float c_acc[NB], ss_acc[NB];
#pragma unroll
  for (int it = 0; it < NB; ++it) c_acc[it] = ss_acc[it] = 0.f;
  __syncthreads();
  for (int64_t c0 = 0; c0 < nwords; c0 += kDenseChunk) {
    // Next chunk's weights and x, in flight during this chunk's work.
    const int64_t cn = c0 + kDenseChunk < nwords ? c0 + kDenseChunk : c0;
    uint4 wn[MB], xan[NB], xbn[NB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) wn[mb] = *reinterpret_cast<const uint4*>(rowp[mb] + cn);
    load_x(cn, xan, xbn);
    // (no sched_barrier here: with loads into loop-carried registers just
    // above, it produced wrong MFMA operands on this compiler)
#pragma unroll
    for (int it = 0; it < NB; ++it) {
      const int item = tid + 256 * it;
      const int col = item % NT, wd = item / NT;
      const bool valid = t0 + col < batch;
      const uint32_t u[8] = {xa[it].x, xa[it].y, xa[it].z, xa[it].w,
                             xb[it].x, xb[it].y, xb[it].z, xb[it].w};
      float v[16];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        v[2 * q] = valid ? __uint_as_float(u[q] << 16) : 0.f;
        v[2 * q + 1] = valid ? __uint_as_float(u[q] & 0xffff0000u) : 0.f;
      }
      uint32_t pr[8];
      float c;
      if constexpr (RMS) {
        float ss = 0.f, hi[16], lo[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          ss += v[q] * v[q];
          const float xh = v[q] * rws[(c0 + wd) * 16 + q];
          hi[q] = bf16_to_f32(f32_to_bf16(xh));
          lo[q] = bf16_to_f32(f32_to_bf16(xh - hi[q]));
        }
        c = prep_word_pairs(hi, pr);
        *reinterpret_cast<uint4*>(&xs[0][wd][0][col][0]) = make_uint4(pr[0], pr[1], pr[2], pr[3]);
        *reinterpret_cast<uint4*>(&xs[0][wd][1][col][0]) = make_uint4(pr[4], pr[5], pr[6], pr[7]);
        c += prep_word_pairs(lo, pr);
        *reinterpret_cast<uint4*>(&xs[NV - 1][wd][0][col][0]) = make_uint4(pr[0], pr[1], pr[2], pr[3]);
        *reinterpret_cast<uint4*>(&xs[NV - 1][wd][1][col][0]) = make_uint4(pr[4], pr[5], pr[6], pr[7]);
        ss_acc[it] += ss;
      } else {
        c = prep_word_pairs(v, pr);
        *reinterpret_cast<uint4*>(&xs[0][wd][0][col][0]) = make_uint4(pr[0], pr[1], pr[2], pr[3]);
        *reinterpret_cast<uint4*>(&xs[0][wd][1][col][0]) = make_uint4(pr[4], pr[5], pr[6], pr[7]);
      }
      c_acc[it] += c;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 4; ++q) {  // word q of the lane's 4 -> k-slices 2q, 2q+1
      uint4 a[MB][2];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const uint32_t wsel = q == 0 ? wq[mb].x : q == 1 ? wq[mb].y : q == 2 ? wq[mb].z : wq[mb].w;
        uint32_t ex[8];
        expand_word(wsel, ex, kc);
        a[mb][0] = make_uint4(ex[0], ex[1], ex[2], ex[3]);
        a[mb][1] = make_uint4(ex[4], ex[5], ex[6], ex[7]);
      }
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int vv = 0; vv < NV; ++vv)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            const uint4 b = *reinterpret_cast<const uint4*>(&xs[vv][4 * g + q][hf][nb * 16 + r16][0]);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) acc[mb][nb] = mfma16(a[mb][hf], b, acc[mb][nb]);
          }
    }
    __syncthreads();
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) wq[mb] = wn[mb];
#pragma unroll
    for (int it = 0; it < NB; ++it) {
      xa[it] = xan[it];
      xb[it] = xbn[it];
    }
  }
  {  // the columns' correction and squares, summed over their threads in a fixed order
    __shared__ float red_c[256], red_s[256];
    float cs = 0.f, s2 = 0.f;
#pragma unroll
    for (int it = 0; it < NB; ++it) {  // every item of this thread is column tid % NT
      cs += c_acc[it];
      s2 += ss_acc[it];
    }
    red_c[tid] = cs;
    red_s[tid] = s2;
    __syncthreads();
    if (tid < NT) {
      float a = 0.f, b = 0.f;
      for (int k = 0; k < 256 / NT; ++k) {
        a += red_c[tid + NT * k];
        b += red_s[tid + NT * k];
      }
      cst[tid] = a;
      ssq[tid] = b;
    }
    __syncthreads();
  }
  // Epilogue: lane holds token col r16 of block nb, rows 4g .. 4g+3 of block mb.
  const int64_t kin = nwords * 16;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int col = nb * 16 + r16;
    const int64_t t = t0 + col;
    if (t >= batch) continue;
    const float cc = cst[col];
    const float scale = RMS ? rsqrtf(ssq[col] / static_cast<float>(kin) + rms_eps) : 1.f;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int64_t n0 = row0 + 16 * mb + 4 * g;
      float o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t n = n0 + i < n_out ? n0 + i : n_out - 1;
        o[i] = ld_t<ADT>(alpha, n) * (acc[mb][nb][i] - cc) * scale;
      }
      if (n0 + 3 < n_out && (ldy % 4) == 0) {
        uint2 r;
        r.x = pack_bf16x2_rn(o[0], o[1]);
        r.y = pack_bf16x2_rn(o[2], o[3]);
        *reinterpret_cast<uint2*>(y + t * ldy + n0) = r;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (n0 + i < n_out) y[t * ldy + n0 + i] = f32_to_bf16(o[i]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// RTN4: y[t, n] = sum_g s[n,g] (sum_{k in g} q x) + b[n,g] sum_{k in g} x.
// GW = words per RTN group (8: group 64, 16: group 128).  Lane group g takes
// words g, g + 4, g + 8, g + 12 of a chunk, so k-slice s covers words
// 4s .. 4s+3 and a group is a run of whole k-slices.
// ---------------------------------------------------------------------------
template <int NB, int GW, int SDT>
__global__ __launch_bounds__(256) void k_rtn4_mfma(
    const uint16_t* __restrict__ x, int64_t batch, int64_t ldx, const uint32_t* __restrict__ w,
    int64_t n_out, int64_t nwords, const void* __restrict__ scales,
    const void* __restrict__ biases, uint16_t* __restrict__ y, int64_t ldy) {
  constexpr int NT = 16 * NB, MB = 2;
  constexpr int GPC = kDenseChunk / GW;  // groups per chunk
  constexpr int SPG = GW / 4;            // k-slices per group
  __shared__ __align__(16) uint32_t xs[kDenseChunk][NT][4];  // word-major (see above)
  __shared__ float xg[NT][GPC];
  __shared__ float sb[2][kDenseRows][GPC];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int64_t t0 = static_cast<int64_t>(blockIdx.y) * NT;
  const int64_t rw0 = static_cast<int64_t>(blockIdx.x) * kDenseRows;
  const int64_t row0 = rw0 + 32 * wv;
  const int64_t n_groups = nwords / GW;
  const uint32_t* rowp[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    int64_t r = row0 + 16 * mb + r16;
    r = r < n_out ? r : n_out - 1;
    rowp[mb] = w + r * nwords + g;
  }
  f32x4d_t out[MB][NB], acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) out[mb][nb] = acc[mb][nb] = f32x4d_t{0.f, 0.f, 0.f, 0.f};
  uint32_t wq[MB][4];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int s = 0; s < 4; ++s) wq[mb][s] = rowp[mb][4 * s];
  for (int64_t c0 = 0; c0 < nwords; c0 += kDenseChunk) {
    const int64_t gb = c0 / GW;  // first group of this chunk
    // Stage x' (16 x pairs) per (token, word) and the group sums X.
    uint4 xr[NB];
#pragma unroll
    for (int it = 0; it < NB; ++it) {
      const int item = tid + 256 * it;
      const int col = item % NT, wd = item / NT;
      int64_t t = t0 + col;
      t = t < batch ? t : batch - 1;
      xr[it] = reinterpret_cast<const uint4*>(x + t * ldx + (c0 + wd) * 8)[0];
    }
    // Scales and biases of this chunk's groups for the workgroup's rows.
    float sbv[2];
    {
      const int which = tid >> 7, rr = tid & 127;
      int64_t r = rw0 + rr;
      r = r < n_out ? r : n_out - 1;
      const void* src = which ? biases : scales;
#pragma unroll
      for (int gi = 0; gi < GPC; ++gi) sbv[gi & 1] = ld_t<SDT>(src, r * n_groups + gb + gi);
    }
    uint32_t wn[MB][4];
    const int64_t cn = c0 + kDenseChunk < nwords ? c0 + kDenseChunk : c0;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int s = 0; s < 4; ++s) wn[mb][s] = rowp[mb][cn + 4 * s];
    // (no sched_barrier here: with loads into loop-carried registers just
    // above, it produced wrong MFMA operands on this compiler)
    if (tid < NT * GPC) xg[tid / GPC][tid % GPC] = 0.f;
    {
      const int which = tid >> 7, rr = tid & 127;
#pragma unroll
      for (int gi = 0; gi < GPC; ++gi) sb[which][rr][gi] = sbv[gi & 1];
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < NB; ++it) {
      const int item = tid + 256 * it;
      const int col = item % NT, wd = item / NT;
      const bool valid = t0 + col < batch;
      const uint32_t u4[4] = {xr[it].x, xr[it].y, xr[it].z, xr[it].w};
      float xv[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        xv[2 * q] = valid ? __uint_as_float(u4[q] << 16) : 0.f;
        xv[2 * q + 1] = valid ? __uint_as_float(u4[q] & 0xffff0000u) : 0.f;
      }
      float sx = 0.f;
      uint32_t pr[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pr[j] = pack_bf16x2(16.f * xv[j], 16.f * xv[j + 4]);
        sx += xv[j] + xv[j + 4];
      }
      *reinterpret_cast<uint4*>(&xs[wd][col][0]) = make_uint4(pr[0], pr[1], pr[2], pr[3]);
      atomicAdd(&xg[col][wd / GW], sx);
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 4; ++s) {  // k-slice s: words 4s .. 4s+3 of the chunk
      uint4 a[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const uint32_t wd = wq[mb][s];
        a[mb] = make_uint4(and_or(wd << 3, kMaskQ4d, kOneBf16x2), and_or(wd >> 1, kMaskQ4d, kOneBf16x2),
                           and_or(wd >> 5, kMaskQ4d, kOneBf16x2), and_or(wd >> 9, kMaskQ4d, kOneBf16x2));
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const uint4 b = *reinterpret_cast<const uint4*>(&xs[4 * s + g][nb * 16 + r16][0]);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[mb][nb] = mfma16(a[mb], b, acc[mb][nb]);
      }
      if ((s + 1) % SPG == 0) {  // end of an RTN group: fold and clear
        const int gi = s / SPG;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const float X = xg[nb * 16 + r16][gi];
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int rr = 32 * wv + 16 * mb + 4 * g + i;
              out[mb][nb][i] += sb[0][rr][gi] * (acc[mb][nb][i] - 16.f * X) + sb[1][rr][gi] * X;
            }
            acc[mb][nb] = f32x4d_t{0.f, 0.f, 0.f, 0.f};
          }
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int s = 0; s < 4; ++s) wq[mb][s] = wn[mb][s];
  }
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int64_t t = t0 + nb * 16 + r16;
    if (t >= batch) continue;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int64_t n0 = row0 + 16 * mb + 4 * g;
      if (n0 + 3 < n_out && (ldy % 4) == 0) {
        uint2 r;
        r.x = pack_bf16x2_rn(out[mb][nb][0], out[mb][nb][1]);
        r.y = pack_bf16x2_rn(out[mb][nb][2], out[mb][nb][3]);
        *reinterpret_cast<uint2*>(y + t * ldy + n0) = r;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (n0 + i < n_out) y[t * ldy + n0 + i] = f32_to_bf16(out[mb][nb][i]);
      }
    }
  }
}

}  // namespace ma

using namespace ma;

// Launchers used by ternary_gemv.hip / rtn4.hip for batch >= 5 (bf16 x,
// [N, K/16] or [N, K/8] codes, nwords % 16 == 0, 16-byte aligned rows).
int launch_tgemm_mfma(const uint16_t* x, int64_t batch, int64_t ldx, const uint32_t* w,
                      int64_t n_out, int64_t nwords, const void* alpha, int alpha_dt,
                      const void* rms_w, int rms_dt, float rms_eps, uint16_t* y, int64_t ldy,
                      hipStream_t s) {
  const int nb = batch <= 16 ? 1 : 2;
  const int64_t nt = 16 * nb;
  // 64-row tiles (one 16-row block per wave): more workgroups for the
  // decoder's 2048-2560-row projections.
  dim3 grid(static_cast<unsigned>(cdiv(n_out, 64)), static_cast<unsigned>(cdiv(batch, nt)));
#define MA_TG(NB, RMS, ADT)                                                                      \
  hipLaunchKernelGGL((k_tgemm_mfma<NB, 1, RMS, ADT>), grid, dim3(256), 0, s, x, batch, ldx, w, \
                     n_out, nwords, alpha, rms_w, rms_dt, rms_eps, y, ldy)
#define MA_TG_A(NB, RMS) \
  if (alpha_dt == MA_F32) MA_TG(NB, RMS, MA_F32); else MA_TG(NB, RMS, MA_BF16);
#define MA_TG_R(NB) \
  if (rms_w) { MA_TG_A(NB, true) } else { MA_TG_A(NB, false) }
  if (nb == 1) { MA_TG_R(1) } else { MA_TG_R(2) }
#undef MA_TG_R
#undef MA_TG_A
#undef MA_TG
  return check_launch("ternary_gemv (mfma)");
}

int launch_rtn4_mfma(const uint16_t* x, int64_t batch, int64_t ldx, const uint32_t* w,
                     int64_t n_out, int64_t nwords, int64_t group, const void* scales,
                     const void* biases, int s_dt, uint16_t* y, int64_t ldy, hipStream_t s) {
  const int nb = batch <= 16 ? 1 : 2;
  const int64_t nt = 16 * nb;
  dim3 grid(static_cast<unsigned>(cdiv(n_out, kDenseRows)), static_cast<unsigned>(cdiv(batch, nt)));
#define MA_RT(NB, GW, SDT)                                                                   \
  hipLaunchKernelGGL((k_rtn4_mfma<NB, GW, SDT>), grid, dim3(256), 0, s, x, batch, ldx, w, \
                     n_out, nwords, scales, biases, y, ldy)
#define MA_RT_S(NB, GW) \
  if (s_dt == MA_F32) MA_RT(NB, GW, MA_F32); else MA_RT(NB, GW, MA_BF16);
#define MA_RT_G(NB) \
  if (group == 64) { MA_RT_S(NB, 8) } else { MA_RT_S(NB, 16) }
  if (nb == 1) { MA_RT_G(1) } else { MA_RT_G(2) }
#undef MA_RT_G
#undef MA_RT_S
#undef MA_RT
  return check_launch("rtn4_gemv (mfma)");
}
