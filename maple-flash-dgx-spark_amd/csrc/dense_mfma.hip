// Batched dense GEMMs on MFMA for the decode step at batch > 4 (gfx950):
// the packed ternary projection (reference _ternary_gemm_kernel,
// src/maple_run/kernels/ternary_gemv.py:156-258, with the optional fused input
// RMSNorm kept as the x_hi + x_lo bf16 split of :241-248) and the 4-bit RTN
// lm_head (_rtn4_gemm_kernel, src/maple_run/kernels/rtn4.py:170-282, in the
// factored per-group form s_g (q.x)_g + b_g sum_g x of :197-208).
//
// v_mfma_f32_16x16x32_bf16 layouts (checked on the device): A lane l holds row
// l%16, k 8(l/16)..+8; B col l%16, k 8(l/16)..+8; C col l%16, rows 4(l/16)..+4.
//
// Ternary: a lane expands one 16-code word into 8 bf16x2 dwords of 1 + c/f
// (expand_word) = two MFMA k-slices; B holds the matching x' = f x pairs, so C
// accumulates sum (f + c) x and y = alpha (C - sum (f + 1) x).  A workgroup
// takes 16 rows and 16 (or 32) tokens with K split over its 8 waves, one
// 16-word chunk per wave at K = 2048, and the partial tiles are added in wave
// order; decode projections have few rows, and a K walk per workgroup left
// most of the chip idle.  With the RMSNorm folded in, from 17 tokens the x'
// operands are built once per token by a first launch into a workspace.
// RTN4: a word's 8 codes expand to 4 dwords of 1 + q/16 = one k-slice against
// x' = 16 x pairs staged in LDS; after each RTN group C is folded into the
// output as s_g (C - 16 X_g) + b_g X_g (X_g = sum of x over the group) and
// cleared.
#include "mfma.h"

namespace ma {

constexpr int kDenseChunk = 16;  // words of K per step
constexpr int kDenseRows = 128;  // rows per workgroup (4 waves x 2 x 16)
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

// ---------------------------------------------------------------------------
// Two-launch form of the RMS-folded ternary GEMM.  k_xprep builds, once per
// token, what the GEMM's B operands are made of -- the x' pairs of the hi and
// lo bf16 halves of x * w_rms, the token's correction sum (f + 1) x and its
// scale rsqrt(mean(x^2) + eps) -- in the GEMM's layout, so that k_tgemm_xpk
// reads them instead of every row tile rebuilding them from x:
//   xp [tile][v][word][half][NT] uint4 (v: hi, lo);  xc [tile * NT + col] = (c, scale)
// Tokens past the batch are zero.  Per word the arithmetic is the one-launch
// GEMM's; the per-token sums add up in another order.
// With a MoE combine in front (cb.slot_out set), x is not read: each word of
// token t is first built as the grouped MoE's combine builds it (k_combine8:
// sum_j w[t, j] * slot_out[inverse[t, j]] in slot order, + residual, rounded
// to bf16), stored to cb.x_out, and then prepared as above.
// ---------------------------------------------------------------------------
constexpr int kXpTile = 32;  // tokens per tile of the two-launch form


__global__ __launch_bounds__(128) void k_xprep(const uint16_t* __restrict__ x, int64_t batch,
                                               int64_t ldx, int64_t nwords,
                                               const void* __restrict__ rms_w, int rms_dt,
                                               float rms_eps, int nt, uint4* __restrict__ xp,
                                               float2* __restrict__ xc, CombineIn cb) {
  __shared__ float red_c[2], red_s[2];
  const int64_t t = blockIdx.x;
  const int64_t tile = t / nt, col = t % nt;
  const int tid = threadIdx.x;
  const bool valid = t < batch;
  float c = 0.f, ss = 0.f;
  // (the combine's arguments read at once: left to itself the compiler read
  // them in two dependent rounds)
  asm volatile("" ::"s"(cb.slot_out), "s"(cb.inverse), "s"(cb.wts), "s"(cb.topk), "s"(cb.res), "s"(cb.x_out));
  // the combine's (row, weight) pairs of this token
  int64_t crow[8];
  float cw[8];
  if (cb.slot_out && valid) slot_pairs8(cb.inverse, cb.wts, t, cb.topk, crow, cw);
  for (int64_t wd = tid; wd < nwords; wd += 128) {
    float v[16];
    if (valid && cb.slot_out) {
      const int64_t n = nwords * 16;
      uint4 sv[8][2], r[2] = {make_uint4(0u, 0u, 0u, 0u), make_uint4(0u, 0u, 0u, 0u)};
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j < cb.topk) {
          const uint4* src = reinterpret_cast<const uint4*>(cb.slot_out + crow[j] * n + wd * 16);
          sv[j][0] = src[0];
          sv[j][1] = src[1];
        }
      if (cb.res) {
        const uint4* src = reinterpret_cast<const uint4*>(cb.res + t * n + wd * 16);
        r[0] = src[0];
        r[1] = src[1];
      }
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        float a[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (j >= cb.topk) break;
          const uint32_t u[4] = {sv[j][hf].x, sv[j][hf].y, sv[j][hf].z, sv[j][hf].w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            a[2 * q] += cw[j] * __uint_as_float(u[q] << 16);
            a[2 * q + 1] += cw[j] * __uint_as_float(u[q] & 0xffff0000u);
          }
        }
        if (cb.res) {
          const uint32_t u[4] = {r[hf].x, r[hf].y, r[hf].z, r[hf].w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            a[2 * q] += __uint_as_float(u[q] << 16);
            a[2 * q + 1] += __uint_as_float(u[q] & 0xffff0000u);
          }
        }
        uint4 o;
        o.x = pack_bf16x2_rn(a[0], a[1]);
        o.y = pack_bf16x2_rn(a[2], a[3]);
        o.z = pack_bf16x2_rn(a[4], a[5]);
        o.w = pack_bf16x2_rn(a[6], a[7]);
        reinterpret_cast<uint4*>(cb.x_out + t * n + wd * 16)[hf] = o;
        const uint32_t ou[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          v[8 * hf + 2 * q] = __uint_as_float(ou[q] << 16);
          v[8 * hf + 2 * q + 1] = __uint_as_float(ou[q] & 0xffff0000u);
        }
      }
    } else if (valid) {
      const uint4* src = reinterpret_cast<const uint4*>(x + t * ldx + wd * 16);
      const uint4 a = src[0], b = src[1];
      const uint32_t u[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        v[2 * q] = __uint_as_float(u[q] << 16);
        v[2 * q + 1] = __uint_as_float(u[q] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int q = 0; q < 16; ++q) v[q] = 0.f;
    }
    float r[16], hi[16], lo[16];
    load_rms16(rms_w, rms_dt, wd, r);
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      ss += v[q] * v[q];
      const float xh = v[q] * r[q];
      hi[q] = bf16_to_f32(f32_to_bf16(xh));
      lo[q] = bf16_to_f32(f32_to_bf16(xh - hi[q]));
    }
    uint32_t pr[8];
    uint4* dst = xp + ((tile * 2 * nwords + wd) * 2) * nt + col;  // v = hi, half 0
    const int64_t vstride = nwords * 2 * nt;
    c += prep_word_pairs(hi, pr);
    dst[0] = make_uint4(pr[0], pr[1], pr[2], pr[3]);
    dst[nt] = make_uint4(pr[4], pr[5], pr[6], pr[7]);
    c += prep_word_pairs(lo, pr);
    dst[vstride] = make_uint4(pr[0], pr[1], pr[2], pr[3]);
    dst[vstride + nt] = make_uint4(pr[4], pr[5], pr[6], pr[7]);
  }
  // fixed order: a butterfly within each wave, then wave 0's sum + wave 1's
  // (a serial pass over the 128 partials by one thread took ~0.4 us)
  c = group_sum<64>(c);
  ss = group_sum<64>(ss);
  if ((tid & 63) == 0) {
    red_c[tid >> 6] = c;
    red_s[tid >> 6] = ss;
  }
  __syncthreads();
  if (tid == 0)
    xc[t] = make_float2(red_c[0] + red_c[1],
                        rsqrtf((red_s[0] + red_s[1]) / static_cast<float>(nwords * 16) + rms_eps));
}

// K split over the waves of a workgroup: 16 rows x NT = 16 NB tokens per
// workgroup, wave w takes chunks w, w + KW, ... and reads its B operands
// straight from xp (each fragment is one 256-byte run per 16 lanes); the KW
// partial tiles are summed in wave order through LDS before the epilogue.
template <int NB, int NV, int ADT, int KW>
__global__ __launch_bounds__(64 * KW) void k_tgemm_xpk(const uint4* __restrict__ xp,
                                                       const float2* __restrict__ xc,
                                                       int64_t batch, const uint32_t* __restrict__ w,
                                                       int64_t n_out, int64_t nwords,
                                                       const void* __restrict__ alpha,
                                                       uint16_t* __restrict__ y, int64_t ldy) {
  constexpr int NT = 16 * NB;
  constexpr int NBF = 4 * 2 * NV * NB;  // B fragments per lane per chunk
  __shared__ float red[KW][NB][4][64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int64_t tile = blockIdx.y;
  const int64_t t0 = tile * NT;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * 16;
  int64_t r = row0 + r16;
  r = r < n_out ? r : n_out - 1;
  const uint32_t* rowp = w + r * nwords + 4 * g;
  const u32x4v_t* tb = reinterpret_cast<const u32x4v_t*>(xp) + tile * NV * nwords * 2 * NT;
  f32x4d_t acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x4d_t{0.f, 0.f, 0.f, 0.f};
  const ExpandConsts kc;
  for (int64_t c0 = 16 * wv; c0 < nwords; c0 += 16 * KW) {
    const uint4 wq = *reinterpret_cast<const uint4*>(rowp + c0);
    u32x4v_t bf[NBF];  // [q][hf][vv][nb]
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int vv = 0; vv < NV; ++vv)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            bf[((q * 2 + hf) * NV + vv) * NB + nb] =
                tb[((vv * nwords + c0 + 4 * g + q) * 2 + hf) * NT + nb * 16 + r16];
    // every load of the chunk in flight before the first MFMA (one round trip)
    __builtin_amdgcn_sched_barrier(0);
    u32x4v_t av[4][2];  // A operands of the lane's 4 words, all built before the MFMAs
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t wsel = q == 0 ? wq.x : q == 1 ? wq.y : q == 2 ? wq.z : wq.w;
      uint32_t ex[8];
      expand_word(wsel, ex, kc);
      av[q][0] = u32x4v_t{ex[0], ex[1], ex[2], ex[3]};
      av[q][1] = u32x4v_t{ex[4], ex[5], ex[6], ex[7]};
    }
    mfma_block_begin();
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int vv = 0; vv < NV; ++vv)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            mfma_acc(acc[nb], av[q][hf], bf[((q * 2 + hf) * NV + vv) * NB + nb]);
    mfma_block_end();
    keep_operands(av, bf, acc);
  }
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wv][nb][i][lane] = acc[nb][i];
  __syncthreads();
  // Thread e < 4 NT: token col e % NT, rows 4 (e / NT) .. +3 of the tile.
  const int e = tid;
  if (e >= 4 * NT) return;
  const int col = e % NT, rq = e / NT;
  const int64_t t = t0 + col;
  if (t >= batch) return;
  const int nb = col / 16, ln = (col % 16) + 16 * rq;  // acc lane holding rows 4 rq ..
  const float2 cs = xc[t];
  const int64_t n0 = row0 + 4 * rq;
  float o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < KW; ++k) s += red[k][nb][i][ln];
    const int64_t n = n0 + i < n_out ? n0 + i : n_out - 1;
    o[i] = ld_t<ADT>(alpha, n) * (s - cs.x) * cs.y;
  }
  if (n0 + 3 < n_out && (ldy % 4) == 0) {
    uint2 rr;
    rr.x = pack_bf16x2_rn(o[0], o[1]);
    rr.y = pack_bf16x2_rn(o[2], o[3]);
    *reinterpret_cast<uint2*>(y + t * ldy + n0) = rr;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (n0 + i < n_out) y[t * ldy + n0 + i] = f32_to_bf16(o[i]);
  }
}

// One-launch K-split form: 16 rows x NT = 16 NB tokens per workgroup, wave w
// takes chunks w, w + KW, ...  A lane's B fragments are the x' pairs of words
// 4g + q of its own token column, so it builds them from x in registers (no
// LDS staging, no workspace), with that word's correction and squares; the
// KW partial tiles and the per-token sums are added in a fixed order through
// LDS.  RDT: -1 without the RMSNorm, else the dtype of w_rms.
template <int NB, int RDT, int ADT, int KW>
__global__ __launch_bounds__(64 * KW) void k_tgemm_ks(
    const uint16_t* __restrict__ x, int64_t batch, int64_t ldx, const uint32_t* __restrict__ w,
    int64_t n_out, int64_t nwords, const void* __restrict__ alpha, const void* __restrict__ rms_w,
    float rms_eps, uint16_t* __restrict__ y, int64_t ldy) {
  constexpr int NT = 16 * NB;
  constexpr bool RMS = RDT >= 0;
  constexpr int NV = RMS ? 2 : 1;
  __shared__ float red[KW][NB][4][64];
  __shared__ float red_c[KW][4][NT], red_s[KW][4][NT];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int64_t t0 = static_cast<int64_t>(blockIdx.y) * NT;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * 16;
  int64_t r = row0 + r16;
  r = r < n_out ? r : n_out - 1;
  const uint32_t* rowp = w + r * nwords + 4 * g;
  const uint16_t* xrow[NB];
  bool valid[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int64_t t = t0 + nb * 16 + r16;
    valid[nb] = t < batch;
    xrow[nb] = x + (valid[nb] ? t : batch - 1) * ldx + 64 * g;  // word 4g of chunk 0
  }
  f32x4d_t acc[NB];
  float cp[NB], sp[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    acc[nb] = f32x4d_t{0.f, 0.f, 0.f, 0.f};
    cp[nb] = sp[nb] = 0.f;
  }
  const ExpandConsts kc;
  constexpr int RV = RDT == MA_F32 ? 16 : 8;  // uint4 of w_rms per lane per chunk
  for (int64_t c0 = 16 * wv; c0 < nwords; c0 += 16 * KW) {
    const uint4 wq = *reinterpret_cast<const uint4*>(rowp + c0);
    u32x4v_t xv[4][NB][2];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const u32x4v_t* src = reinterpret_cast<const u32x4v_t*>(xrow[nb] + (c0 + q) * 16);
        xv[q][nb][0] = src[0];
        xv[q][nb][1] = src[1];
      }
    u32x4v_t rv[RMS ? RV : 1];
    if constexpr (RMS) {
      const u32x4v_t* src = reinterpret_cast<const u32x4v_t*>(
          static_cast<const char*>(rms_w) + (c0 + 4 * g) * 16 * (RDT == MA_F32 ? 4 : 2));
#pragma unroll
      for (int i = 0; i < RV; ++i) rv[i] = src[i];
    }
    // every load of the chunk in flight before the first use (one round trip)
    __builtin_amdgcn_sched_barrier(0);
    // Two words per step: their A and B operands are all built (VALU) before
    // the step's MFMAs issue, and stay live until the MFMAs' results exist, so
    // no operand register is rewritten while an MFMA may still read it.
#pragma unroll
    for (int qh = 0; qh < 4; qh += 2) {
      u32x4v_t av[2][2];             // [word][half]
      u32x4v_t bv[2][NB][NV][2];     // [word][token block][hi/lo][half]
#pragma unroll
      for (int qi = 0; qi < 2; ++qi) {
        const int q = qh + qi;
        const uint32_t wsel = q == 0 ? wq.x : q == 1 ? wq.y : q == 2 ? wq.z : wq.w;
        uint32_t ex[8];
        expand_word(wsel, ex, kc);
        av[qi][0] = u32x4v_t{ex[0], ex[1], ex[2], ex[3]};
        av[qi][1] = u32x4v_t{ex[4], ex[5], ex[6], ex[7]};
        float rr[16];
        if constexpr (RMS) {
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            if constexpr (RDT == MA_F32) {
              rr[j] = __uint_as_float(rv[4 * q + j / 4][j % 4]);
            } else {
              const uint32_t u = rv[2 * q + j / 8][(j % 8) / 2];
              rr[j] = __uint_as_float((j & 1) ? (u & 0xffff0000u) : (u << 16));
            }
          }
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          float v[16];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const uint32_t u = xv[q][nb][j / 4][j % 4];
            v[2 * j] = valid[nb] ? __uint_as_float(u << 16) : 0.f;
            v[2 * j + 1] = valid[nb] ? __uint_as_float(u & 0xffff0000u) : 0.f;
          }
          uint32_t pr[8];
          if constexpr (RMS) {
            float hi[16], lo[16], ss = 0.f;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
              ss += v[j] * v[j];
              const float xh = v[j] * rr[j];
              hi[j] = bf16_to_f32(f32_to_bf16(xh));
              lo[j] = bf16_to_f32(f32_to_bf16(xh - hi[j]));
            }
            sp[nb] += ss;
            float c = prep_word_pairs(hi, pr);
            bv[qi][nb][0][0] = u32x4v_t{pr[0], pr[1], pr[2], pr[3]};
            bv[qi][nb][0][1] = u32x4v_t{pr[4], pr[5], pr[6], pr[7]};
            c += prep_word_pairs(lo, pr);
            bv[qi][nb][NV - 1][0] = u32x4v_t{pr[0], pr[1], pr[2], pr[3]};
            bv[qi][nb][NV - 1][1] = u32x4v_t{pr[4], pr[5], pr[6], pr[7]};
            cp[nb] += c;
          } else {
            cp[nb] += prep_word_pairs(v, pr);
            bv[qi][nb][0][0] = u32x4v_t{pr[0], pr[1], pr[2], pr[3]};
            bv[qi][nb][0][1] = u32x4v_t{pr[4], pr[5], pr[6], pr[7]};
          }
        }
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        pin(cp[nb]);
        pin(sp[nb]);
      }
      mfma_block_begin();
#pragma unroll
      for (int qi = 0; qi < 2; ++qi)
#pragma unroll
        for (int vv = 0; vv < NV; ++vv)
#pragma unroll
          for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
              mfma_acc(acc[nb], av[qi][hf], bv[qi][nb][vv][hf]);
      mfma_block_end();
      keep_operands(av, bv, acc);
    }
  }
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wv][nb][i][lane] = acc[nb][i];
    red_c[wv][g][nb * 16 + r16] = cp[nb];  // this lane's (g, token) share
    red_s[wv][g][nb * 16 + r16] = sp[nb];
  }
  __syncthreads();
  // Thread e < 4 NT: token col e % NT, rows 4 (e / NT) .. +3 of the tile.
  const int e = tid;
  if (e >= 4 * NT) return;
  const int col = e % NT, rq = e / NT;
  const int64_t t = t0 + col;
  if (t >= batch) return;
  const int nb = col / 16, ln = (col % 16) + 16 * rq;  // acc lane holding rows 4 rq ..
  float cc = 0.f, ss = 0.f;
#pragma unroll
  for (int k = 0; k < KW; ++k)
#pragma unroll
    for (int gg = 0; gg < 4; ++gg) {
      cc += red_c[k][gg][col];
      ss += red_s[k][gg][col];
    }
  const float scale = RMS ? rsqrtf(ss / static_cast<float>(nwords * 16) + rms_eps) : 1.f;
  const int64_t n0 = row0 + 4 * rq;
  float o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < KW; ++k) s += red[k][nb][i][ln];
    const int64_t n = n0 + i < n_out ? n0 + i : n_out - 1;
    o[i] = ld_t<ADT>(alpha, n) * (s - cc) * scale;
  }
  if (n0 + 3 < n_out && (ldy % 4) == 0) {
    uint2 rr;
    rr.x = pack_bf16x2_rn(o[0], o[1]);
    rr.y = pack_bf16x2_rn(o[2], o[3]);
    *reinterpret_cast<uint2*>(y + t * ldy + n0) = rr;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (n0 + i < n_out) y[t * ldy + n0 + i] = f32_to_bf16(o[i]);
  }
}

// ---------------------------------------------------------------------------
// RTN4: y[t, n] = sum_g s[n,g] (sum_{k in g} q x) + b[n,g] sum_{k in g} x.
// GW = words per RTN group (8: group 64, 16: group 128).  Lane group g loads
// its words of a chunk with vector loads (one 16-byte load of words 4g ..
// 4g+3 for GW = 16; two 8-byte loads of words 2g, 2g+1 and 8+2g, 9+2g for
// GW = 8), and k-slice s takes word chunk_word(g, s) of each lane group, so
// that every k-slice lies in one RTN group.
// ---------------------------------------------------------------------------
template <int GW>
__device__ __forceinline__ int chunk_word(int g, int s) {
  if constexpr (GW == 16) return 4 * g + s;
  else return s < 2 ? 2 * g + s : 8 + 2 * g + (s - 2);
}

template <int GW>
__device__ __forceinline__ void load_chunk_words(const uint32_t* p, uint32_t (&q)[4]) {
  if constexpr (GW == 16) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    q[0] = v.x, q[1] = v.y, q[2] = v.z, q[3] = v.w;
  } else {
    const uint2 a = *reinterpret_cast<const uint2*>(p), b = *reinterpret_cast<const uint2*>(p + 8);
    q[0] = a.x, q[1] = a.y, q[2] = b.x, q[3] = b.y;
  }
}

template <int NB, int GW, int SDT>
__global__ __launch_bounds__(256) void k_rtn4_mfma(
    const uint16_t* __restrict__ x, int64_t batch, int64_t ldx, const uint32_t* __restrict__ w,
    int64_t n_out, int64_t nwords, const void* __restrict__ scales,
    const void* __restrict__ biases, uint16_t* __restrict__ y, int64_t ldy) {
  constexpr int NT = 16 * NB, MB = 2;
  constexpr int GPC = kDenseChunk / GW;  // groups per chunk
  constexpr int SPG = GW / 4;            // k-slices per group
  __shared__ __align__(16) uint32_t xs[kDenseChunk][NT][4];  // word-major (see above)
  __shared__ float xw[kDenseChunk][NT];  // each word's sum of x, added per group in word order
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
    rowp[mb] = w + r * nwords + (GW == 16 ? 4 * g : 2 * g);
  }
  f32x4d_t out[MB][NB], acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) out[mb][nb] = acc[mb][nb] = f32x4d_t{0.f, 0.f, 0.f, 0.f};
  uint32_t wq[MB][4];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) load_chunk_words<GW>(rowp[mb], wq[mb]);
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
    for (int mb = 0; mb < MB; ++mb) load_chunk_words<GW>(rowp[mb] + cn, wn[mb]);
    // (no sched_barrier here: with loads into loop-carried registers just
    // above, it produced wrong MFMA operands on this compiler)
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
      xw[wd][col] = sx;
    }
    __syncthreads();
    if (tid < NT * GPC) {  // group sums in a fixed order: the same bits on every run
      const int col = tid / GPC, gi = tid % GPC;
      float sx = 0.f;
#pragma unroll
      for (int wd = 0; wd < GW; ++wd) sx += xw[gi * GW + wd][col];
      xg[col][gi] = sx;
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 4; ++s) {  // k-slice s: word chunk_word(g, s) of lane group g
      // operands first, then one block of in-place MFMAs (the hand-spaced
      // discipline of mfma.h: compiler-scheduled chains here gave wrong sums
      // for some instantiations)
      u32x4v_t av[MB], bv[NB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const uint32_t wd = wq[mb][s];
        av[mb] = u32x4v_t{and_or(wd << 3, kMaskQ4d, kOneBf16x2), and_or(wd >> 1, kMaskQ4d, kOneBf16x2),
                          and_or(wd >> 5, kMaskQ4d, kOneBf16x2), and_or(wd >> 9, kMaskQ4d, kOneBf16x2)};
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        bv[nb] = *reinterpret_cast<const u32x4v_t*>(&xs[chunk_word<GW>(g, s)][nb * 16 + r16][0]);
      mfma_block_begin();
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) mfma_acc(acc[mb][nb], av[mb], bv[nb]);
      mfma_block_end();
      keep_b(av, acc[0]);
      keep_b(bv, acc[0]);
      if ((s + 1) % SPG == 0) {  // end of an RTN group: fold and clear
        const int gi = s / SPG;
        // s (acc - 16 X) + b X = s acc + (b - 16 s) X: two FMAs per output
        float sr[MB][4], br[MB][4];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int rr = 32 * wv + 16 * mb + 4 * g + i;
            sr[mb][i] = sb[0][rr][gi];
            br[mb][i] = sb[1][rr][gi] - 16.f * sr[mb][i];
          }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const float X = xg[nb * 16 + r16][gi];
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
            for (int i = 0; i < 4; ++i)  // explicit FMAs: every build rounds the fold alike
              out[mb][nb][i] = __builtin_fmaf(sr[mb][i], acc[mb][nb][i], __builtin_fmaf(br[mb][i], X, out[mb][nb][i]));
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

// ---------------------------------------------------------------------------
// RTN4 with a workspace: the x' operands and group sums of every token tile
// are built once (k_rtn4_xprep), then each workgroup of k_rtn4_mfma_dma copies
// chunk c + 1's x' and group sums into LDS with the LDS DMA while chunk c
// multiplies: no staging arithmetic or registers in the K loop, one barrier
// per chunk, and every load of the loop issued a chunk ahead.  Same per-word
// arithmetic and fixed-order sums as k_rtn4_mfma (the group sums are added in
// word order by the prep launch), so the two give the same bits.
// ---------------------------------------------------------------------------
// Workspace: per token tile and chunk, the x' words in k_rtn4_mfma's LDS
// layout [word][token][4 u32] (NT x 256 B), then the group sums [token][GPC].
size_t rtn4_ws_bytes(int64_t batch, int64_t nwords, int64_t group) {
  const int64_t nt = batch <= 16 ? 16 : 32, tiles = cdiv(batch, nt), chunks = nwords / kDenseChunk;
  const int64_t gpc = kDenseChunk / (group / 8);
  return static_cast<size_t>(tiles * chunks * nt) * (kDenseChunk * 16 + gpc * 4);
}

template <int NB, int GW>
__global__ __launch_bounds__(256) void k_rtn4_xprep(const uint16_t* __restrict__ x, int64_t batch, int64_t ldx,
                                                    int64_t nwords, uint4* __restrict__ xq, float* __restrict__ xgs) {
  constexpr int NT = 16 * NB, GPC = kDenseChunk / GW;
  __shared__ float xw[kDenseChunk][NT];
  const int tid = threadIdx.x;
  const int64_t tile = blockIdx.x, c = blockIdx.y, nch = nwords / kDenseChunk;
  const int64_t t0 = tile * NT, c0 = c * kDenseChunk;
  uint4* const dst = xq + (tile * nch + c) * (kDenseChunk * NT);
#pragma unroll
  for (int it = 0; it < NB; ++it) {
    const int item = tid + 256 * it;
    const int col = item % NT, wd = item / NT;
    const bool valid = t0 + col < batch;
    const int64_t t = valid ? t0 + col : batch - 1;
    const uint4 xr = reinterpret_cast<const uint4*>(x + t * ldx + (c0 + wd) * 8)[0];
    const uint32_t u4[4] = {xr.x, xr.y, xr.z, xr.w};
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
    dst[wd * NT + col] = make_uint4(pr[0], pr[1], pr[2], pr[3]);
    xw[wd][col] = sx;
  }
  __syncthreads();
  if (tid < NT * GPC) {  // group sums in word order (as k_rtn4_mfma adds them)
    const int col = tid / GPC, gi = tid % GPC;
    float sx = 0.f;
#pragma unroll
    for (int wd = 0; wd < GW; ++wd) sx += xw[gi * GW + wd][col];
    xgs[(tile * nch + c) * (NT * GPC) + tid] = sx;
  }
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;
// s_waitcnt immediate (gfx9 encoding): vmcnt(n), expcnt and lgkmcnt left open.
constexpr int vmcnt_only(int n) { return (n & 0xF) | (0x7 << 4) | (0xF << 8) | ((n >> 4) << 14); }

// One chunk of k_rtn4_mfma_dma: issue chunk c + 1's copies (x' into xn, the
// group sums into gn), its scales / biases and its weights, then chunk c's
// MFMAs and folds on xc / gc / sbc, then wait for the copies and the scales,
// stage the scales into sbn, and meet at the barrier.
template <int NB, int GW, int SDT>
__device__ __forceinline__ void rtn4_dma_chunk(
    const uint32_t* rp, int64_t moff1, int64_t c0, int64_t nwords, const uint4* __restrict__ xq_t,
    const float* __restrict__ xg_t, const void* __restrict__ scales, const void* __restrict__ biases,
    int64_t rw0, int64_t n_out, int64_t n_groups, const uint32_t* xc, const float* gc, uint32_t* xn, float* gn,
    float (*sbc)[kDenseRows][kDenseChunk / GW], float (*sbn)[kDenseRows][kDenseChunk / GW],
    uint32_t (&wq)[2][4], f32x4d_t (&out)[2][NB], f32x4d_t (&acc)[2][NB]) {
  constexpr int NT = 16 * NB, MB = 2, GPC = kDenseChunk / GW, SPG = GW / 4;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const bool more = c0 + kDenseChunk < nwords;
  const int64_t cn = more ? c0 + kDenseChunk : c0, chn = cn / kDenseChunk;
  // this chunk's weights (loaded during the last one) are in, nothing else is outstanding
  __builtin_amdgcn_s_waitcnt(0);
  MA_ISSUE_FENCE();
  if (more) {
#pragma unroll
    for (int i = 0; i < NB; ++i)  // x': NT * 16 slots of 16 bytes, in order
      __builtin_amdgcn_global_load_lds(xq_t + chn * (kDenseChunk * NT) + tid + 256 * i,
                                       (lds_ptr_t)(xn + 4 * (64 * wv + 256 * i)), 16, 0, 0);
    if (wv == 0 && lane < NT * GPC)  // group sums: NT * GPC floats
      __builtin_amdgcn_global_load_lds(xg_t + chn * (NT * GPC) + lane, (lds_ptr_t)gn, 4, 0, 0);
  }
  float sbv[2];
  {
    const int which = tid >> 7, rr = tid & 127;
    int64_t r = rw0 + rr;
    r = r < n_out ? r : n_out - 1;
    const void* src = which ? biases : scales;
#pragma unroll
    for (int gi = 0; gi < GPC; ++gi) sbv[gi & 1] = ld_t<SDT>(src, r * n_groups + cn / GW + gi);
  }
  MA_ISSUE_FENCE();  // the weights are issued last
  uint32_t wn[MB][4];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) load_chunk_words<GW>(rp + mb * moff1 + cn, wn[mb]);
  MA_ISSUE_FENCE();
#pragma unroll
  for (int s = 0; s < 4; ++s) {  // k-slice s: word chunk_word(g, s) of lane group g
    u32x4v_t av[MB], bv[NB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const uint32_t wd = wq[mb][s];
      av[mb] = u32x4v_t{and_or(wd << 3, kMaskQ4d, kOneBf16x2), and_or(wd >> 1, kMaskQ4d, kOneBf16x2),
                        and_or(wd >> 5, kMaskQ4d, kOneBf16x2), and_or(wd >> 9, kMaskQ4d, kOneBf16x2)};
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      bv[nb] = *reinterpret_cast<const u32x4v_t*>(xc + (chunk_word<GW>(g, s) * NT + nb * 16 + r16) * 4);
    mfma_block_begin();
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) mfma_acc(acc[mb][nb], av[mb], bv[nb]);
    mfma_block_end();
    keep_b(av, acc[0]);
    keep_b(bv, acc[0]);
    if ((s + 1) % SPG == 0) {  // end of an RTN group: s acc + (b - 16 s) X, then clear
      const int gi = s / SPG;
      float sr[MB][4], br[MB][4];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int rr = 32 * wv + 16 * mb + 4 * g + i;
          sr[mb][i] = sbc[0][rr][gi];
          br[mb][i] = sbc[1][rr][gi] - 16.f * sr[mb][i];
        }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const float X = gc[(nb * 16 + r16) * GPC + gi];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
          for (int i = 0; i < 4; ++i)  // the FMAs of k_rtn4_mfma, in its order
            out[mb][nb][i] = __builtin_fmaf(sr[mb][i], acc[mb][nb][i], __builtin_fmaf(br[mb][i], X, out[mb][nb][i]));
          acc[mb][nb] = f32x4d_t{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
  }
  // the copies and the scales have landed (the weights, issued after them, may not have)
  __builtin_amdgcn_s_waitcnt(vmcnt_only(MB * (GW == 16 ? 1 : 2)));
  {
    const int which = tid >> 7, rr = tid & 127;
#pragma unroll
    for (int gi = 0; gi < GPC; ++gi) sbn[which][rr][gi] = sbv[gi & 1];
  }
  __syncthreads();
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int q = 0; q < 4; ++q) wq[mb][q] = wn[mb][q];
}

template <int NB, int GW, int SDT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(5, 8))) void k_rtn4_mfma_dma(
    const uint4* __restrict__ xq, const float* __restrict__ xgs, int64_t batch, const uint32_t* __restrict__ w,
    int64_t n_out, int64_t nwords, const void* __restrict__ scales, const void* __restrict__ biases,
    uint16_t* __restrict__ y, int64_t ldy) {
  constexpr int NT = 16 * NB, MB = 2, GPC = kDenseChunk / GW;
  // two copies of each buffer, distinct arrays (the compiler then sees that a
  // chunk's LDS reads and the copies in flight into the other do not overlap)
  __shared__ __align__(16) uint32_t xa[kDenseChunk * NT * 4], xb[kDenseChunk * NT * 4];
  __shared__ __align__(16) float ga[NT * GPC], gb[NT * GPC];
  __shared__ float sb[2][2][kDenseRows][GPC];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int64_t tile = blockIdx.y, t0 = tile * NT;
  const int64_t rw0 = static_cast<int64_t>(blockIdx.x) * kDenseRows;
  const int64_t row0 = rw0 + 32 * wv;
  const int64_t n_groups = nwords / GW, nch = nwords / kDenseChunk;
  const uint4* const xq_t = xq + tile * nch * (kDenseChunk * NT);
  const float* const xg_t = xgs + tile * nch * (NT * GPC);
  // the lane's row of block 0, and block 1's 16 rows further (n_out % 32 ==
  // 0, so a wave's 32 rows are all in or all past n_out; those past it read
  // row n_out - 1 and store nothing)
  const int64_t rb0 = row0 + r16 < n_out ? row0 + r16 : n_out - 1;
  const int64_t moff1 = row0 + 16 < n_out ? 16 * nwords : 0;
  const uint32_t* const rp = w + rb0 * nwords + (GW == 16 ? 4 * g : 2 * g);
  f32x4d_t out[MB][NB], acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) out[mb][nb] = acc[mb][nb] = f32x4d_t{0.f, 0.f, 0.f, 0.f};
  // chunk 0: weights, copies, scales
  uint32_t wq[MB][4];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) load_chunk_words<GW>(rp + mb * moff1, wq[mb]);
#pragma unroll
  for (int i = 0; i < NB; ++i)
    __builtin_amdgcn_global_load_lds(xq_t + tid + 256 * i, (lds_ptr_t)(xa + 4 * (64 * wv + 256 * i)), 16, 0, 0);
  if (wv == 0 && lane < NT * GPC) __builtin_amdgcn_global_load_lds(xg_t + lane, (lds_ptr_t)ga, 4, 0, 0);
  {
    const int which = tid >> 7, rr = tid & 127;
    int64_t r = rw0 + rr;
    r = r < n_out ? r : n_out - 1;
    const void* src = which ? biases : scales;
    float v[2];
#pragma unroll
    for (int gi = 0; gi < GPC; ++gi) v[gi & 1] = ld_t<SDT>(src, r * n_groups + gi);
#pragma unroll
    for (int gi = 0; gi < GPC; ++gi) sb[0][which][rr][gi] = v[gi & 1];
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int64_t c0 = 0; c0 < nwords; c0 += 2 * kDenseChunk) {
    rtn4_dma_chunk<NB, GW, SDT>(rp, moff1, c0, nwords, xq_t, xg_t, scales, biases, rw0, n_out, n_groups, xa, ga, xb, gb,
                                sb[0], sb[1], wq, out, acc);
    if (c0 + kDenseChunk < nwords)
      rtn4_dma_chunk<NB, GW, SDT>(rp, moff1, c0 + kDenseChunk, nwords, xq_t, xg_t, scales, biases, rw0, n_out, n_groups,
                                  xb, gb, xa, ga, sb[1], sb[0], wq, out, acc);
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

// Workspace of the two-launch ternary GEMM (x' operands of every token tile,
// then (c, scale) per token).
// Workspace of the two-launch RMS-folded ternary GEMM: the x' operands (hi and
// lo halves) of every 32-token tile, then (c, scale) per token.
size_t tgemm_xp_bytes(int64_t batch, int64_t nwords) {
  const int64_t tiles = cdiv(batch, kXpTile);
  return static_cast<size_t>(tiles * 2 * nwords * 2 * kXpTile) * 16 +
         static_cast<size_t>(tiles * kXpTile) * 8;
}

// Launchers used by ternary_gemv.hip / rtn4.hip for batch >= 5 (bf16 x,
// [N, K/16] or [N, K/8] codes, nwords % 16 == 0, 16-byte aligned rows).
// Two-launch form: RMS-folded only (rms_w != NULL), workspace of
// tgemm_xp_bytes(batch, nwords) bytes, 256-byte aligned.
int launch_tgemm_xp(const uint16_t* x, int64_t batch, int64_t ldx, const uint32_t* w,
                    int64_t n_out, int64_t nwords, const void* alpha, int alpha_dt,
                    const void* rms_w, int rms_dt, float rms_eps, uint16_t* y, int64_t ldy,
                    void* workspace, hipStream_t s, const CombineIn& cb) {
  const int64_t tiles = cdiv(batch, kXpTile);
  uint4* xp = static_cast<uint4*>(workspace);
  float2* xc = reinterpret_cast<float2*>(xp + tiles * 2 * nwords * 2 * kXpTile);
  hipLaunchKernelGGL(k_xprep, dim3(static_cast<unsigned>(tiles * kXpTile)), dim3(128), 0, s, x,
                     batch, ldx, nwords, rms_w, rms_dt, rms_eps, kXpTile, xp, xc, cb);
  dim3 grid(static_cast<unsigned>(cdiv(n_out, 16)), static_cast<unsigned>(tiles));
  if (alpha_dt == MA_F32)
    hipLaunchKernelGGL((k_tgemm_xpk<kXpTile / 16, 2, MA_F32, 8>), grid, dim3(512), 0, s, xp, xc,
                       batch, w, n_out, nwords, alpha, y, ldy);
  else
    hipLaunchKernelGGL((k_tgemm_xpk<kXpTile / 16, 2, MA_BF16, 8>), grid, dim3(512), 0, s, xp, xc,
                       batch, w, n_out, nwords, alpha, y, ldy);
  return check_launch("ternary_gemv (mfma, two launches)");
}

// One-launch form: 16-token tiles (the kernel's VGPR use at 32 tokens halves
// the workgroups a CU holds; 16-token tiles were as fast or faster).
int launch_tgemm_mfma(const uint16_t* x, int64_t batch, int64_t ldx, const uint32_t* w,
                      int64_t n_out, int64_t nwords, const void* alpha, int alpha_dt,
                      const void* rms_w, int rms_dt, float rms_eps, uint16_t* y, int64_t ldy,
                      hipStream_t s) {
  dim3 grid(static_cast<unsigned>(cdiv(n_out, 16)), static_cast<unsigned>(cdiv(batch, 16)));
#define MA_TG(RDT, ADT)                                                                        \
  hipLaunchKernelGGL((k_tgemm_ks<1, RDT, ADT, 8>), grid, dim3(512), 0, s, x, batch, ldx, w, \
                     n_out, nwords, alpha, rms_w, rms_eps, y, ldy)
#define MA_TG_A(RDT) \
  if (alpha_dt == MA_F32) MA_TG(RDT, MA_F32); else MA_TG(RDT, MA_BF16);
  if (!rms_w) { MA_TG_A(-1) } else if (rms_dt == MA_F32) { MA_TG_A(MA_F32) } else { MA_TG_A(MA_BF16) }
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

// The workspace form: prep launch, then the DMA-fed GEMM (groups of 128;
// workspace of rtn4_ws_bytes(batch, nwords, 128) bytes, 256-byte aligned;
// n_out % 32 == 0).  (Groups of 64 hold twice the scales per chunk and spill
// at the occupancy this form needs; they keep the one-launch k_rtn4_mfma.)
int launch_rtn4_mfma_ws(const uint16_t* x, int64_t batch, int64_t ldx, const uint32_t* w,
                        int64_t n_out, int64_t nwords, int64_t group, const void* scales,
                        const void* biases, int s_dt, uint16_t* y, int64_t ldy, void* workspace,
                        hipStream_t s) {
  if (group != 128) return fail(MA_EVALUE, "rtn4_gemv_ws: the workspace form takes groups of 128");
  const int nb = batch <= 16 ? 1 : 2;
  const int64_t nt = 16 * nb, tiles = cdiv(batch, nt), chunks = nwords / kDenseChunk;
  uint4* xq = static_cast<uint4*>(workspace);
  float* xg = reinterpret_cast<float*>(xq + tiles * chunks * kDenseChunk * nt);
  dim3 gp(static_cast<unsigned>(tiles), static_cast<unsigned>(chunks));
  dim3 grid(static_cast<unsigned>(cdiv(n_out, kDenseRows)), static_cast<unsigned>(tiles));
#define MA_RD(NB, SDT)                                                                                  \
  hipLaunchKernelGGL((k_rtn4_xprep<NB, 16>), gp, dim3(256), 0, s, x, batch, ldx, nwords, xq, xg);       \
  hipLaunchKernelGGL((k_rtn4_mfma_dma<NB, 16, SDT>), grid, dim3(256), 0, s, xq, xg, batch, w, n_out,     \
                     nwords, scales, biases, y, ldy)
  if (nb == 1) {
    if (s_dt == MA_F32) { MA_RD(1, MA_F32); } else { MA_RD(1, MA_BF16); }
  } else {
    if (s_dt == MA_F32) { MA_RD(2, MA_F32); } else { MA_RD(2, MA_BF16); }
  }
#undef MA_RD
  return check_launch("rtn4_gemv (mfma, workspace)");
}
