// Grouped expert GEMMs on MFMA for batched decode and prefill (gfx950).
//
// After dispatch (pairs sorted by expert), every expert's tokens form a dense
// [tokens x K] operand, so the SwiGLU up+gate projection and the down
// projection become per-expert GEMMs: y = W_e (rows x K) . X_e^T (K x tokens).
//
// A operand (weights): a lane loads 16 bytes = 4 words = 64 codes of one row
// per 256-code chunk and expands each word with expand_word (common.h) into
// 8 bf16x2 dwords of 1 + c/f -- exactly the dword order of the bf16 x' pairs,
// which is an (arbitrary but shared) permutation of K inside each word.
// B operand (activations): x' = f * x pairs staged in LDS per chunk.  The
// MFMA then accumulates sum (f + c) x; subtracting C_t = sum (f + 1) x per
// token leaves sum (c - 1) x, the ternary product (float32 accumulation).
//
// v_mfma_f32_16x16x32_bf16 lane layout (checked on the device):
//   A: lane l holds row l%16, k 8(l/16)..+8;  B: col l%16, k 8(l/16)..+8;
//   C: lane l holds col l%16, rows 4(l/16)..+4.
//
// Stage 1: a workgroup owns 128 intermediate rows (each wave 32 up rows and
// the 32 matching gate rows, so SwiGLU is applied in registers) and a tile of
// 16*NB pairs of one expert.  It writes h (rounded to bf16 like the
// reference's x.dtype store, ternary_expert.py:441) in the x' pair layout the
// down stage reads, and optionally in the plain [slot, I] layout.
// Stage 2: a workgroup owns 256 output rows (each wave 64) and writes each
// pair's down output rounded to bf16 (ternary_expert.py:208); a gather
// kernel then forms y[t] = sum_j w[t,j] out[pair(t,j)] (+ residual) in
// float32 (fused_norm.py:83-96).
#include <mutex>

#include "mfma.h"

namespace ma {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kChunkWords = 16;  // 256 codes of K per step

__device__ __forceinline__ f32x4_t mfma_bf16(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Tile `tile` of a grouped launch with NT pairs per tile -> expert e, first
// sorted position pos0 and pair count np.  Each wave computes it (no LDS).
// Returns false for tiles past the end (the grid is an upper bound).
__device__ __forceinline__ bool decode_tile(const int32_t* __restrict__ offsets, int n_exp,
                                            int64_t tile, int nt, int& e, int& pos0, int& np) {
  const int lane = threadIdx.x & 63;
  int run = 0;  // tiles of the experts before this 64-expert slice
  for (int base = 0; base < n_exp; base += 64) {
    const int ee = base + lane;
    int tiles = 0;
    int o0 = 0, o1 = 0;
    if (ee < n_exp) {
      o0 = offsets[ee];
      o1 = offsets[ee + 1];
      tiles = (o1 - o0 + nt - 1) / nt;
    }
    int incl = tiles;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int v = __shfl_up(incl, off, 64);
      if (lane >= off) incl += v;
    }
    const int excl = incl - tiles;
    const bool mine = ee < n_exp && tile >= run + excl && tile < run + incl;
    const uint64_t m = __ballot(mine);
    if (m) {
      const int src = __ffsll(static_cast<unsigned long long>(m)) - 1;
      e = __shfl(ee, src, 64);
      const int t_in = static_cast<int>(tile) - run - __shfl(excl, src, 64);
      const int start = __shfl(o0, src, 64);
      const int end = __shfl(o1, src, 64);
      pos0 = start + t_in * nt;
      np = min(nt, end - pos0);
      return true;
    }
    run += __shfl(incl, 63, 64);
  }
  return false;
}

// Convert 16 bf16 activations (two uint4) into 8 x' pair dwords; returns
// sum (f + 1) x over them.
__device__ __forceinline__ float x16_to_pairs(uint4 a, uint4 b, uint32_t pr[8]) {
  const uint32_t u[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  float v[16];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    v[2 * q] = __uint_as_float(u[q] << 16);
    v[2 * q + 1] = __uint_as_float(u[q] & 0xffff0000u);
  }
  return prep_word_pairs(v, pr);
}

// sum (f + 1)/f * (lo + hi) over 8 x' pair dwords (recovers sum (f + 1) x).
__device__ __forceinline__ float pairs_cst(const uint32_t pr[8]) {
  float c = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float f = pair_scale(j);
    c += ((f + 1.0f) / f) * (__uint_as_float(pr[j] << 16) + __uint_as_float(pr[j] & 0xffff0000u));
  }
  return c;
}

template <int NB, int ADT>
__global__ __launch_bounds__(256) void k_grouped_swiglu(
    const uint16_t* __restrict__ x, int64_t ldx, int64_t topk,
    const uint32_t* __restrict__ w, int64_t n_half, int64_t nwords,
    const void* __restrict__ alpha, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ pair_ids, int n_exp,
    uint16_t* __restrict__ hp, uint16_t* __restrict__ h, int64_t ldh) {
  constexpr int NT = 16 * NB;
  __shared__ __align__(16) uint32_t xs[kChunkWords][2][NT][4];  // word-major: conflict-free B reads
  __shared__ float cst[NT], cw[kChunkWords][NT];  // corrections: per word, then summed in word order
  __shared__ int32_t tok[NT], pid[NT];
  int e, pos0, np;
  if (!decode_tile(offsets, n_exp, blockIdx.y, NT, e, pos0, np)) return;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  if (tid < NT) {
    const int p = tid < np ? pair_ids[pos0 + tid] : -1;
    pid[tid] = p;
    tok[tid] = p >= 0 ? static_cast<int>(p / topk) : -1;
    cst[tid] = 0.f;
  }
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * 128 + 32 * wv;
  const uint32_t* we = w + static_cast<int64_t>(e) * (2 * n_half) * nwords;
  const uint32_t* rowp[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    int64_t i = i0 + 16 * (mb & 1) + r16;
    i = i < n_half ? i : n_half - 1;
    rowp[mb] = we + (i + (mb >> 1) * n_half) * nwords + 4 * g;
  }
  f32x4_t acc[4][NB];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const ExpandConsts kc;
  __syncthreads();
  // Weights and x of chunk c0 (x' staging items: NT columns x 16 words, NB
  // per thread); the next chunk's are in flight during this chunk's work.
  auto load_chunk = [&](int64_t c0, uint4 (&wq)[4], uint4 (&xa)[NB], uint4 (&xb)[NB]) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) wq[mb] = *reinterpret_cast<const uint4*>(rowp[mb] + c0);
#pragma unroll
    for (int it = 0; it < NB; ++it) {
      const int item = tid + 256 * it;
      const int col = item % NT, wd = item / NT;
      const int t = tok[col];
      const uint4* src = reinterpret_cast<const uint4*>(x + static_cast<int64_t>(t < 0 ? 0 : t) * ldx + (c0 + wd) * 16);
      xa[it] = src[0];
      xb[it] = src[1];
    }
  };
  uint4 wq[4], xa[NB], xb[NB];
  load_chunk(0, wq, xa, xb);
  for (int64_t c0 = 0; c0 < nwords; c0 += kChunkWords) {
    uint4 wn[4], xan[NB], xbn[NB];
    load_chunk(c0 + kChunkWords < nwords ? c0 + kChunkWords : c0, wn, xan, xbn);
    // (no sched_barrier here: with loads into loop-carried registers just
    // above, it produced wrong MFMA operands on this compiler)
#pragma unroll
    for (int it = 0; it < NB; ++it) {
      const int item = tid + 256 * it;
      const int col = item % NT, wd = item / NT;
      uint32_t pr[8];
      float c = 0.f;
      if (tok[col] >= 0) {
        c = x16_to_pairs(xa[it], xb[it], pr);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) pr[j] = 0u;
      }
      *reinterpret_cast<uint4*>(&xs[wd][0][col][0]) = make_uint4(pr[0], pr[1], pr[2], pr[3]);
      *reinterpret_cast<uint4*>(&xs[wd][1][col][0]) = make_uint4(pr[4], pr[5], pr[6], pr[7]);
      cw[wd][col] = c;
    }
    __syncthreads();
    if (tid < NT) {  // a fixed order: the same bits on every run
      float c = cst[tid];
#pragma unroll
      for (int wd = 0; wd < kChunkWords; ++wd) c += cw[wd][tid];
      cst[tid] = c;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {  // word q of the lane's 4 -> MFMA steps 2q, 2q+1
      uint4 a[4][2];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const uint32_t wsel = q == 0 ? wq[mb].x : q == 1 ? wq[mb].y : q == 2 ? wq[mb].z : wq[mb].w;
        uint32_t ex[8];
        expand_word(wsel, ex, kc);
        a[mb][0] = make_uint4(ex[0], ex[1], ex[2], ex[3]);
        a[mb][1] = make_uint4(ex[4], ex[5], ex[6], ex[7]);
      }
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const uint4 b = *reinterpret_cast<const uint4*>(&xs[4 * g + q][hf][nb * 16 + r16][0]);
#pragma unroll
          for (int mb = 0; mb < 4; ++mb) acc[mb][nb] = mfma_bf16(a[mb][hf], b, acc[mb][nb]);
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) wq[mb] = wn[mb];
#pragma unroll
    for (int it = 0; it < NB; ++it) {
      xa[it] = xan[it];
      xb[it] = xbn[it];
    }
  }
  // Epilogue: rows i0 + 16 mb + 4 g + r (up: mb 0,1; gate: mb 2,3 -> same rows).
  const int64_t nwh = n_half / 16;
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t i = i0 + 16 * mb + 4 * g + r;
      if (i >= n_half) continue;
      const int64_t ia = i < n_half ? i : n_half - 1;
      const float au = ld_t<ADT>(alpha, static_cast<int64_t>(e) * 2 * n_half + ia);
      const float ag = ld_t<ADT>(alpha, static_cast<int64_t>(e) * 2 * n_half + n_half + ia);
      const int pos = static_cast<int>(i & 15), j = pos & 7, hh = pos >> 3;
      const float f = pair_scale(j);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int col = nb * 16 + r16;
        if (col >= np) continue;
        const float c = cst[col];
        const float up = au * (acc[mb][nb][r] - c);
        const float gt = ag * (acc[mb + 2][nb][r] - c);
        const uint16_t hb = f32_to_bf16(swiglu_act(up, gt));
        if (hp) {
          const float hv = bf16_to_f32(hb) * f;  // exact: power-of-two scale
          hp[((static_cast<int64_t>(pos0 + col) * nwh + (i >> 4)) * 8 + j) * 2 + hh] =
              static_cast<uint16_t>(bf16_bits_exact(hv));
        }
        if (h) h[static_cast<int64_t>(pid[col]) * ldh + i] = hb;
      }
    }
  }
}

template <int NB, int ADT>
__global__ __launch_bounds__(256) void k_grouped_down(
    const uint32_t* __restrict__ hp, const uint32_t* __restrict__ w, int64_t n_out,
    int64_t nwk, const void* __restrict__ alpha, const int32_t* __restrict__ offsets,
    int n_exp, uint16_t* __restrict__ out) {
  constexpr int NT = 16 * NB;
  __shared__ __align__(16) uint32_t xs[kChunkWords][2][NT][4];  // word-major: conflict-free B reads
  __shared__ float cst[NT], cw[kChunkWords][NT];  // corrections: per word, then summed in word order
  int e, pos0, np;
  if (!decode_tile(offsets, n_exp, blockIdx.y, NT, e, pos0, np)) return;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  if (tid < NT) cst[tid] = 0.f;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 256 + 64 * wv;
  const uint32_t* we = w + static_cast<int64_t>(e) * n_out * nwk;
  const uint32_t* rowp[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    int64_t n = n0 + 16 * mb + r16;
    n = n < n_out ? n : n_out - 1;
    rowp[mb] = we + n * nwk + 4 * g;
  }
  f32x4_t acc[4][NB];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const ExpandConsts kc;
  __syncthreads();
  auto load_chunk = [&](int64_t c0, uint4 (&wq)[4], uint4 (&ha)[NB], uint4 (&hb)[NB]) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) wq[mb] = *reinterpret_cast<const uint4*>(rowp[mb] + c0);
#pragma unroll
    for (int it = 0; it < NB; ++it) {
      const int item = tid + 256 * it;
      const int col = item % NT, wd = item / NT;
      const int64_t prow = pos0 + (col < np ? col : 0);
      const uint4* src = reinterpret_cast<const uint4*>(hp + (prow * nwk + c0 + wd) * 8);
      ha[it] = src[0];
      hb[it] = src[1];
    }
  };
  uint4 wq[4], ha[NB], hb[NB];
  load_chunk(0, wq, ha, hb);
  for (int64_t c0 = 0; c0 < nwk; c0 += kChunkWords) {
    uint4 wn[4], han[NB], hbn[NB];
    load_chunk(c0 + kChunkWords < nwk ? c0 + kChunkWords : c0, wn, han, hbn);
    // (no sched_barrier here: with loads into loop-carried registers just
    // above, it produced wrong MFMA operands on this compiler)
#pragma unroll
    for (int it = 0; it < NB; ++it) {
      const int item = tid + 256 * it;
      const int col = item % NT, wd = item / NT;
      uint32_t pr[8] = {ha[it].x, ha[it].y, ha[it].z, ha[it].w, hb[it].x, hb[it].y, hb[it].z, hb[it].w};
      if (col >= np) {
#pragma unroll
        for (int j = 0; j < 8; ++j) pr[j] = 0u;
      }
      *reinterpret_cast<uint4*>(&xs[wd][0][col][0]) = make_uint4(pr[0], pr[1], pr[2], pr[3]);
      *reinterpret_cast<uint4*>(&xs[wd][1][col][0]) = make_uint4(pr[4], pr[5], pr[6], pr[7]);
      cw[wd][col] = pairs_cst(pr);
    }
    __syncthreads();
    if (tid < NT) {  // a fixed order: the same bits on every run
      float c = cst[tid];
#pragma unroll
      for (int wd = 0; wd < kChunkWords; ++wd) c += cw[wd][tid];
      cst[tid] = c;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint4 a[4][2];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const uint32_t wsel = q == 0 ? wq[mb].x : q == 1 ? wq[mb].y : q == 2 ? wq[mb].z : wq[mb].w;
        uint32_t ex[8];
        expand_word(wsel, ex, kc);
        a[mb][0] = make_uint4(ex[0], ex[1], ex[2], ex[3]);
        a[mb][1] = make_uint4(ex[4], ex[5], ex[6], ex[7]);
      }
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const uint4 b = *reinterpret_cast<const uint4*>(&xs[4 * g + q][hf][nb * 16 + r16][0]);
#pragma unroll
          for (int mb = 0; mb < 4; ++mb) acc[mb][nb] = mfma_bf16(a[mb][hf], b, acc[mb][nb]);
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) wq[mb] = wn[mb];
#pragma unroll
    for (int it = 0; it < NB; ++it) {
      ha[it] = han[it];
      hb[it] = hbn[it];
    }
  }
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t n = n0 + 16 * mb + 4 * g + r;
      if (n >= n_out) continue;
      const float a = ld_t<ADT>(alpha, static_cast<int64_t>(e) * n_out + n);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int col = nb * 16 + r16;
        if (col >= np) continue;
        out[static_cast<int64_t>(pos0 + col) * n_out + n] = f32_to_bf16(a * (acc[mb][nb][r] - cst[col]));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Decode form (few pairs per expert): 16-pair tiles, K split over the KW waves
// of a workgroup, each wave's operands loaded and built in registers (no LDS
// staging) and the partial tiles added in wave order through LDS; with a
// handful of tokens per expert, a K walk per workgroup left the chip idle.
// Same per-word arithmetic as the kernels above; every sum has a fixed order.
// ---------------------------------------------------------------------------

// SwiGLU stage: a workgroup takes 16 MBH intermediate rows (MBH 16-row blocks
// of up rows and the matching gate rows) of one 16-pair tile; wave w takes the
// 16-word chunks w, w + KW, ... of K.  PAIRS: the activations arrive as x'
// pairs with their per-token correction (x_pairs, x_corr: built once per
// token upstream) and are loaded as B operands directly; otherwise each lane
// builds its B operands from x.
template <int MBH, int ADT, int KW, bool PAIRS>
__global__ __launch_bounds__(64 * KW) void k_grouped_swiglu_ks(
    const uint16_t* __restrict__ x, int64_t ldx, const uint32_t* __restrict__ x_pairs,
    const float* __restrict__ x_corr, int64_t topk,
    const uint32_t* __restrict__ w, int64_t n_half, int64_t nwords,
    const void* __restrict__ alpha, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ pair_ids, int n_exp,
    uint16_t* __restrict__ hp, uint16_t* __restrict__ h, int64_t ldh) {
  constexpr int MB = 2 * MBH;  // row blocks: up 0 .. MBH-1, gate MBH .. MB-1
  static_assert(KW >= MBH, "the epilogue takes 64 threads per up block");
  __shared__ float red[KW][MB][4][64];
  __shared__ float red_c[KW][4][16];
  int e, pos0, np;
  if (!decode_tile(offsets, n_exp, blockIdx.y, 16, e, pos0, np)) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * 16 * MBH;
  const uint32_t* we = w + static_cast<int64_t>(e) * (2 * n_half) * nwords;
  const uint32_t* rowp[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    int64_t i = i0 + 16 * (mb % MBH) + r16;
    i = i < n_half ? i : n_half - 1;
    rowp[mb] = we + (i + (mb / MBH) * n_half) * nwords + 4 * g;
  }
  // this lane's B column: pair pos0 + r16 (token row of x), zero past np
  const bool valid = r16 < np;
  const int64_t tok = valid ? pair_ids[pos0 + r16] / topk : 0;
  const uint16_t* xrow = x + tok * ldx + 64 * g;
  const uint32_t* prow = x_pairs + (tok * nwords + 4 * g) * 8;
  f32x4d_t acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4d_t{0.f, 0.f, 0.f, 0.f};
  float cp = 0.f;
  const ExpandConsts kc;
  for (int64_t c0 = 16 * wv; c0 < nwords; c0 += 16 * KW) {
    u32x4v_t wq[MB], xv[4][2];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) wq[mb] = *reinterpret_cast<const u32x4v_t*>(rowp[mb] + c0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x4v_t* src = PAIRS ? reinterpret_cast<const u32x4v_t*>(prow + (c0 + q) * 8)
                                  : reinterpret_cast<const u32x4v_t*>(xrow + (c0 + q) * 16);
      xv[q][0] = src[0];
      xv[q][1] = src[1];
    }
    MA_ISSUE_FENCE();  // every load of the chunk in flight before the first use
#pragma unroll
    for (int qh = 0; qh < 4; qh += 2) {  // two words per step (operand registers)
      u32x4v_t av[2][MB][2], bv[2][2];
#pragma unroll
      for (int qi = 0; qi < 2; ++qi) {
        const int q = qh + qi;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          uint32_t ex[8];
          expand_word(wq[mb][q], ex, kc);
          av[qi][mb][0] = u32x4v_t{ex[0], ex[1], ex[2], ex[3]};
          av[qi][mb][1] = u32x4v_t{ex[4], ex[5], ex[6], ex[7]};
        }
        if constexpr (PAIRS) {
          bv[qi][0] = valid ? xv[q][0] : u32x4v_t{0u, 0u, 0u, 0u};
          bv[qi][1] = valid ? xv[q][1] : u32x4v_t{0u, 0u, 0u, 0u};
        } else {
          uint32_t pr[8];
          const float c = x16_to_pairs(make_uint4(xv[q][0].x, xv[q][0].y, xv[q][0].z, xv[q][0].w),
                                       make_uint4(xv[q][1].x, xv[q][1].y, xv[q][1].z, xv[q][1].w), pr);
          cp += valid ? c : 0.f;
          bv[qi][0] = valid ? u32x4v_t{pr[0], pr[1], pr[2], pr[3]} : u32x4v_t{0u, 0u, 0u, 0u};
          bv[qi][1] = valid ? u32x4v_t{pr[4], pr[5], pr[6], pr[7]} : u32x4v_t{0u, 0u, 0u, 0u};
        }
      }
      pin(cp);
      mfma_block_begin();
#pragma unroll
      for (int qi = 0; qi < 2; ++qi)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) mfma_acc(acc[mb], av[qi][mb][hf], bv[qi][hf]);
      mfma_block_end();
      keep_b(av, acc);
      keep_b(bv, acc);
    }
  }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wv][mb][r][lane] = acc[mb][r];
  if constexpr (!PAIRS) red_c[wv][g][r16] = cp;
  __syncthreads();
  // Thread t < 64 MBH: pair column col = t % 16, rows 4 rq .. +3 of up block mbu.
  if (tid >= 64 * MBH) return;
  const int col = tid & 15, rq = (tid >> 4) & 3, mbu = tid >> 6;
  if (col >= np) return;
  const int pid = pair_ids[pos0 + col];
  float c = 0.f;
  if constexpr (PAIRS) {
    c = x_corr[pid / topk];
  } else {
#pragma unroll
    for (int k = 0; k < KW; ++k)
#pragma unroll
      for (int gg = 0; gg < 4; ++gg) c += red_c[k][gg][col];
  }
  const int ln = col + 16 * rq;
  const int64_t nwh = n_half / 16;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t i = i0 + 16 * mbu + 4 * rq + r;
    if (i >= n_half) continue;
    float su = 0.f, sg = 0.f;
#pragma unroll
    for (int k = 0; k < KW; ++k) {
      su += red[k][mbu][r][ln];
      sg += red[k][mbu + MBH][r][ln];
    }
    const float au = ld_t<ADT>(alpha, static_cast<int64_t>(e) * 2 * n_half + i);
    const float ag = ld_t<ADT>(alpha, static_cast<int64_t>(e) * 2 * n_half + n_half + i);
    const uint16_t hb = f32_to_bf16(swiglu_act(au * (su - c), ag * (sg - c)));
    if (hp) {
      const int pos = static_cast<int>(i & 15), j = pos & 7, hh = pos >> 3;
      const float hv = bf16_to_f32(hb) * pair_scale(j);  // exact: power-of-two scale
      hp[((static_cast<int64_t>(pos0 + col) * nwh + (i >> 4)) * 8 + j) * 2 + hh] =
          static_cast<uint16_t>(bf16_bits_exact(hv));
    }
    if (h) h[static_cast<int64_t>(pid) * ldh + i] = hb;
  }
}

// Down stage: a workgroup takes 16 MB output rows of one 16-pair tile; wave w
// takes the 4 QW-word chunks w, w + KW, ... of K (QW words per lane), reading
// h's x' pairs straight from the pair-format buffer.
template <int MB, int ADT, int KW, int QW>
__global__ __launch_bounds__(64 * KW) void k_grouped_down_ks(
    const uint32_t* __restrict__ hp, const uint32_t* __restrict__ w, int64_t n_out,
    int64_t nwk, const void* __restrict__ alpha, const int32_t* __restrict__ offsets,
    int n_exp, uint16_t* __restrict__ out) {
  constexpr int CW = 4 * QW;  // words per chunk
  static_assert(KW >= MB, "the epilogue takes 64 threads per row block");
  __shared__ float red[KW][MB][4][64];
  __shared__ float red_c[KW][4][16];
  int e, pos0, np;
  if (!decode_tile(offsets, n_exp, blockIdx.y, 16, e, pos0, np)) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16 * MB;
  const uint32_t* we = w + static_cast<int64_t>(e) * n_out * nwk;
  const uint32_t* rowp[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    int64_t n = n0 + 16 * mb + r16;
    n = n < n_out ? n : n_out - 1;
    rowp[mb] = we + n * nwk + QW * g;
  }
  const bool valid = r16 < np;
  const uint32_t* hrow = hp + static_cast<int64_t>(pos0 + (valid ? r16 : 0)) * nwk * 8 + QW * g * 8;
  f32x4d_t acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4d_t{0.f, 0.f, 0.f, 0.f};
  float cp = 0.f;
  const ExpandConsts kc;
  for (int64_t c0 = CW * wv; c0 < nwk; c0 += CW * KW) {
    uint32_t wq[MB][QW];
    u32x4v_t bv[QW][2];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      if constexpr (QW == 2) {
        const uint2 v2 = *reinterpret_cast<const uint2*>(rowp[mb] + c0);
        wq[mb][0] = v2.x;
        wq[mb][1] = v2.y;
      } else {
#pragma unroll
        for (int q = 0; q < QW; ++q) wq[mb][q] = rowp[mb][c0 + q];
      }
    }
#pragma unroll
    for (int q = 0; q < QW; ++q) {
      const u32x4v_t* src = reinterpret_cast<const u32x4v_t*>(hrow + (c0 + q) * 8);
      bv[q][0] = src[0];
      bv[q][1] = src[1];
    }
    MA_ISSUE_FENCE();  // every load of the chunk in flight before the first use
#pragma unroll
    for (int q = 0; q < QW; ++q) {  // one word per step (operand registers)
      u32x4v_t av[MB][2];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        uint32_t ex[8];
        expand_word(wq[mb][q], ex, kc);
        av[mb][0] = u32x4v_t{ex[0], ex[1], ex[2], ex[3]};
        av[mb][1] = u32x4v_t{ex[4], ex[5], ex[6], ex[7]};
      }
      if (!valid) bv[q][0] = bv[q][1] = u32x4v_t{0u, 0u, 0u, 0u};
      const uint32_t pr[8] = {bv[q][0].x, bv[q][0].y, bv[q][0].z, bv[q][0].w,
                              bv[q][1].x, bv[q][1].y, bv[q][1].z, bv[q][1].w};
      cp += pairs_cst(pr);
      pin(cp);
      mfma_block_begin();
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) mfma_acc(acc[mb], av[mb][hf], bv[q][hf]);
      mfma_block_end();
      keep_b(av, acc);
      keep_b(bv[q], acc);
    }
  }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wv][mb][r][lane] = acc[mb][r];
  red_c[wv][g][r16] = cp;
  __syncthreads();
  // Thread t < 64 MB: pair column col = t % 16, rows 4 rq .. +3 of block mb.
  if (tid >= 64 * MB) return;
  const int col = tid & 15, rq = (tid >> 4) & 3, mb = tid >> 6;
  if (col >= np) return;
  float c = 0.f;
#pragma unroll
  for (int k = 0; k < KW; ++k)
#pragma unroll
    for (int gg = 0; gg < 4; ++gg) c += red_c[k][gg][col];
  const int ln = col + 16 * rq;
  const int64_t nb0 = n0 + 16 * mb + 4 * rq;
  float o[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < KW; ++k) s += red[k][mb][r][ln];
    const int64_t n = nb0 + r < n_out ? nb0 + r : n_out - 1;
    o[r] = ld_t<ADT>(alpha, static_cast<int64_t>(e) * n_out + n) * (s - c);
  }
  uint16_t* orow = out + static_cast<int64_t>(pos0 + col) * n_out;
  if (nb0 + 3 < n_out) {
    uint2 rr;
    rr.x = pack_bf16x2_rn(o[0], o[1]);
    rr.y = pack_bf16x2_rn(o[2], o[3]);
    *reinterpret_cast<uint2*>(orow + nb0) = rr;
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (nb0 + r < n_out) orow[nb0 + r] = f32_to_bf16(o[r]);
  }
}

// ---------------------------------------------------------------------------
// Decode form, tile-resident: a workgroup stages its 16-pair tile's B operands
// for all of K in LDS once (one sync), then each wave takes whole 16-row
// blocks over all of K: a block's weights for the full K are loaded up front
// (8 words per lane at K = 2048 ... per chunk of 16 words one uint4), so a
// wave keeps all its weight bytes in flight at once and needs no cross-wave
// reduction.  Same per-word arithmetic as the kernels above; each output is
// one MFMA chain (fixed order).
// ---------------------------------------------------------------------------
constexpr int kErWaves = 8;
// K of the tile-resident forms, in 256-code chunks (instantiated for the
// synthetic model's hidden 2048 and intermediate 768; other sizes take the
// K-split forms).
constexpr int kErChunksUp = 8, kErChunksDown = 3;

// SwiGLU: BPW up blocks (and the matching gate blocks) per wave; x' pairs of
// the tile's tokens (x_pairs [T, K / 2] uint32, x_corr [T]) staged in LDS.
template <int BPW, int ADT, int NCH, int QPB>
__global__ __launch_bounds__(64 * kErWaves) void k_grouped_swiglu_er(
    const uint32_t* __restrict__ x_pairs, const float* __restrict__ x_corr, int64_t topk,
    const uint32_t* __restrict__ w, int64_t n_half, const void* __restrict__ alpha,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ pair_ids, int n_exp,
    uint16_t* __restrict__ hp, uint16_t* __restrict__ h, int64_t ldh) {
  constexpr int NW = 16 * NCH;  // words of K
  __shared__ u32x4v_t xs[NW][2][16];
  __shared__ int32_t s_pid[16], s_tok[16];
  __shared__ float s_c[16];
  int e, pos0, np;
  if (!decode_tile(offsets, n_exp, blockIdx.y, 16, e, pos0, np)) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int64_t nblk = n_half / 16;
  const int64_t b0 = (static_cast<int64_t>(blockIdx.x) * kErWaves + wv) * BPW;  // first up block
  const uint32_t* we = w + static_cast<int64_t>(e) * (2 * n_half) * NW;
  // Issue order matters (memory counters complete in issue order): the pair
  // ids, then the tile's x' pairs, then the weights, so that staging x' waits
  // for nothing behind it and the weights stream while it happens.
  if (tid < 16) {
    const int p = tid < np ? pair_ids[pos0 + tid] : -1;
    s_pid[tid] = p;
    s_tok[tid] = p >= 0 ? static_cast<int>(p / topk) : -1;
  }
  __syncthreads();
  // the tile's x' pairs: item = (col, word, half), 16-byte loads
  constexpr int kItems = 16 * NW * 2, kPer = (kItems + 64 * kErWaves - 1) / (64 * kErWaves);
  u32x4v_t sv[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int it = tid + 64 * kErWaves * k;
    const int col = (it < kItems ? it : 0) / (NW * 2), rem = it % (NW * 2);
    const int tk = s_tok[col];
    sv[k] = u32x4v_t{0u, 0u, 0u, 0u};
    if (it < kItems && tk >= 0)
      sv[k] = *reinterpret_cast<const u32x4v_t*>(x_pairs + static_cast<int64_t>(tk) * (NW * 8) + rem * 4);
  }
  float cx = 0.f;
  if (tid < 16 && s_tok[tid] >= 0) cx = x_corr[s_tok[tid]];
  // weights of this wave's blocks for all of K
  u32x4v_t wq[2 * BPW][NCH];
#pragma unroll
  for (int j = 0; j < 2 * BPW; ++j) {
    int64_t blk = b0 + (j % BPW);
    blk = blk < nblk ? blk : nblk - 1;
    const uint32_t* rp = we + ((j / BPW) * n_half + blk * 16 + r16) * NW + 4 * g;
#pragma unroll
    for (int c = 0; c < NCH; ++c) wq[j][c] = *reinterpret_cast<const u32x4v_t*>(rp + 16 * c);
  }
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int it = tid + 64 * kErWaves * k;
    if (it < kItems) xs[(it % (NW * 2)) >> 1][it & 1][it / (NW * 2)] = sv[k];
  }
  if (tid < 16) s_c[tid] = cx;
  __syncthreads();
  // two accumulators per block (the two halves of each word), so a block's
  // MFMAs are independent of each other
  f32x4d_t acc[2 * BPW][2];
#pragma unroll
  for (int j = 0; j < 2 * BPW; ++j) acc[j][0] = acc[j][1] = f32x4d_t{0.f, 0.f, 0.f, 0.f};
  const ExpandConsts kc;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
#pragma unroll
    for (int q0 = 0; q0 < 4; q0 += QPB) {  // QPB words per MFMA block
      u32x4v_t av[QPB][2 * BPW][2], bv[QPB][2];
#pragma unroll
      for (int qi = 0; qi < QPB; ++qi) {
#pragma unroll
        for (int j = 0; j < 2 * BPW; ++j) {
          uint32_t ex[8];
          expand_word(wq[j][c][q0 + qi], ex, kc);
          av[qi][j][0] = u32x4v_t{ex[0], ex[1], ex[2], ex[3]};
          av[qi][j][1] = u32x4v_t{ex[4], ex[5], ex[6], ex[7]};
        }
        bv[qi][0] = xs[16 * c + 4 * g + q0 + qi][0][r16];
        bv[qi][1] = xs[16 * c + 4 * g + q0 + qi][1][r16];
      }
      mfma_block_begin();
#pragma unroll
      for (int qi = 0; qi < QPB; ++qi)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
          for (int j = 0; j < 2 * BPW; ++j) mfma_acc(acc[j][hf], av[qi][j][hf], bv[qi][hf]);
      mfma_block_end();
      keep_b(av, acc[0]);
      keep_b(bv, acc[0]);
    }
  }
  f32x4d_t accs[2 * BPW];
#pragma unroll
  for (int j = 0; j < 2 * BPW; ++j) accs[j] = acc[j][0] + acc[j][1];
  // Epilogue: lane holds pair column r16, rows 4 g .. +3 of each block.
  if (r16 >= np) return;
  const float cc = s_c[r16];
  const int pid = s_pid[r16];
  const int64_t nwh = n_half / 16;
#pragma unroll
  for (int j = 0; j < BPW; ++j) {
    const int64_t blk = b0 + j;
    if (blk >= nblk) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t i = blk * 16 + 4 * g + r;
      const float au = ld_t<ADT>(alpha, static_cast<int64_t>(e) * 2 * n_half + i);
      const float ag = ld_t<ADT>(alpha, static_cast<int64_t>(e) * 2 * n_half + n_half + i);
      const uint16_t hb = f32_to_bf16(swiglu_act(au * (accs[j][r] - cc), ag * (accs[BPW + j][r] - cc)));
      if (hp) {
        const int pos = static_cast<int>(i & 15), jj = pos & 7, hh = pos >> 3;
        const float hv = bf16_to_f32(hb) * pair_scale(jj);  // exact: power-of-two scale
        hp[((static_cast<int64_t>(pos0 + r16) * nwh + (i >> 4)) * 8 + jj) * 2 + hh] =
            static_cast<uint16_t>(bf16_bits_exact(hv));
      }
      if (h) h[static_cast<int64_t>(pid) * ldh + i] = hb;
    }
  }
}

// Down: BPW output blocks per wave; h's x' pairs of the tile (hp rows pos0 ..)
// staged in LDS with each pair's correction.
template <int BPW, int ADT, int NCH>
__global__ __launch_bounds__(64 * kErWaves) void k_grouped_down_er(
    const uint32_t* __restrict__ hp, const uint32_t* __restrict__ w, int64_t n_out,
    const void* __restrict__ alpha, const int32_t* __restrict__ offsets, int n_exp,
    uint16_t* __restrict__ out) {
  constexpr int NW = 16 * NCH;  // words of K
  __shared__ u32x4v_t xs[NW][2][16];
  __shared__ float s_cw[16][NW];
  __shared__ float s_c[16];
  int e, pos0, np;
  if (!decode_tile(offsets, n_exp, blockIdx.y, 16, e, pos0, np)) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int64_t nblk = n_out / 16;
  const int64_t b0 = (static_cast<int64_t>(blockIdx.x) * kErWaves + wv) * BPW;
  const uint32_t* we = w + static_cast<int64_t>(e) * n_out * NW;
  // stage: item = (col, word): both halves of the word and its correction;
  // these loads go out before the weights' (memory counters complete in issue
  // order), so staging does not wait for the weight stream
  constexpr int kItems = 16 * NW, kPer = (kItems + 64 * kErWaves - 1) / (64 * kErWaves);
  u32x4v_t sv[kPer][2];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int it = tid + 64 * kErWaves * k;
    const int col = it / NW, wd = it % NW;
    sv[k][0] = sv[k][1] = u32x4v_t{0u, 0u, 0u, 0u};
    if (it < kItems && col < np) {
      const u32x4v_t* src = reinterpret_cast<const u32x4v_t*>(hp + (static_cast<int64_t>(pos0 + col) * NW + wd) * 8);
      sv[k][0] = src[0];
      sv[k][1] = src[1];
    }
  }
  // weights of this wave's blocks for all of K
  u32x4v_t wq[BPW][NCH];
#pragma unroll
  for (int j = 0; j < BPW; ++j) {
    int64_t blk = b0 + j;
    blk = blk < nblk ? blk : nblk - 1;
    const uint32_t* rp = we + (blk * 16 + r16) * NW + 4 * g;
#pragma unroll
    for (int c = 0; c < NCH; ++c) wq[j][c] = *reinterpret_cast<const u32x4v_t*>(rp + 16 * c);
  }
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int it = tid + 64 * kErWaves * k;
    if (it >= kItems) continue;
    const int col = it / NW, wd = it % NW;
    xs[wd][0][col] = sv[k][0];
    xs[wd][1][col] = sv[k][1];
    const uint32_t pr[8] = {sv[k][0].x, sv[k][0].y, sv[k][0].z, sv[k][0].w,
                            sv[k][1].x, sv[k][1].y, sv[k][1].z, sv[k][1].w};
    s_cw[col][wd] = pairs_cst(pr);
  }
  __syncthreads();
  if (tid < 16) {  // fixed order
    float c = 0.f;
    for (int wd = 0; wd < NW; ++wd) c += s_cw[tid][wd];
    s_c[tid] = c;
  }
  f32x4d_t acc[BPW][2];  // per word half: a block's MFMAs are independent
#pragma unroll
  for (int j = 0; j < BPW; ++j) acc[j][0] = acc[j][1] = f32x4d_t{0.f, 0.f, 0.f, 0.f};
  const ExpandConsts kc;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      u32x4v_t av[BPW][2], bv[2];
#pragma unroll
      for (int j = 0; j < BPW; ++j) {
        uint32_t ex[8];
        expand_word(wq[j][c][q], ex, kc);
        av[j][0] = u32x4v_t{ex[0], ex[1], ex[2], ex[3]};
        av[j][1] = u32x4v_t{ex[4], ex[5], ex[6], ex[7]};
      }
      bv[0] = xs[16 * c + 4 * g + q][0][r16];
      bv[1] = xs[16 * c + 4 * g + q][1][r16];
      mfma_block_begin();
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int j = 0; j < BPW; ++j) mfma_acc(acc[j][hf], av[j][hf], bv[hf]);
      mfma_block_end();
      keep_b(av, acc[0]);
      keep_b(bv, acc[0]);
    }
  }
  f32x4d_t accs[BPW];
#pragma unroll
  for (int j = 0; j < BPW; ++j) accs[j] = acc[j][0] + acc[j][1];
  __syncthreads();  // s_c
  if (r16 >= np) return;
  const float cc = s_c[r16];
  uint16_t* orow = out + static_cast<int64_t>(pos0 + r16) * n_out;
#pragma unroll
  for (int j = 0; j < BPW; ++j) {
    const int64_t blk = b0 + j;
    if (blk >= nblk) continue;
    const int64_t n0 = blk * 16 + 4 * g;
    float o[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) o[r] = ld_t<ADT>(alpha, static_cast<int64_t>(e) * n_out + n0 + r) * (accs[j][r] - cc);
    uint2 rr;
    rr.x = pack_bf16x2_rn(o[0], o[1]);
    rr.y = pack_bf16x2_rn(o[2], o[3]);
    *reinterpret_cast<uint2*>(orow + n0) = rr;
  }
}

// y[t, n] = sum_j w[t, j] * out[inverse[t*k + j], n] (+ residual), float32 sum.
__global__ __launch_bounds__(256) void k_combine(const uint16_t* __restrict__ out,
                                                 const int32_t* __restrict__ inverse,
                                                 const float* __restrict__ wts, int64_t topk,
                                                 int64_t n, const void* __restrict__ res,
                                                 int res_dt, uint16_t* __restrict__ y) {
  const int64_t t = blockIdx.y;
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 2;
  if (i >= n) return;
  float a0 = 0.f, a1 = 0.f;
  for (int64_t j = 0; j < topk; ++j) {
    const float wj = wts[t * topk + j];
    const uint32_t v = *reinterpret_cast<const uint32_t*>(out + static_cast<int64_t>(inverse[t * topk + j]) * n + i);
    a0 += wj * __uint_as_float(v << 16);
    a1 += wj * __uint_as_float(v & 0xffff0000u);
  }
  if (res) {
    a0 += ld_f(res, res_dt, t * n + i);
    a1 += ld_f(res, res_dt, t * n + i + 1);
  }
  *reinterpret_cast<uint32_t*>(y + t * n + i) =
      static_cast<uint32_t>(f32_to_bf16(a0)) | (static_cast<uint32_t>(f32_to_bf16(a1)) << 16);
}

// The same combine for top-k <= K, bf16 rows, 8 outputs per thread: the
// token's k (position, weight) pairs are wave-uniform scalar loads, then every
// slot's 16-byte load and the residual's are issued before the sums (the
// arithmetic and its order are k_combine's).
template <int K>
__global__ __launch_bounds__(256) void k_combine8(const uint16_t* __restrict__ out,
                                                  const int32_t* __restrict__ inverse,
                                                  const float* __restrict__ wts, int topk,
                                                  int64_t n, const uint16_t* __restrict__ res,
                                                  uint16_t* __restrict__ y) {
  const int64_t t = blockIdx.y;
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 8;
  int64_t row[K];
  float wj[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    row[j] = j < topk ? inverse[t * topk + j] : 0;
    wj[j] = j < topk ? wts[t * topk + j] : 0.f;
  }
  if (i >= n) return;
  uint4 v[K], r = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
  for (int j = 0; j < K; ++j)
    if (j < topk) v[j] = *reinterpret_cast<const uint4*>(out + row[j] * n + i);
  if (res) r = *reinterpret_cast<const uint4*>(res + t * n + i);
  float a[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) a[e] = 0.f;
#pragma unroll
  for (int j = 0; j < K; ++j) {
    if (j >= topk) break;
    const uint32_t u[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      a[2 * q] += wj[j] * __uint_as_float(u[q] << 16);
      a[2 * q + 1] += wj[j] * __uint_as_float(u[q] & 0xffff0000u);
    }
  }
  if (res) {
    const uint32_t u[4] = {r.x, r.y, r.z, r.w};
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
  *reinterpret_cast<uint4*>(y + t * n + i) = o;
}

}  // namespace ma

using namespace ma;

// Up to this many pairs per expert on average (decode batches) the K-split
// kernels run; above it (prefill) the LDS-staged tiles of up to 64 pairs.
constexpr int64_t kKsMaxPairsPerExpert = 16;

static int grouped_nb(int64_t n_pairs, int64_t n_exp) {
  const int64_t per = n_pairs / (n_exp > 0 ? n_exp : 1);
  return per >= 48 ? 4 : (per >= 24 ? 2 : 1);
}

extern "C" size_t ma_grouped_workspace_bytes(int64_t n_pairs, int64_t inter, int64_t hidden) {
  // pair-format h [P, inter] bf16 + per-pair down outputs [P, hidden] bf16
  return static_cast<size_t>(n_pairs) * (inter + hidden) * 2 + 256;
}

// Argument checks shared by ma_moe_grouped and ma_moe_grouped_noalloc.
static int grouped_check(const void* x, int64_t ldx, int64_t tokens, int64_t top_k,
                         int alpha_dtype, int64_t n_experts, int64_t hidden, int64_t inter,
                         const char* what) {
  if (tokens < 0 || top_k < 1 || n_experts < 1 || n_experts > 1024)
    return fail(MA_EVALUE, "%s: bad sizes", what);
  if (hidden % 256 || inter % 256)
    return fail(MA_EVALUE, "%s: hidden (%lld) and intermediate (%lld) must be multiples of 256", what,
                (long long)hidden, (long long)inter);
  if (alpha_dtype != MA_BF16 && alpha_dtype != MA_F32)
    return fail(MA_ETYPE, "%s: row_alpha must be bfloat16 or float32", what);
  if ((reinterpret_cast<uintptr_t>(x) & 15u) || (ldx % 8))
    return fail(MA_EVALUE, "%s: x rows must be 16-byte aligned", what);
  return MA_OK;
}

// The launches of one grouped MoE call; workspace holds
// ma_grouped_workspace_bytes(tokens * top_k, inter, hidden) bytes.
static int grouped_launch(const void* x, int64_t ldx, const uint32_t* x_pairs, const float* x_corr,
                          int64_t tokens, int64_t top_k, const uint32_t* up_gate,
                          const void* up_gate_alpha, const uint32_t* down, const void* down_alpha,
                          int alpha_dtype, int64_t n_experts, int64_t hidden, int64_t inter,
                          const int32_t* offsets, const int32_t* pair_ids, const int32_t* inverse,
                          const float* topk_weight, const void* residual, int residual_dtype,
                          void* h_out, int64_t ldh, void* y, void* workspace, void* stream) {
  const int64_t n_pairs = tokens * top_k;
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint16_t* hp = static_cast<uint16_t*>(workspace);
  uint16_t* out = hp + n_pairs * inter;
  const int ne = static_cast<int>(n_experts);
  const auto* xb = static_cast<const uint16_t*>(x);
  auto* hb = static_cast<uint16_t*>(h_out);
  if (n_pairs <= kKsMaxPairsPerExpert * n_experts) {
    // decode: 16-pair tiles, K split over the waves of a workgroup
    const unsigned max_tiles = static_cast<unsigned>(n_pairs / 16 + n_experts);
    dim3 g1(static_cast<unsigned>(cdiv(inter, 32)), max_tiles);
    dim3 g2(static_cast<unsigned>(cdiv(hidden, 64)), max_tiles);
    // tile-resident forms: 16 rows (up + gate) / 32 rows per wave
    dim3 ge1(static_cast<unsigned>(cdiv(inter, 16 * kErWaves)), max_tiles);
    dim3 ge2(static_cast<unsigned>(cdiv(hidden, 32 * kErWaves)), max_tiles);
#define MA_GROUPED_KS(ADT)                                                                       \
  if (x_pairs && hidden == 16 * 16 * kErChunksUp)                                                \
    hipLaunchKernelGGL((k_grouped_swiglu_er<1, ADT, kErChunksUp, 1>), ge1, dim3(64 * kErWaves),  \
                       0, s, x_pairs, x_corr, top_k, up_gate, inter, up_gate_alpha, offsets,     \
                       pair_ids, ne, hp, hb, ldh);                                               \
  else if (x_pairs)                                                                              \
    hipLaunchKernelGGL((k_grouped_swiglu_ks<2, ADT, 8, true>), g1, dim3(512), 0, s, xb, ldx,     \
                       x_pairs, x_corr, top_k, up_gate, inter, hidden / 16, up_gate_alpha,      \
                       offsets, pair_ids, ne, hp, hb, ldh);                                      \
  else                                                                                           \
    hipLaunchKernelGGL((k_grouped_swiglu_ks<2, ADT, 8, false>), g1, dim3(512), 0, s, xb, ldx,    \
                       x_pairs, x_corr, top_k, up_gate, inter, hidden / 16, up_gate_alpha,      \
                       offsets, pair_ids, ne, hp, hb, ldh);                                      \
  if (inter == 16 * 16 * kErChunksDown)                                                          \
    hipLaunchKernelGGL((k_grouped_down_er<2, ADT, kErChunksDown>), ge2, dim3(64 * kErWaves), 0,  \
                       s, reinterpret_cast<const uint32_t*>(hp), down, hidden, down_alpha,       \
                       offsets, ne, out);                                                        \
  else                                                                                           \
    hipLaunchKernelGGL((k_grouped_down_ks<4, ADT, 8, 2>), g2, dim3(512), 0, s,                   \
                       reinterpret_cast<const uint32_t*>(hp), down, hidden, inter / 16,          \
                       down_alpha, offsets, ne, out);
    if (alpha_dtype == MA_BF16) { MA_GROUPED_KS(MA_BF16) } else { MA_GROUPED_KS(MA_F32) }
#undef MA_GROUPED_KS
  } else {
  const int nb = grouped_nb(n_pairs, n_experts);
  const int nt = 16 * nb;
  const unsigned max_tiles = static_cast<unsigned>(n_pairs / nt + n_experts);
  dim3 g1(static_cast<unsigned>(cdiv(inter, 128)), max_tiles);
  dim3 g2(static_cast<unsigned>(cdiv(hidden, 256)), max_tiles);
#define MA_GROUPED(NB, ADT)                                                                      \
  hipLaunchKernelGGL((k_grouped_swiglu<NB, ADT>), g1, dim3(256), 0, s, xb, ldx, top_k, up_gate,  \
                     inter, hidden / 16, up_gate_alpha, offsets, pair_ids, ne, hp, hb, ldh);     \
  hipLaunchKernelGGL((k_grouped_down<NB, ADT>), g2, dim3(256), 0, s,                             \
                     reinterpret_cast<const uint32_t*>(hp), down, hidden, inter / 16, down_alpha, \
                     offsets, ne, out);
  if (alpha_dtype == MA_BF16) {
    if (nb == 4) { MA_GROUPED(4, MA_BF16) } else if (nb == 2) { MA_GROUPED(2, MA_BF16) } else { MA_GROUPED(1, MA_BF16) }
  } else {
    if (nb == 4) { MA_GROUPED(4, MA_F32) } else if (nb == 2) { MA_GROUPED(2, MA_F32) } else { MA_GROUPED(1, MA_F32) }
  }
#undef MA_GROUPED
  }
  if (y) {
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (top_k <= 8 && (!residual || (residual_dtype == MA_BF16 && a16(residual))) && a16(y) &&
        hidden % 8 == 0) {
      dim3 g3(static_cast<unsigned>(cdiv(hidden, 256 * 8)), static_cast<unsigned>(tokens));
      hipLaunchKernelGGL(k_combine8<8>, g3, dim3(256), 0, s, out, inverse, topk_weight,
                         static_cast<int>(top_k), hidden, static_cast<const uint16_t*>(residual),
                         static_cast<uint16_t*>(y));
    } else {
      dim3 g3(static_cast<unsigned>(cdiv(hidden, 512)), static_cast<unsigned>(tokens));
      hipLaunchKernelGGL(k_combine, g3, dim3(256), 0, s, out, inverse, topk_weight, top_k, hidden,
                         residual, residual_dtype, static_cast<uint16_t*>(y));
    }
  }
  return check_launch("moe_grouped");
}

extern "C" int ma_moe_grouped(const void* x, int64_t ldx, const uint32_t* x_pairs,
                              const float* x_corr, int64_t tokens, int64_t top_k,
                              const uint32_t* up_gate, const void* up_gate_alpha,
                              const uint32_t* down, const void* down_alpha, int alpha_dtype,
                              int64_t n_experts, int64_t hidden, int64_t inter,
                              const int32_t* offsets, const int32_t* pair_ids,
                              const int32_t* inverse, const float* topk_weight,
                              const void* residual, int residual_dtype, void* h_out, int64_t ldh,
                              void* y, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = grouped_check(x, ldx, tokens, top_k, alpha_dtype, n_experts, hidden, inter, "moe_grouped"))
    return rc;
  const int64_t n_pairs = tokens * top_k;
  if (n_pairs == 0) return MA_OK;
  if (!workspace || workspace_bytes < ma_grouped_workspace_bytes(n_pairs, inter, hidden))
    return fail(MA_EVALUE, "moe_grouped: workspace too small");
  return grouped_launch(x, ldx, x_pairs, x_corr, tokens, top_k, up_gate, up_gate_alpha, down,
                        down_alpha, alpha_dtype, n_experts, hidden, inter, offsets, pair_ids,
                        inverse, topk_weight, residual, residual_dtype, h_out, ldh, y, workspace,
                        stream);
}

// ---------------------------------------------------------------------------
// ma_moe_grouped without a workspace argument and without any allocation:
// the staging buffer is this file-scope device array, one per GPU, held until
// the process ends.  In host code `scratch` names a host-side stand-in, so
// kernels get the device address from hipGetSymbolAddress, taken once per
// device on that device's first call.
// ---------------------------------------------------------------------------
constexpr size_t kGroupedScratchBytes = size_t{16} << 20;
static __device__ __align__(256) uint8_t scratch[kGroupedScratchBytes];

static void* grouped_scratch_ptr() {
  static std::mutex mu;
  static void* ptrs[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    fail(MA_ERUNTIME, "moe_grouped_noalloc: no current HIP device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
      fail(MA_ERUNTIME, "moe_grouped_noalloc: device address of the scratch array unavailable");
      return nullptr;
    }
    ptrs[dev] = p;
  }
  return ptrs[dev];
}

extern "C" size_t ma_moe_grouped_noalloc_max_bytes(void) { return kGroupedScratchBytes; }

extern "C" int ma_moe_grouped_noalloc(const void* x, int64_t ldx, const uint32_t* x_pairs,
                                      const float* x_corr, int64_t tokens, int64_t top_k,
                                      const uint32_t* up_gate, const void* up_gate_alpha,
                                      const uint32_t* down, const void* down_alpha,
                                      int alpha_dtype, int64_t n_experts, int64_t hidden,
                                      int64_t inter, const int32_t* offsets,
                                      const int32_t* pair_ids, const int32_t* inverse,
                                      const float* topk_weight, const void* residual,
                                      int residual_dtype, void* h_out, int64_t ldh, void* y,
                                      void* stream) {
  const char* what = "moe_grouped_noalloc";
  if (int rc = grouped_check(x, ldx, tokens, top_k, alpha_dtype, n_experts, hidden, inter, what))
    return rc;
  if (!y)
    return fail(MA_EVALUE, "%s: y is required (the per-pair outputs stay in the internal scratch)", what);
  const int64_t n_pairs = tokens * top_k;
  if (n_pairs == 0) return MA_OK;
  const size_t need = ma_grouped_workspace_bytes(n_pairs, inter, hidden);
  if (need > kGroupedScratchBytes)
    return fail(MA_EVALUE,
                "%s: %lld (token, expert) pairs need %zu bytes of staging; the built-in scratch holds %zu "
                "(use ma_moe_grouped with a workspace)",
                what, static_cast<long long>(n_pairs), need, kGroupedScratchBytes);
  void* ws = grouped_scratch_ptr();
  if (!ws) return MA_ERUNTIME;
  return grouped_launch(x, ldx, x_pairs, x_corr, tokens, top_k, up_gate, up_gate_alpha, down,
                        down_alpha, alpha_dtype, n_experts, hidden, inter, offsets, pair_ids,
                        inverse, topk_weight, residual, residual_dtype, h_out, ldh, y, ws, stream);
}
