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
#include "common.h"

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
  __shared__ float cst[NT];
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
      atomicAdd(&cst[col], c);
    }
    __syncthreads();
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
  __shared__ float cst[NT];
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
      atomicAdd(&cst[col], pairs_cst(pr));
    }
    __syncthreads();
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

}  // namespace ma

using namespace ma;

static int grouped_nb(int64_t n_pairs, int64_t n_exp) {
  const int64_t per = n_pairs / (n_exp > 0 ? n_exp : 1);
  return per >= 48 ? 4 : (per >= 24 ? 2 : 1);
}

extern "C" size_t ma_grouped_workspace_bytes(int64_t n_pairs, int64_t inter, int64_t hidden) {
  // pair-format h [P, inter] bf16 + per-pair down outputs [P, hidden] bf16
  return static_cast<size_t>(n_pairs) * (inter + hidden) * 2 + 256;
}

extern "C" int ma_moe_grouped(const void* x, int64_t ldx, int64_t tokens, int64_t top_k,
                              const uint32_t* up_gate, const void* up_gate_alpha,
                              const uint32_t* down, const void* down_alpha, int alpha_dtype,
                              int64_t n_experts, int64_t hidden, int64_t inter,
                              const int32_t* offsets, const int32_t* pair_ids,
                              const int32_t* inverse, const float* topk_weight,
                              const void* residual, int residual_dtype, void* h_out, int64_t ldh,
                              void* y, void* workspace, size_t workspace_bytes, void* stream) {
  if (tokens < 0 || top_k < 1 || n_experts < 1 || n_experts > 1024)
    return fail(MA_EVALUE, "moe_grouped: bad sizes");
  if (hidden % 256 || inter % 256)
    return fail(MA_EVALUE, "moe_grouped: hidden (%lld) and intermediate (%lld) must be multiples of 256",
                (long long)hidden, (long long)inter);
  if (alpha_dtype != MA_BF16 && alpha_dtype != MA_F32)
    return fail(MA_ETYPE, "moe_grouped: row_alpha must be bfloat16 or float32");
  if ((reinterpret_cast<uintptr_t>(x) & 15u) || (ldx % 8))
    return fail(MA_EVALUE, "moe_grouped: x rows must be 16-byte aligned");
  const int64_t n_pairs = tokens * top_k;
  if (n_pairs == 0) return MA_OK;
  if (!workspace || workspace_bytes < ma_grouped_workspace_bytes(n_pairs, inter, hidden))
    return fail(MA_EVALUE, "moe_grouped: workspace too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint16_t* hp = static_cast<uint16_t*>(workspace);
  uint16_t* out = hp + n_pairs * inter;
  const int nb = grouped_nb(n_pairs, n_experts);
  const int nt = 16 * nb;
  const unsigned max_tiles = static_cast<unsigned>(n_pairs / nt + n_experts);
  const int ne = static_cast<int>(n_experts);
  dim3 g1(static_cast<unsigned>(cdiv(inter, 128)), max_tiles);
  dim3 g2(static_cast<unsigned>(cdiv(hidden, 256)), max_tiles);
  const auto* xb = static_cast<const uint16_t*>(x);
  auto* hb = static_cast<uint16_t*>(h_out);
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
  if (y) {
    dim3 g3(static_cast<unsigned>(cdiv(hidden, 512)), static_cast<unsigned>(tokens));
    hipLaunchKernelGGL(k_combine, g3, dim3(256), 0, s, out, inverse, topk_weight, top_k, hidden,
                       residual, residual_dtype, static_cast<uint16_t*>(y));
  }
  return check_launch("moe_grouped");
}
