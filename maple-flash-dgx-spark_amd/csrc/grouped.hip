// Grouped expert GEMMs on MFMA for batched decode and prefill (gfx950).
//
// After dispatch (pairs sorted by expert), every expert's tokens form a dense
// [tokens x K] operand, so the SwiGLU up+gate projection and the down
// projection become per-expert GEMMs: y = W_e (rows x K) . X_e^T (K x tokens).
//
// A operand (weights): each lane expands its own packed words with
// expand_word (common.h) into bf16x2 dwords of 1 + c/f -- exactly the dword
// order of the bf16 x' pairs, an (arbitrary but shared) permutation of K
// inside each word.  B operand (activations): x' = f * x pairs.  The MFMA then
// accumulates sum (f + c) x; subtracting C_t = sum (f + 1) x per token
// leaves sum (c - 1) x, the ternary product (float32 accumulation).
//
// v_mfma_f32_16x16x32_bf16 lane layout (checked on the device):
//   A: lane l holds row l%16, k 8(l/16)..+8;  B: col l%16, k 8(l/16)..+8;
//   C: lane l holds col l%16, rows 4(l/16)..+4.
//
// Two forms: decode batches (few pairs per expert: 16-pair tiles, K split
// over the waves, operands in registers) and prefill (128-pair x 256-row
// tiles with the x' operands staged in LDS).  Stage 1 computes h (each wave
// holds up rows and the matching gate rows, so SwiGLU is applied in
// registers), rounded to bf16 like the reference's x.dtype store
// (ternary_expert.py:441), in the x' pair layout the down stage reads and
// optionally in the plain [slot, I] layout.  Stage 2 writes each pair's down
// output rounded to bf16 (ternary_expert.py:208); a gather kernel then forms
// y[t] = sum_j w[t,j] out[pair(t,j)] (+ residual) in float32
// (fused_norm.py:83-96).
#include <mutex>

#include "mfma.h"

namespace ma {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));


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
constexpr int kErAhead = 2;  // weight chunks in flight per wave ahead of the MFMAs

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
  // weights of this wave's blocks, chunk by chunk, kErAhead chunks ahead of
  // their use: with every wave's whole share requested at once (16 KB), the
  // tile's x' loads queued behind the other workgroups' weight streams for
  // ~6 us before the first MFMA could start; a short pipeline keeps the
  // queues short, and the MFMAs run while the later chunks stream
  const uint32_t* rp[2 * BPW];
#pragma unroll
  for (int j = 0; j < 2 * BPW; ++j) {
    int64_t blk = b0 + (j % BPW);
    blk = blk < nblk ? blk : nblk - 1;
    rp[j] = we + ((j / BPW) * n_half + blk * 16 + r16) * NW + 4 * g;
  }
  u32x4v_t wq[2 * BPW][NCH];
#pragma unroll
  for (int c = 0; c < kErAhead && c < NCH; ++c)
#pragma unroll
    for (int j = 0; j < 2 * BPW; ++j) wq[j][c] = *reinterpret_cast<const u32x4v_t*>(rp[j] + 16 * c);
  MA_ISSUE_FENCE();
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
    if (c + kErAhead < NCH) {
#pragma unroll
      for (int j = 0; j < 2 * BPW; ++j)
        wq[j][c + kErAhead] = *reinterpret_cast<const u32x4v_t*>(rp[j] + 16 * (c + kErAhead));
    }
    MA_ISSUE_FENCE();
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
  // weights of this wave's blocks for all of K (a pipeline as in the SwiGLU
  // stage measured no faster here: K is only 3 chunks)
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
  static_assert(K == 8, "slot pairs");
  int64_t row[8];
  float wj[8];
  slot_pairs8(inverse, wts, t, topk, row, wj);
  if (i >= n) return;
  uint4 v[K], r = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
  for (int j = 0; j < K; ++j) v[j] = *reinterpret_cast<const uint4*>(out + row[j] * n + i);
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

// ---------------------------------------------------------------------------
// Prefill form (many pairs per expert): tiles of 128 pairs x 256 weight rows,
// eight waves (4 along the rows x 2 along the pairs, 64 x 64 each), K walked
// in steps of 8 words (128 codes).  The pairs' x' operands of a step (32 KB)
// are copied into LDS by the LDS DMA (global_load_lds_dwordx4: no staging
// registers), double-buffered: the next step's copy and weights are in flight
// during this step's MFMAs, one barrier per step.  That keeps a workgroup
// under 128 VGPRs and 70 KB of LDS, so two run on a CU.  x' pairs and the
// per-token correction are built once per token (k_gp_prep), so staging is a
// copy.  Each lane expands its own weight words in registers, half a word
// (the 4 operand dwords one MFMA takes) at a time: a lane group g takes
// words 2g and 2g+1 of a step, substep s (K = 32) the pairs 4(s & 1)..+3 of
// word 2g + (s >> 1) -- the same K permutation on both operands.  Tiles go to
// workgroups so that the row tiles of one pair tile share an XCD (workgroups
// are placed on the 8 XCDs round-robin), which keeps that tile's x' in one L2.
// ---------------------------------------------------------------------------
namespace gp {
constexpr int kTok = 128;    // pairs per tile
constexpr int kRows = 256;   // weight rows per tile (SwiGLU: 128 up + the 128 matching gate rows)
constexpr int kWords = 8;    // packed words of K per step
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kXcds = 8;
// One step's x' in LDS: 16-byte slot p * 16 + (c ^ (p % 16)) holds chunk c
// (word c / 2, half c % 2) of pair p -- each pair's 256 bytes in one run, the
// chunks XOR-swizzled so that the B reads (16 pairs of one chunk) hit 16
// different bank groups; the DMA fills slots in order, so each copy's source
// is chosen to match.
constexpr int kXsDwords = kTok * 2 * kWords * 4;  // one buffer (32 KB)
// After the K loop the same LDS stages the output tile for coalesced stores:
// h as [pair][128 outputs] (rows padded to 136 bf16), the down outputs as
// [pair][256 rows] (rows padded to 264 bf16); the padding keeps the 16 pair
// columns of a lane group on different banks and every row 16-byte aligned.
constexpr int kHRow = 136, kORow = 264;
// Buffer A also stages the output tile: all of h (128 x 136 bf16), or half of
// the down tile's pairs at a time (64 x 264 bf16).
constexpr int kXaDwords = (kTok * kHRow / 2 > kTok / 2 * kORow / 2) ? kTok * kHRow / 2 : kTok / 2 * kORow / 2;
static_assert(kXaDwords >= kXsDwords, "buffer A holds a step");
}  // namespace gp

// x' pairs of every token once: xp [T, nwords * 8] (word w: pair j =
// (f_j x[16w+j], f_j x[16w+j+8])) and xc[t] = sum (f + 1) x over the row, in
// a fixed order.
__global__ __launch_bounds__(128) void k_gp_prep(const uint16_t* __restrict__ x, int64_t ldx,
                                                 int64_t nwords, uint32_t* __restrict__ xp,
                                                 float* __restrict__ xc) {
  __shared__ float red[2];
  const int64_t t = blockIdx.x;
  const int tid = threadIdx.x;
  float c = 0.f;
  for (int64_t wd = tid; wd < nwords; wd += 128) {
    const uint4* src = reinterpret_cast<const uint4*>(x + t * ldx + wd * 16);
    uint32_t pr[8];
    c += x16_to_pairs(src[0], src[1], pr);
    uint4* dst = reinterpret_cast<uint4*>(xp + (t * nwords + wd) * 8);
    dst[0] = make_uint4(pr[0], pr[1], pr[2], pr[3]);
    dst[1] = make_uint4(pr[4], pr[5], pr[6], pr[7]);
  }
  c = group_sum<64>(c);
  if ((tid & 63) == 0) red[tid >> 6] = c;
  __syncthreads();
  if (tid == 0) xc[t] = red[0] + red[1];
}

// Tile of workgroup L (workgroups go to the 8 XCDs round-robin: L on XCD
// L % 8, the XCD's slot L / 8).  The M pair tiles (experts in order, each
// expert's tiles consecutive) are cut into 8 contiguous ranges of ceil(M / 8),
// one per XCD, and an XCD's slots walk its range pair tile by pair tile, the
// row tiles of a pair tile together: so an expert's pair tiles run on one
// XCD (two at a range boundary) and read its codes through one L2, and the
// row tiles of a pair tile share its x'.  M is counted from the dispatch
// offsets (the grid is sized for the most tiles T k / 128 + E).  Returns
// false for the workgroups past the XCD's range.
__device__ __forceinline__ bool gp_tile(const int32_t* __restrict__ offsets, int n_exp, int n_rtiles, int& mtile,
                                        int& rtile) {
  const int lane = threadIdx.x & 63;
  int m = 0;  // pair tiles of every expert
  for (int base = 0; base < n_exp; base += 64) {
    const int ee = base + lane;
    m += ee < n_exp ? (offsets[ee + 1] - offsets[ee] + gp::kTok - 1) / gp::kTok : 0;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m += __shfl_xor(m, off, 64);
  m = __builtin_amdgcn_readfirstlane(m);
  const int L = blockIdx.x, xcd = L % gp::kXcds, slot = L / gp::kXcds;
  const int per = (m + gp::kXcds - 1) / gp::kXcds;
  const int local = slot / n_rtiles;
  mtile = xcd * per + local;
  rtile = slot % n_rtiles;
  return local < per && mtile < m;
}

// One K step of a wave: 4 row blocks x 4 pair blocks x 4 substeps of
// v_mfma_f32_16x16x32_bf16.  wq: the lane's two words of its 4 row blocks;
// xsb: the step's x' in the swizzled layout (pair col0 + 16 nb + r16 has
// p % 16 == r16).
__device__ __forceinline__ void gp_step(const uint2 (&wq)[4], const uint32_t* __restrict__ xsb,
                                        int g, int r16, int col0, f32x4_t (&acc)[4][4],
                                        const ExpandConsts& kc) {
#pragma unroll
  for (int ww = 0; ww < 2; ++ww) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int c = (2 * g + ww) * 2 + hh;
      uint4 b[4];
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        b[nb] = *reinterpret_cast<const uint4*>(xsb + ((col0 + nb * 16 + r16) * 16 + (c ^ r16)) * 4);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const uint4 a = expand_half(ww ? wq[mb].y : wq[mb].x, hh, kc);
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = mfma_bf16(a, b[nb], acc[mb][nb]);
      }
    }
  }
}

// A step's x' copies: 2048 slots of 16 B, 4 per thread; copy i of thread tid
// fills slot S = tid + 512 i (so each wave's copy i fills 64 consecutive
// slots, as the LDS DMA writes them) with chunk c = (S % 16) ^ (p % 16) of
// pair p = S / 16.  rows[p] is pair p's row in the uint32 array base (row
// length ld); src[i] is copy i's source at K word 0.
// The four offsets live in LDS (soff[thread], read back at each step): in
// registers they pushed the K loop past its 128 VGPRs, and the compiler
// reloaded a spilled value from scratch memory at every step.
struct GpDma {
  const uint32_t* base;  // the same in every lane
  const uint4* soff;     // LDS: soff[t].x .. .w = thread t's copy i source at K word 0, in uint32 from base
                         // (< 2^32: checked by the host)
};
__device__ __forceinline__ GpDma gp_dma_sources(const uint32_t* base, int64_t ld, const int32_t* rows,
                                                uint4* soff) {
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int S = threadIdx.x + gp::kThreads * i, p = S / 16, c = (S % 16) ^ (p % 16);
    o[i] = static_cast<uint32_t>(static_cast<int64_t>(rows[p]) * ld + (c >> 1) * 8 + 4 * (c & 1));
  }
  soff[threadIdx.x] = make_uint4(o[0], o[1], o[2], o[3]);  // read back only by this thread
  return GpDma{base, soff};
}
typedef __attribute__((address_space(3))) void* lds_void_t;
// s_waitcnt immediate (gfx9 encoding): vmcnt(4), expcnt and lgkmcnt left open.
constexpr int kVmcnt4 = 0x4 | (0x7 << 4) | (0xF << 8);
// vmcnt(4) and lgkmcnt(0), expcnt left open.
constexpr int kVmcnt4Lgkm0 = 0x4 | (0x7 << 4);

// The copies of the step at K word k0 into the LDS buffer xsb (in flight
// until the issuing wave's vector memory counter drains).
__device__ __forceinline__ void gp_dma(const GpDma& d, int64_t k0, uint32_t* xsb) {
  const int wv = threadIdx.x >> 6;
  const uint4 o4 = d.soff[threadIdx.x];
  const uint32_t off[4] = {o4.x, o4.y, o4.z, o4.w};
#pragma unroll
  for (int i = 0; i < 4; ++i)
    __builtin_amdgcn_global_load_lds(d.base + off[i] + k0 * 8,
                                     (lds_void_t)(xsb + 4 * (64 * wv + gp::kThreads * i)), 16, 0, 0);
}

// One step of the K loop: take this step's weights out of w, issue the next
// step's x' copies into ``nxt`` (if there is a next step) and its weights
// into w, then this step's MFMAs on ``cur``, then wait for the copies and
// meet at the barrier.  The weights move to their own registers at the top,
// after the wait that covers their loads: a copy at the end of the step
// would have to wait for the loads just issued, in the middle of the step.
__device__ __forceinline__ void gp_kstep(const uint32_t* rp, const int64_t (&moff)[4], int64_t k0, int64_t nwk,
                                         const GpDma& d, const uint32_t* cur, uint32_t* nxt,
                                         uint2 (&w)[4], int g, int r16, int col0, f32x4_t (&acc)[4][4],
                                         const ExpandConsts& kc) {
  using namespace gp;
  const int64_t kn = k0 + kWords < nwk ? k0 + kWords : k0;
  // This step's weights (loaded during the last step) are in: nothing else
  // is outstanding, so the copies and loads below are all this wave has in
  // flight during the MFMAs.
  __builtin_amdgcn_s_waitcnt(0);
  MA_ISSUE_FENCE();
  uint2 wq[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) wq[mb] = w[mb];
  MA_ISSUE_FENCE();
  if (k0 + kWords < nwk) gp_dma(d, kn, nxt);
  MA_ISSUE_FENCE();  // the copies are issued before the weights
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) w[mb] = *reinterpret_cast<const uint2*>(rp + moff[mb] + kn);
  MA_ISSUE_FENCE();  // the next step's loads go out before this step's MFMAs
  gp_step(wq, cur, g, r16, col0, acc, kc);
  // This wave's copies have landed: at most the 4 weight loads issued after
  // them are outstanding (vector memory completes in issue order); those
  // are waited for where the next step uses them.
  __builtin_amdgcn_s_waitcnt(kVmcnt4Lgkm0);
  // The next buffer is in and this one is free to refill once every wave is
  // here.  A plain barrier: __syncthreads' fence would also wait for the
  // weight loads just issued (it drains every outstanding write to LDS, and
  // the LDS DMA counts in the same counter as those loads).
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  // Register copies the loop needs between steps stay here, after the
  // barrier, where the next step's first wait covers their loads.
  MA_ISSUE_FENCE();
}

// The K loop shared by both stages: acc += W x x', the lane's weight row of
// block mb at rp + moff[mb] (moff the same in every lane; nwk words), the
// pairs' x' rows in d; weights one step ahead in registers, x' one step ahead
// by DMA into the other LDS buffer.  The two buffers are distinct arrays and
// the loop is unrolled by two, so the compiler sees that a step's LDS reads
// and the copies in flight into the other buffer do not overlap (it would
// otherwise wait for the copies before the reads).
__device__ __forceinline__ void gp_kloop(const uint32_t* rp, const int64_t (&moff)[4], int64_t nwk, const GpDma& d,
                                         uint32_t* xa, uint32_t* xb, int g, int r16, int col0,
                                         f32x4_t (&acc)[4][4]) {
  using namespace gp;
  const ExpandConsts kc;
  uint2 wq[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) wq[mb] = *reinterpret_cast<const uint2*>(rp + moff[mb]);
  gp_dma(d, 0, xa);
  __builtin_amdgcn_s_waitcnt(0);  // this wave's copies have landed
  __syncthreads();                // and every other wave's
  for (int64_t k0 = 0; k0 < nwk; k0 += 2 * kWords) {
    gp_kstep(rp, moff, k0, nwk, d, xa, xb, wq, g, r16, col0, acc, kc);
    if (k0 + kWords < nwk) gp_kstep(rp, moff, k0 + kWords, nwk, d, xb, xa, wq, g, r16, col0, acc, kc);
  }
}

// SwiGLU stage: h = SwiGLU(up, gate) of 128 outputs (rows [o, o+128) of the
// up half and the matching gate rows) for a tile of 128 pairs of expert e,
// rounded to bf16 and written in the x' pair layout the down stage reads (hp)
// and optionally in slot order (h); hcorr[pos * n_rtiles + rtile] gets the
// tile's part of the down stage's correction sum (f + 1) h.
template <int ADT>
__global__ __launch_bounds__(gp::kThreads) __attribute__((amdgpu_waves_per_eu(4, 4))) void k_gp_swiglu(
    const uint32_t* __restrict__ xp, const float* __restrict__ xc, int64_t topk,
    const uint32_t* __restrict__ w, int64_t n_half, int64_t nwords,
    const void* __restrict__ alpha, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ pair_ids, int n_exp, uint16_t* __restrict__ hp,
    float* __restrict__ hcorr, uint16_t* __restrict__ h, int64_t ldh) {
  using namespace gp;
  __shared__ __align__(16) uint32_t xa[kXaDwords];
  __shared__ __align__(16) uint32_t xb[kXsDwords];
  __shared__ float cst[kTok], hcp[4][kTok];
  __shared__ int32_t tokrow[kTok], pid[kTok];
  __shared__ uint4 dsoff[kThreads];
  const int n_rtiles = static_cast<int>((n_half + kRows / 2 - 1) / (kRows / 2));
  int mtile, rtile;
  if (!gp_tile(offsets, n_exp, n_rtiles, mtile, rtile)) return;
  int e, pos0, np;
  if (!decode_tile(offsets, n_exp, mtile, kTok, e, pos0, np)) return;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wr = wv & 3, wm = wv >> 2, r16 = lane & 15, g = lane >> 4;
  if (tid < kTok) {
    const int p = tid < np ? pair_ids[pos0 + tid] : -1;
    pid[tid] = p;
    const int t = p >= 0 ? static_cast<int>(p / topk) : 0;
    tokrow[tid] = t;
    cst[tid] = p >= 0 ? xc[t] : 0.f;
  }
  const int64_t o0 = static_cast<int64_t>(rtile) * (kRows / 2) + wr * 32;  // this wave's first output
  const uint32_t* we = w + static_cast<int64_t>(e) * 2 * n_half * nwords;
  // (n_half % 128 == 0: every row of the tile exists)
  const uint32_t* rp = we + (o0 + r16) * nwords + 2 * g;
  int64_t moff[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) moff[mb] = (16 * (mb & 1) + (mb >> 1) * n_half) * nwords;
  __syncthreads();  // tokrow
  const GpDma xsrc = gp_dma_sources(xp, nwords * 8, tokrow, dsoff);
  f32x4_t acc[4][4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  gp_kloop(rp, moff, nwords, xsrc, xa, xb, g, r16, wm * 64, acc);
  // Epilogue: lane (r16, g) of row block mb holds rows 4g..4g+3 of the block
  // for pair column wm*64 + nb*16 + r16.  h goes to LDS in the x' pair layout
  // of its 8 words (the loop's last barrier has freed the LDS), then out in
  // 16-byte pieces, each pair's 256 bytes contiguous.
  // Output i = o0 + 16 mb + 4 g + r (< n_half: n_half % 128 == 0) sits at
  // position 4 g + r of its 16-output word, i.e. pair j = (4 g + r) & 7 (so
  // pair_scale(j) = pair_scale(r)), half g >> 1, word 2 wr + mb of the tile.
  uint16_t* hst = reinterpret_cast<uint16_t*>(xa);
  const int64_t otile = static_cast<int64_t>(rtile) * (kRows / 2);
  const int64_t abase = static_cast<int64_t>(e) * 2 * n_half;
  float au[2][4], ag[2][4];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t i = o0 + 16 * mb + 4 * g + r;
      au[mb][r] = ld_t<ADT>(alpha, abase + i);
      ag[mb][r] = ld_t<ADT>(alpha, abase + n_half + i);
    }
  float cc[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) cc[nb] = cst[wm * 64 + nb * 16 + r16];
  const int hbase = (2 * wr * 8) * 2 + (g >> 1);
  float hcl[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = (4 * g + r) & 7;
      const float f = pair_scale(r);
      const int hoff = hbase + (mb * 8 + j) * 2;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const int col = wm * 64 + nb * 16 + r16;
        const float up = au[mb][r] * (acc[mb][nb][r] - cc[nb]);
        const float gt = ag[mb][r] * (acc[mb + 2][nb][r] - cc[nb]);
        const uint16_t hb = f32_to_bf16(swiglu_act(up, gt));
        const float hv = bf16_to_f32(hb);
        hst[col * kHRow + hoff] = static_cast<uint16_t>(bf16_bits_exact(hv * f));  // exact: power-of-two scale
        // (+0.0 for the pad columns: hcl starts at +0.0, so no sum changes)
        hcl[nb] += col < np ? (f + 1.0f) * hv : 0.0f;
        if (h) {
          if (col < np) h[static_cast<int64_t>(pid[col]) * ldh + o0 + 16 * mb + 4 * g + r] = hb;
        }
      }
    }
  }
  // the tile's correction part per pair: lane groups, then row waves, in order
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    float v = hcl[nb];
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    if (g == 0) hcp[wr][wm * 64 + nb * 16 + r16] = v;
  }
  __syncthreads();
  if (tid < np) {
    const float v = ((hcp[0][tid] + hcp[1][tid]) + hcp[2][tid]) + hcp[3][tid];
    hcorr[static_cast<int64_t>(pos0 + tid) * n_rtiles + rtile] = v;
  }
  // the tile's h (n_half % 128 == 0: whole words), 16 B per copy
#pragma unroll
  for (int k = 0; k < kTok * 16 / kThreads; ++k) {
    const int c = tid + kThreads * k, col = c / 16, part = c % 16;
    if (col < np)
      *reinterpret_cast<uint4*>(hp + static_cast<int64_t>(pos0 + col) * n_half + otile + part * 8) =
          *reinterpret_cast<const uint4*>(hst + col * kHRow + part * 8);
  }
}

// Down stage: out[pos, n] = bf16(alpha[e, n] * sum_k (c - 1) h) for a tile of
// 128 pairs and 256 output rows; the correction is the sum of the SwiGLU
// stage's n_ctiles parts, added in tile order.
template <int ADT>
__global__ __launch_bounds__(gp::kThreads) __attribute__((amdgpu_waves_per_eu(4, 4))) void k_gp_down(
    const uint32_t* __restrict__ hp, const float* __restrict__ hcorr, int n_ctiles,
    const uint32_t* __restrict__ w, int64_t n_out, int64_t nwk, const void* __restrict__ alpha,
    const int32_t* __restrict__ offsets, int n_exp, uint16_t* __restrict__ out) {
  using namespace gp;
  __shared__ __align__(16) uint32_t xa[kXaDwords];
  __shared__ __align__(16) uint32_t xb[kXsDwords];
  __shared__ float cst[kTok];
  __shared__ int32_t prow[kTok];
  __shared__ uint4 dsoff[kThreads];
  const int n_rtiles = static_cast<int>((n_out + kRows - 1) / kRows);
  int mtile, rtile;
  if (!gp_tile(offsets, n_exp, n_rtiles, mtile, rtile)) return;
  int e, pos0, np;
  if (!decode_tile(offsets, n_exp, mtile, kTok, e, pos0, np)) return;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wr = wv & 3, wm = wv >> 2, r16 = lane & 15, g = lane >> 4;
  if (tid < kTok) {
    float c = 0.f;
    if (tid < np)
      for (int ct = 0; ct < n_ctiles; ++ct) c += hcorr[static_cast<int64_t>(pos0 + tid) * n_ctiles + ct];
    cst[tid] = c;
    prow[tid] = pos0 + (tid < np ? tid : np - 1);
  }
  const int64_t n0 = static_cast<int64_t>(rtile) * kRows + wr * 64;
  const uint32_t* we = w + static_cast<int64_t>(e) * n_out * nwk;
  // (n_out % 256 == 0: every row of the tile exists)
  const uint32_t* rp = we + (n0 + r16) * nwk + 2 * g;
  int64_t moff[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) moff[mb] = 16 * mb * nwk;
  __syncthreads();  // prow
  const GpDma xsrc = gp_dma_sources(hp, nwk * 8, prow, dsoff);
  f32x4_t acc[4][4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  gp_kloop(rp, moff, nwk, xsrc, xa, xb, g, r16, wm * 64, acc);
  // The tile goes out through LDS buffer A as [pair][256 rows], half of the
  // pairs at a time (the waves holding them write, then every thread copies
  // them out in 16-byte pieces, each pair's 512 bytes contiguous; n_out % 256
  // == 0).  The loop's last barrier has freed the buffer.
  uint2 v[4][4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    const int64_t n = n0 + 16 * mb + 4 * g;
    float a[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) a[r] = ld_t<ADT>(alpha, static_cast<int64_t>(e) * n_out + (n + r < n_out ? n + r : n_out - 1));
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const float c = cst[wm * 64 + nb * 16 + r16];
      v[mb][nb].x = pack_bf16x2_rn(a[0] * (acc[mb][nb][0] - c), a[1] * (acc[mb][nb][1] - c));
      v[mb][nb].y = pack_bf16x2_rn(a[2] * (acc[mb][nb][2] - c), a[3] * (acc[mb][nb][3] - c));
    }
  }
  uint16_t* ost = reinterpret_cast<uint16_t*>(xa);
  const int64_t ntile0 = static_cast<int64_t>(rtile) * kRows;
  for (int half = 0; half < 2; ++half) {
    if (wm == half) {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
          *reinterpret_cast<uint2*>(ost + (nb * 16 + r16) * kORow + wr * 64 + 16 * mb + 4 * g) = v[mb][nb];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kTok / 2 * 32 / kThreads; ++k) {
      const int c = tid + kThreads * k, colh = c / 32, part = c % 32, col = half * (kTok / 2) + colh;
      if (col < np)
        *reinterpret_cast<uint4*>(out + static_cast<int64_t>(pos0 + col) * n_out + ntile0 + part * 8) =
            *reinterpret_cast<const uint4*>(ost + colh * kORow + part * 8);
    }
    __syncthreads();  // the buffer is free for the next half
  }
}

}  // namespace ma

using namespace ma;

// Up to this many pairs per expert on average (decode batches) the K-split
// kernels run; above it (prefill) the LDS-staged tiles of up to 64 pairs.
constexpr int64_t kKsMaxPairsPerExpert = 16;

static size_t align256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

// Workspace of one call: pair-format h [P, inter] bf16, per-pair down outputs
// [P, hidden] bf16; in the prefill form also the x' pairs of the tokens
// [T, hidden / 2] uint32, their corrections [T] float32 and the SwiGLU tiles'
// correction parts [P, inter / 128] float32.
static bool grouped_prefill_form(int64_t n_pairs, int64_t n_experts) {
  return n_pairs > kKsMaxPairsPerExpert * n_experts;
}
static size_t grouped_bytes(int64_t n_pairs, int64_t tokens, int64_t inter, int64_t hidden, bool prefill) {
  size_t b = align256(static_cast<size_t>(n_pairs) * inter * 2) + align256(static_cast<size_t>(n_pairs) * hidden * 2);
  if (prefill)
    b += align256(static_cast<size_t>(tokens) * hidden * 2) + align256(static_cast<size_t>(tokens) * 4) +
         align256(static_cast<size_t>(n_pairs) * cdiv(inter, gp::kRows / 2) * 4);
  return b;
}

extern "C" size_t ma_grouped_workspace_bytes(int64_t n_pairs, int64_t inter, int64_t hidden) {
  // an upper bound over both forms (tokens <= pairs)
  return grouped_bytes(n_pairs, n_pairs, inter, hidden, true);
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
  char* wsb = static_cast<char*>(workspace);
  uint16_t* hp = reinterpret_cast<uint16_t*>(wsb);
  uint16_t* out = reinterpret_cast<uint16_t*>(wsb + align256(static_cast<size_t>(n_pairs) * inter * 2));
  const int ne = static_cast<int>(n_experts);
  const auto* xb = static_cast<const uint16_t*>(x);
  auto* hb = static_cast<uint16_t*>(h_out);
  if (!grouped_prefill_form(n_pairs, n_experts)) {
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
    // prefill: the tokens' x' pairs once (or those of ma_moe_route), then
    // tiles of 128 pairs x 256 weight rows.  The tiles' copy sources are
    // 32-bit uint32 offsets into x' and h.
    if (static_cast<uint64_t>(tokens) * hidden / 2 >= (uint64_t{1} << 32) ||
        static_cast<uint64_t>(n_pairs) * inter / 2 >= (uint64_t{1} << 32))
      return fail(MA_EVALUE, "moe_grouped: %lld tokens x hidden %lld (or their pairs x intermediate %lld) "
                  "exceed the 16 GiB the batched kernels address; split the batch",
                  (long long)tokens, (long long)hidden, (long long)inter);
    char* p = reinterpret_cast<char*>(out) + align256(static_cast<size_t>(n_pairs) * hidden * 2);
    const uint32_t* xpp = x_pairs;
    const float* xcc = x_corr;
    if (!x_pairs) {
      uint32_t* xw = reinterpret_cast<uint32_t*>(p);
      float* cw = reinterpret_cast<float*>(p + align256(static_cast<size_t>(tokens) * hidden * 2));
      hipLaunchKernelGGL(k_gp_prep, dim3(static_cast<unsigned>(tokens)), dim3(128), 0, s, xb, ldx, hidden / 16, xw, cw);
      xpp = xw;
      xcc = cw;
    }
    float* hcorr = reinterpret_cast<float*>(p + align256(static_cast<size_t>(tokens) * hidden * 2) +
                                            align256(static_cast<size_t>(tokens) * 4));
    const int64_t mtiles = cdiv(n_pairs, gp::kTok) + n_experts;  // an upper bound
    const int64_t mt8 = cdiv(mtiles, gp::kXcds) * gp::kXcds;
    const int rt1 = static_cast<int>(cdiv(inter, gp::kRows / 2)), rt2 = static_cast<int>(cdiv(hidden, gp::kRows));
    const dim3 g1(static_cast<unsigned>(mt8 * rt1)), g2(static_cast<unsigned>(mt8 * rt2));
#define MA_GP(ADT)                                                                                 \
  hipLaunchKernelGGL((k_gp_swiglu<ADT>), g1, dim3(gp::kThreads), 0, s, xpp, xcc, top_k, up_gate, \
                     inter, hidden / 16, up_gate_alpha, offsets, pair_ids, ne, hp, hcorr, hb, ldh);  \
  hipLaunchKernelGGL((k_gp_down<ADT>), g2, dim3(gp::kThreads), 0, s,                              \
                     reinterpret_cast<const uint32_t*>(hp), hcorr, rt1, down, hidden, inter / 16, \
                     down_alpha, offsets, ne, out);
    if (alpha_dtype == MA_BF16) {
      MA_GP(MA_BF16)
    } else {
      MA_GP(MA_F32)
    }
#undef MA_GP
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
  if (!workspace || workspace_bytes < grouped_bytes(n_pairs, tokens, inter, hidden,
                                                    grouped_prefill_form(n_pairs, n_experts)))
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
  const size_t need = grouped_bytes(n_pairs, tokens, inter, hidden, grouped_prefill_form(n_pairs, n_experts));
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
