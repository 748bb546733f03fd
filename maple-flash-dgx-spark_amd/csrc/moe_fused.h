// Shared pieces of the one-launch MoE layer kernels (moe_fused.hip: one grid
// barrier between SwiGLU and down; moe_xcd.hip: the work split by XCD): the
// workspace layout and the optional next-projection tail.
#pragma once

#include "grid_sync.h"
#include "ternary_engine.h"
#include "tgemv_fast.h"

namespace ma {

// Workspace layout (256-byte lines of uint32 words; every counter and flag has
// a line of its own so that arrivals and polls on different ones do not meet):
//   line 0, word 2     error (1 = a wait timed out)
//   lines 1 .. 16      h barrier: group arrival counters (line 17 unused)
//   lines 18 .. 33     group flags, all holding the number of barriers
//                      passed on this workspace once a barrier is over
//   lines 34 .. 49     y barrier (calls with a next projection): group
//                      arrival counters (line 50 unused)
//   [16 KB, 48 KB)     grid kernel: router logits, one tagged 64-bit word
//                      (tag << 32 | float bits) per expert every 128 bytes
//   [48 KB, 64 KB)     grid kernel: h, bf16 [TK * I]
//   [64 KB, 96 KB)     XCD kernel: each workgroup's call count (one uint32
//                      every 128 bytes, written only by its workgroup)
//   [96 KB, 128 KB)    XCD kernel: one 4 KB region per XCD, touched only by
//                      that XCD's workgroups: 64 tagged router logits, then
//                      h of the XCD's slot as (tag16 << 16 | bf16) words
//   [128 KB, 256 KB)   XCD kernel: the weighted down outputs of every slot,
//                      tagged 64-bit words [8][H]
//   [256 KB, 320 KB)   XCD kernel with a next projection: one 8 KB region per
//                      XCD holding that XCD's copy of y, two bf16 values per
//                      tagged 64-bit word (tag << 32 | y[2m + 1] << 16 | y[2m])
//   [320 KB, 384 KB)   XCD kernel with the O projection in front: each XCD's
//                      copy of o, laid out as y
//   [384 KB, 400 KB)   XCD kernel built with MA_PHASE_STAMPS only: per
//                      workgroup 16 words, word i the 100 MHz real-time
//                      counter when the workgroup reached phase i, word 15
//                      its XCD (unused otherwise)
//   [400 KB, 401 KB)   XCD kernel: the layout check, one word per (XCD,
//                      workgroup number on it), written with the call's tag
//                      (XCD x's 32 words touched only by XCD x)
//   line 0, word 4     XCD kernel: 1 once a call found the workgroups not
//                      spread over the XCDs as the kernel assumes (sticky)
constexpr int kSubB = 1, kTopB = kSubB + kBarGroups, kFlags = kTopB + 1;
constexpr int kSubC = kFlags + kBarGroups, kTopC = kSubC + kBarGroups;
constexpr size_t kLogitOff = 16384;
constexpr int kLogitStride = 16;  // uint64 words between logits
constexpr size_t kMoeWsHeader = 49152;
constexpr size_t kXEpochOff = 65536, kXRegionOff = 98304, kXRegion = 4096, kXPartOff = 131072;
constexpr size_t kXYOff = kXPartOff + 8 * 2048 * 8, kXYRegion = 8192;
constexpr size_t kXOOff = kXYOff + 8 * kXYRegion;
constexpr size_t kXStampOff = kXOOff + 8 * kXYRegion;
constexpr int kXStampWords = 16;
constexpr size_t kXPresentOff = kXStampOff + 256 * kXStampWords * 4;
constexpr size_t kXWsBytes = kXPresentOff + 256 * 4;
constexpr int kXLayoutWord = 4;
static_assert(kTopC < static_cast<int>(kLogitOff / 256), "workspace lines");
static_assert(kLogitOff + 256 * kLogitStride * 8 <= kMoeWsHeader, "workspace logits");
static_assert(kMoeWsHeader + 8 * 768 * 2 <= kXEpochOff, "grid kernel h");
static_assert(kXEpochOff + 256 * 128 <= kXRegionOff && kXRegionOff + 8 * kXRegion <= kXPartOff, "XCD layout");
static_assert(2048 / 2 * 8 <= kXYRegion, "XCD y region");

// Phase stamps of the XCD kernel (builds with -DMA_PHASE_STAMPS, the
// library's stamped variant; a no-op otherwise): lane 0 of the calling wave
// writes the real-time counter into word i of its workgroup's stamp row.
#ifdef MA_PHASE_STAMPS
#define MA_XSTAMP(i) \
  do { if (lane == 0) stamps[i] = static_cast<uint32_t>(__builtin_amdgcn_s_memrealtime()); } while (0)
#else
#define MA_XSTAMP(i) do {} while (0)
#endif
// The same from a function given the stamp row (null: none), lane 0 of wave 0.
#ifdef MA_PHASE_STAMPS
#define MA_XSTAMP_AT(row, i)                                                           \
  do {                                                                                \
    if ((row) && tid == 0) (row)[i] = static_cast<uint32_t>(__builtin_amdgcn_s_memrealtime()); \
  } while (0)
#else
#define MA_XSTAMP_AT(row, i) do {} while (0)
#endif

// The RMS weights a thread of the next projection's x' build multiplies in:
// thread t < 2 NWH takes values j0 .. j0 + 3 and j0 + 8 .. j0 + 11 of word
// t / 2 (j0 = 4 (t & 1)); PIT passes of NTH threads.
template <int PIT>
struct NxRms {
  uint64_t wa[PIT][2], wb[PIT][2];
};
template <int NWH, int NTH, int PIT = (NWH * 2 + NTH - 1) / NTH>
__device__ __forceinline__ NxRms<PIT> load_nx_rms(const float* __restrict__ nx_rms, int tid) {
  NxRms<PIT> r;
#pragma unroll
  for (int k = 0; k < PIT; ++k) {
    const int t = tid + NTH * k < NWH * 2 ? tid + NTH * k : NWH * 2 - 1;
    const int w = t >> 1, j0 = 4 * (t & 1);
    r.wa[k][0] = reinterpret_cast<const uint64_t*>(nx_rms + w * 16 + j0)[0];
    r.wa[k][1] = reinterpret_cast<const uint64_t*>(nx_rms + w * 16 + j0)[1];
    r.wb[k][0] = reinterpret_cast<const uint64_t*>(nx_rms + w * 16 + j0 + 8)[0];
    r.wb[k][1] = reinterpret_cast<const uint64_t*>(nx_rms + w * 16 + j0 + 8)[1];
  }
  return r;
}

// Next projection, run by every workgroup of a one-launch layer once its rows
// of y are out: nx_out = ternary_gemv(y, nx_w, nx_alpha, rms_weight = nx_rms)
// -- reference kernels/ternary_gemv.py:110-146 -- with the standalone fast
// GEMV's per-lane arithmetic in the same order (so the same bits).  nxw / nxa
// hold this workgroup's rows (prefetched by the caller: row wg * nx_rq + p * W
// * RPIH + wv * RPIH + lane / LPRH).  y comes either from global memory, stored
// there with device-coherent stores, after a grid barrier (counters at kSubC,
// release flags at kFlags holding f_old), or (XY) from the XCD's own tagged
// copy yx (two values per 64-bit word, tag ytag), polled word by word.
// Returns true if a wait timed out.
template <int KWH, int LPRH, int W, int NXP, bool XY = false>
__device__ __forceinline__ bool next_projection(const uint16_t* __restrict__ y, const float* __restrict__ nx_rms,
                                                float nx_eps, int nx_rows, int nx_rq,
                                                uint16_t* __restrict__ nx_out, const uint32_t (&nxw)[NXP][KWH],
                                                const float (&nxa)[NXP], uint32_t* ws, uint32_t f_old, int G,
                                                int wg, int tid, int lane, int wv, uint64_t t0,
                                                const uint64_t* yx = nullptr, uint32_t ytag = 0,
                                                uint64_t wait_bound = kGridSpin, uint32_t* stamps = nullptr,
                                                const NxRms<(KWH * LPRH * 2 + 64 * W - 1) / (64 * W)>* rms_pre =
                                                    nullptr) {
  constexpr int NWH = KWH * LPRH;
  constexpr int NTH = 64 * W;
  constexpr int RPIH = 64 / LPRH;
  // y, and its RMS-folded x' pairs (hi and lo words, and the value each pair
  // carries) for every word of y, laid out so that the LPRH lanes sharing a
  // row read consecutive entries: word w = LPRH-lane l's KWH-th word i sits at
  // column i * LPRH + l
  __shared__ __align__(16) uint32_t pxh[8][NWH], pxl[8][NWH];
  // per word w and half h: the sum of squares of its raw values 8 h .. + 8,
  // and its pairs 4 h .. + 4's part of the correction term
  __shared__ float sq[2][NWH], cq[2][NWH];
  const int klh = lane % LPRH, subh = lane / LPRH;

  bool timed_out = false;
  if constexpr (!XY) {
    __builtin_amdgcn_s_waitcnt(0);  // this workgroup's y stores have completed
    __syncthreads();
    if (wv == 0) timed_out = grid_barrier_flags(ws + kLine * kSubC, ws + kLine * kFlags, f_old, G, wg, lane, t0);
    __syncthreads();  // every wave waits for the barrier before reading y
  }
  {  // y into LDS, and its x' pairs: thread t builds pairs j0 .. j0 + 3 of
     // word t / 2 (j0 = 4 (t & 1)), each from values j and j + 8 of the word
     // times their RMS weights
    constexpr int PIT = (NWH * 2 + NTH - 1) / NTH;
    uint64_t y0[PIT], y1[PIT], ya[PIT], yb[PIT];
    // the RMS weights: loaded by the caller ahead of time (rms_pre), or here
    // (issued before the reads of y, so a wait for y also waits for them)
    const NxRms<PIT> rw = rms_pre ? *rms_pre : load_nx_rms<NWH, NTH>(nx_rms, tid);
#pragma unroll
    for (int k = 0; k < PIT; ++k) {
      const bool live = tid + NTH * k < NWH * 2;  // threads past the last word build nothing
      const int t = live ? tid + NTH * k : NWH * 2 - 1;
      const int w = t >> 1, j0 = 4 * (t & 1);
      if constexpr (XY) {  // the 16 values of word w: tagged words 8 w .. 8 w + 7
        const CoherentBuf yq(yx, NWH * 8 * 8);
        uint4 q[4] = {};
        for (;;) {
          MA_POLL_RELOAD();
          uint32_t bad = 0;
          if (live) {
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = yq.ld4u(static_cast<uint32_t>((8 * w + 2 * i) * 8));
#pragma unroll
            for (int i = 0; i < 4; ++i) bad |= (q[i].y ^ ytag) | (q[i].w ^ ytag);
          }
          if (__all(bad == 0) || timed_out) break;
          __builtin_amdgcn_s_sleep(1);
          timed_out = (__builtin_amdgcn_s_memrealtime() - t0) > wait_bound;
        }
        // u[m]: values 2 m and 2 m + 1 of the word, as in memory
        const uint32_t u[8] = {q[0].x, q[0].z, q[1].x, q[1].z, q[2].x, q[2].z, q[3].x, q[3].z};
        const int h = t & 1;
        y0[k] = u[4 * h] | (static_cast<uint64_t>(u[4 * h + 1]) << 32);
        y1[k] = u[4 * h + 2] | (static_cast<uint64_t>(u[4 * h + 3]) << 32);
        ya[k] = u[2 * h] | (static_cast<uint64_t>(u[2 * h + 1]) << 32);
        yb[k] = u[4 + 2 * h] | (static_cast<uint64_t>(u[5 + 2 * h]) << 32);
      } else {
        const uint64_t* yp = reinterpret_cast<const uint64_t*>(y + w * 16 + 8 * (t & 1));
        y0[k] = ld_coh64(yp);  // values 8 (t & 1) .. + 8 of word w, raw
        y1[k] = ld_coh64(yp + 1);
        ya[k] = ld_coh64(reinterpret_cast<const uint64_t*>(y + w * 16 + j0));
        yb[k] = ld_coh64(reinterpret_cast<const uint64_t*>(y + w * 16 + j0 + 8));
      }
    }
#pragma unroll
    for (int k = 0; k < PIT; ++k) {
      const int t = tid + NTH * k;
      if (t < NWH * 2) {
        const int w = t >> 1, j0 = 4 * (t & 1);
        const int col = (w % KWH) * LPRH + w / KWH;
        const uint32_t raw[4] = {static_cast<uint32_t>(y0[k]), static_cast<uint32_t>(y0[k] >> 32),
                                 static_cast<uint32_t>(y1[k]), static_cast<uint32_t>(y1[k] >> 32)};
        float s2 = 0.f, ch = 0.f;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const float v0 = __uint_as_float(raw[m] << 16), v1 = __uint_as_float(raw[m] & 0xffff0000u);
          s2 += v0 * v0;
          s2 += v1 * v1;
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int j = j0 + jj;
          const uint32_t ua = static_cast<uint32_t>(ya[k] >> (16 * jj)) & 0xffffu;
          const uint32_t ub = static_cast<uint32_t>(yb[k] >> (16 * jj)) & 0xffffu;
          const float ra_w = __uint_as_float(static_cast<uint32_t>(rw.wa[k][jj >> 1] >> (32 * (jj & 1))));
          const float rb_w = __uint_as_float(static_cast<uint32_t>(rw.wb[k][jj >> 1] >> (32 * (jj & 1))));
          const float xa = __uint_as_float(ua << 16) * ra_w, xb2 = __uint_as_float(ub << 16) * rb_w;
          const float f = pair_scale(j);
          uint16_t ha, la, hb, lb;
          const float r0 = split_hi_lo(f * xa, ha, la);
          const float r1 = split_hi_lo(f * xb2, hb, lb);
          pxh[j][col] = static_cast<uint32_t>(ha) | (static_cast<uint32_t>(hb) << 16);
          pxl[j][col] = static_cast<uint32_t>(la) | (static_cast<uint32_t>(lb) << 16);
          ch += ((f + 1.0f) / f) * (r0 + r1);
        }
        sq[t & 1][w] = s2;
        cq[t & 1][w] = ch;
      }
    }
  }
  MA_XSTAMP_AT(stamps, 12);  // this thread's part of y seen
  __syncthreads();
  // Per K slice (the KWH words of LPRH-lane l, as the standalone GEMV splits
  // a row), once for all rows, by wave 0, in the standalone GEMV's order:
  // the slice's correction term, and the RMS scale from the sum of squares,
  // each word's two halves added, then the words in order; the sum of
  // squares reduced over the slices as the standalone GEMV's lanes reduce
  // it, and kept per lane (the reduction's association differs between
  // lanes, so lane l's scale may differ from lane 0's in the last bit).
  __shared__ float s_corr[LPRH], s_rstd[LPRH];
  if (wv == 0) {
    const int l = lane % LPRH;
    float c = 0.f, ss = 0.f;
#pragma unroll
    for (int i = 0; i < KWH; ++i) {
      const int w = l * KWH + i;
      ss += sq[0][w] + sq[1][w];
      c += cq[0][w] + cq[1][w];
    }
    ss = group_sum<LPRH>(ss);
    if (lane < LPRH) {
      s_corr[lane] = c;
      s_rstd[lane] = rsqrtf(ss / static_cast<float>(NWH * 16) + nx_eps);
    }
  }
  __syncthreads();
  MA_XSTAMP_AT(stamps, 13);  // y, its x' pairs and the slices' terms staged
  // A wave with no rows of this workgroup is done (nothing below waits for it).
  if (wv * RPIH >= nx_rq) return timed_out;
  uint32_t xh[KWH][8], xl[KWH][8];
#pragma unroll
  for (int i = 0; i < KWH; ++i) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      xh[i][j] = pxh[j][i * LPRH + klh];
      xl[i][j] = pxl[j][i * LPRH + klh];
    }
  }
  const float c = s_corr[klh], rstd = s_rstd[klh];
  const ExpandConsts kc;
#pragma unroll
  for (int p = 0; p < NXP; ++p) {
    float acc[2] = {0.f, 0.f};
#pragma unroll
    for (int i = 0; i < KWH; ++i) {
      uint32_t e[8];
      expand_word(nxw[p][i], e, kc);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        acc[j & 1] = dot2(e[j], xh[i][j], acc[j & 1]);
        acc[j & 1] = dot2(e[j], xl[i][j], acc[j & 1]);
      }
    }
    const float d = group_sum<LPRH>(((acc[0] + acc[1]) - c) * (nxa[p] * rstd));
    const int rl = p * W * RPIH + wv * RPIH + subh;
    const int r = wg * nx_rq + rl;
    if (klh == 0 && rl < nx_rq && r < nx_rows) nx_out[r] = f32_to_bf16(d);
  }
  MA_XSTAMP_AT(stamps, 14);  // projection rows out
  return timed_out;
}

// The XCD kernel's launcher (moe_xcd.hip): whether it is built for the call's
// shape, and the launch (same arguments as ma_moe_fused after validation).
bool moe_xcd_supported(int64_t n_experts, int64_t hidden, int64_t inter, int64_t top_k, hipStream_t st);
int moe_xcd_launch(const void* x, const void* x_add, const void* norm_weight, int norm_dtype, float eps,
                   const void* residual, const void* gate_weight, const float* router_bias, int64_t n_experts,
                   int64_t hidden, int64_t inter, const uint32_t* up_gate, const void* up_gate_alpha,
                   const uint32_t* down, const void* down_alpha, int alpha_dtype, void* y, int32_t* topk_ids,
                   float* topk_weight, void* workspace, const uint32_t* next_w, const void* next_alpha,
                   const float* next_rms, float next_eps, int64_t next_rows, void* next_out, const void* attn,
                   const uint32_t* o_w, const void* o_alpha, const void* prefetch, int64_t prefetch_bytes,
                   hipStream_t st);

}  // namespace ma
