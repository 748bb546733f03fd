// Decode attention for q_len = 1 (gfx950): QK RMSNorm + partial RoPE + KV
// write, and split-sequence GQA whose partials are merged in the same launch:
// the splits of a (row, KV head) meet at a barrier of their own, then each
// merges a slice of the output, so one launch does the whole attention.  A
// fused entry point also does the QK-norm/RoPE/KV write inside the same
// launch.
//
// Semantics of reference src/maple_run/kernels/decode_attn.py:
//   apply_qkv_decode (:16-62, :65-163, :362-439): per head x * rsqrt(mean(x^2)
//     + eps) * w, float32; rotate-half RoPE on the first rotary_dim dims with
//     cos/sin in the activation dtype (rows gathered from the float32 table,
//     model.py:94-109); q stored bf16; K and V stored at position seqlen[b]
//     of cache row row_map[b] (b without a map).
//   decode_gqa_attn (:167-359, :470-592): positions [start, min(seqlen[b] + 1,
//     max_len)), start = kv_len - window for a sliding window; scores
//     q.k * scale, softmax in float32 with P rounded to bf16 before P.V,
//     splits merged with exp(m_s - max) weights.
// Positions are clamped to [0, max_len) and mapped rows to [0, cache_rows), so
// nothing is written or read outside the cache.
#include <cstdlib>
#include <cstring>

#include "grid_sync.h"
#include "tgemv_fast.h"

namespace ma {

// head_dim 64 (the synthetic decoder) and 128 (Maple-Preview) are built: each
// lane of a wave owns dims lane + 64 e, e < HD / 64.
constexpr int kSplit = 128;                 // positions per chunk
constexpr int kAttnThreads = 256;           // 4 waves, 32 positions of a chunk each
constexpr int kMaxGroup = 16;               // query heads per KV head
constexpr int kVtRow = kSplit / 2 + 2;      // LDS row (one dim) of V position
                                            // pairs in words, padded
constexpr int kCombineChunk = 4;            // splits whose partials one merge lane loads together
constexpr int kOWords = 4;                  // O projection: words of K per lane (K = 32 x 4 x 16 = 2048)
constexpr int kOPass = 2;                   // O projection: row passes (8 rows each) per workgroup
constexpr int kSyncLine = 64;               // uint32 words per 256-byte line of the sync area
constexpr uint64_t kAttnSpin = 20000000ull; // 0.2 s of the 100 MHz realtime counter
constexpr int kTargetGroups = 512;          // workgroups an attention launch aims for (swept: 512 best at batch 32)


// Attention output store: 4 bf16 values; device-coherent when other
// workgroups of the launch read them back (the O projection below).
__device__ __forceinline__ void store_out(uint16_t* p, uint2 r, bool coherent) {
  if (coherent)
    st_coh64(reinterpret_cast<uint64_t*>(p), (static_cast<uint64_t>(r.y) << 32) | r.x);
  else
    *reinterpret_cast<uint2*>(p) = r;
}

struct RopeSrc {
  const void* cos;
  const void* sin;
  int dt;         // dtype of cos/sin
  int64_t ld;     // row stride in elements
  int64_t n_pos;  // > 0: table rows indexed by position; 0: row b
  int rot;
  int use_rope;
};

// cos/sin for dim d = lane + 64 e of the row used at position ``pos`` of batch
// row b, rounded to bf16 (the activation dtype) as the reference's table
// gather does.
__device__ __forceinline__ float2 rope_coeffs(const RopeSrc& r, int64_t b, int64_t pos, int e) {
  if (!r.use_rope || r.rot <= 0) return make_float2(1.f, 0.f);
  const int d = (threadIdx.x & 63) + 64 * e;
  const int64_t row = r.n_pos > 0 ? (pos < r.n_pos ? pos : r.n_pos - 1) : b;
  const int dd = d < r.rot ? d : 0;
  return make_float2(bf16_to_f32(f32_to_bf16(ld_f(r.cos, r.dt, row * r.ld + dd))),
                     bf16_to_f32(f32_to_bf16(ld_f(r.sin, r.dt, row * r.ld + dd))));
}

// rope_coeffs in two steps for the attention's prologue: the raw words,
// loaded whether or not RoPE is on (from ``safe``, any readable 4-byte
// aligned address, when it is off), then their conversion -- the same
// values, with the loads issued together and no wait until the use.
struct RopeWords {
  AnyWord c, s;
};
__device__ __forceinline__ RopeWords rope_words(const RopeSrc& r, int64_t b, int64_t pos, int e,
                                                const void* safe) {
  const bool on = r.use_rope && r.rot > 0;
  const int d = (threadIdx.x & 63) + 64 * e;
  const int64_t row = r.n_pos > 0 ? (pos < r.n_pos ? pos : r.n_pos - 1) : b;
  const int64_t i = on ? row * r.ld + (d < r.rot ? d : 0) : 0;
  const int dt = on ? r.dt : MA_F32;
  return {ld_any_word(on ? r.cos : safe, dt, i), ld_any_word(on ? r.sin : safe, dt, i)};
}
__device__ __forceinline__ float2 rope_of_words(const RopeSrc& r, const RopeWords& w) {
  if (!r.use_rope || r.rot <= 0) return make_float2(1.f, 0.f);
  return make_float2(bf16_to_f32(f32_to_bf16(any_word_f(w.c, r.dt))),
                     bf16_to_f32(f32_to_bf16(any_word_f(w.s, r.dt))));
}

// RMSNorm of one head held wave-wide (lane owns dims lane + 64 e), then
// rotate-half RoPE on the first ``rot`` dims with the lane's coefficients.
template <int E>
__device__ __forceinline__ void norm_rope_lane(float (&y)[E], const float (&x)[E], const float (&w)[E],
                                               const float2 (&cs)[E], const RopeSrc& r, float eps) {
  const int lane = threadIdx.x & 63;
  float sq = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) sq += x[e] * x[e];
  const float ss = group_sum<64>(sq);
  const float inv = rsqrtf(ss / (64 * E) + eps);
#pragma unroll
  for (int e = 0; e < E; ++e) y[e] = x[e] * inv * w[e];
  if (r.use_rope && r.rot > 0) {
    const int half = r.rot / 2;
    float other[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int d = lane + 64 * e;
      const int pd = d < half ? d + half : d - half;
      float o = 0.f;
#pragma unroll
      for (int f = 0; f < E; ++f) {
        const float v = __shfl(y[f], pd & 63, 64);
        o = (pd >> 6) == f ? v : o;
      }
      other[e] = o;
    }
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int d = lane + 64 * e;
      if (d < r.rot) y[e] = d < half ? y[e] * cs[e].x - other[e] * cs[e].y : y[e] * cs[e].x + other[e] * cs[e].y;
    }
  }
}

// Two wave-uniform 8-byte values read with scalar loads issued back to back
// and one wait for both.
__device__ __forceinline__ void ld_scalar_pair(const int64_t* a, const int64_t* b, int64_t& va,
                                               int64_t& vb) {
  asm volatile(
      "s_load_dwordx2 %0, %2, 0x0\n\t"
      "s_load_dwordx2 %1, %3, 0x0\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(va), "=&s"(vb)
      : "s"(a), "s"(b)
      : "memory");
}

__device__ __forceinline__ int64_t clamp64(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

// One wave per (head slot, row): q heads [0, nq), k heads [nq, nq + nkv), v
// heads after that.  Lane l owns dimensions l + 64 e.
template <int HD>
__global__ __launch_bounds__(64) void k_qk_norm_rope_store(
    const uint16_t* __restrict__ qkv, int64_t ldq, const void* __restrict__ q_w,
    const void* __restrict__ k_w, int w_dt, RopeSrc rope, float eps,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache, const int64_t* __restrict__ seqlen,
    const int64_t* __restrict__ row_map, int64_t cache_rows, int nq, int nkv, int64_t max_len) {
  constexpr int E = HD / 64;
  const int lane = threadIdx.x;
  const int hs = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int64_t pos = clamp64(seqlen[b], 0, max_len - 1);
  const int64_t crow = row_map ? clamp64(row_map[b], 0, cache_rows - 1) : b;
  const uint16_t* row = qkv + b * ldq;
  if (hs >= nq + nkv) {  // V: copy
    const int h = hs - nq - nkv;
#pragma unroll
    for (int e = 0; e < E; ++e)
      v_cache[((crow * nkv + h) * max_len + pos) * HD + lane + 64 * e] = row[(nq + nkv + h) * HD + lane + 64 * e];
    return;
  }
  const bool is_q = hs < nq;
  float x[E], w[E], y[E];
  float2 cs[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    x[e] = bf16_to_f32(row[hs * HD + lane + 64 * e]);
    w[e] = ld_f(is_q ? q_w : k_w, w_dt, lane + 64 * e);
    cs[e] = rope_coeffs(rope, b, pos, e);
  }
  norm_rope_lane<E>(y, x, w, cs, rope, eps);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const uint16_t yb = f32_to_bf16(y[e]);
    if (is_q)
      q_out[(b * nq + hs) * HD + lane + 64 * e] = yb;
    else
      k_cache[((crow * nkv + (hs - nq)) * max_len + pos) * HD + lane + 64 * e] = yb;
  }
}

typedef __bf16 bf16x8a_t __attribute__((ext_vector_type(8)));
typedef float f32x4a_t __attribute__((ext_vector_type(4)));

// 2^x in one v_exp_f32 (2^-inf = 0).
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ f32x4a_t mfma_att(uint4 a, uint4 b, f32x4a_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8a_t, a),
                                                 __builtin_bit_cast(bf16x8a_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t sel32(bool c, uint32_t a, uint32_t b) { return c ? a : b; }

// One workgroup (256 threads, 4 waves) per (split, KV head, row); a split
// walks chunks of 128 positions (the grid holds about kTargetGroups
// workgroups), wave w owning positions 32w .. 32w+31 of each chunk.  On
// v_mfma_f32_16x16x32_bf16 (A lane l: row l%16, k 8(l/16)..+8; B: col l%16,
// k 8(l/16)..+8; C: col l%16, rows 4(l/16)..+4):
//   S^T = K Q^T: A = K rows loaded straight from the cache (16 positions x
//     32 dims), B = q (16 head slots; slots >= group are zero), so lane l
//     ends with head l%16's scores for positions 4(l/16)..+4 of each block;
//   online softmax per head over the chunk (running max and sum, P rounded
//     to bf16 as the reference does before P.V);
//   O += P V: the lane's own 8 P values are its A fragment (k order:
//     positions 4g..4g+3 of block 0 then of block 1), and B takes V in the
//     same order from LDS, where V is stored transposed in position pairs
//     (vt[d][m] = (v_2m[d], v_2m+1[d]), built with one DPP exchange).
//   FUSED: the group's q heads are RMS-normalised + roped from the qkv row;
//     the split holding position seqlen[b] builds the new K/V, uses them in
//     place of what it read and stores them to the cache at the end.
// One split: normalise and store.  Several: (acc, m, l) partials with
// device-coherent stores, a barrier among the splits of the (row, KV head)
// (an arrival counter and a generation word, each on its own line of the
// sync area: the last to arrive clears the counter and advances the
// generation the others poll), then split s merges output items [s * ipw,
// (s + 1) * ipw): every split reads a small slice of the partials instead of
// one split reading them all.  The splits of a pair are consecutive in
// dispatch order and far fewer than the GPU holds at once, so they are all
// resident; the wait is bounded (about 0.2 s) and records a timeout in word 2
// of the sync area instead of hanging.
//
// XL (used where the GPU hands workgroup i to XCD (i + o) mod 8): a 1-D grid
// of 8 * S * ceil(n_pairs / 8) workgroups, S = splits per pair.  Workgroup L
// is split S - 1 - (L / 8) mod S of pair 8 * (L / 8 / S) + L mod 8 (the last
// splits first: the one with the new position does the most before its
// barrier, and the splits dispatched last may share a CU -- at batch 1, 34
// splits per XCD of 32 CUs; owner-first measured 1,396 against 1,370
// tok/s), so every split of
// a pair runs on one XCD and the hand-off stays in that XCD's L2: partials go
// out as plain stores, each split then raises its own flag (word 1 + split of
// the pair's arrival line) to the pair's generation + 1 and polls its
// siblings' flags with L1-bypassing loads; split 0 advances the generation
// once it has seen every flag.  Workgroups past the last pair only take part
// in the O projection.  A pair's S splits are consecutive in its XCD's
// dispatch order, so they are resident together when S workgroups fit on one
// XCD.
template <bool FUSED, int HD, bool XL>
// (The arguments the prologue's first loads need come first: the first 14
// dwords arrive preloaded in SGPRs, the rest are read from memory.)
__global__ __launch_bounds__(kAttnThreads) void k_decode_attn(
    const int64_t* __restrict__ seqlen, const int64_t* __restrict__ row_map,
    const uint16_t* __restrict__ src, int64_t ldq, int nq, int nkv, int n_rows, int xl_splits,
    int64_t max_len, const void* __restrict__ qn_w, const void* __restrict__ kn_w, int w_dt,
    RopeSrc rope, float eps, uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
    int64_t cache_rows, int64_t window, float scale, int max_splits, uint32_t* __restrict__ sync,
    float* __restrict__ part_acc, float* __restrict__ part_ml, uint16_t* __restrict__ out,
    const uint32_t* __restrict__ o_w, const void* __restrict__ o_alpha, int o_alpha_dt, int o_rows,
    uint16_t* __restrict__ o_out) {
  constexpr int E = HD / 64;   // dims per lane in the wave-wide head layouts
  constexpr int KS = HD / 32;  // 32-dim slices of K per score MFMA chain
  constexpr int NB = HD / 16;  // 16-dim output blocks of P.V
  constexpr int IPH = HD / 4;  // 4-dim output items per head
  __shared__ __align__(16) uint16_t qs[kMaxGroup][HD];
  __shared__ __align__(16) uint32_t vt[HD][kVtRow];
  __shared__ __align__(16) uint16_t kvnew[2][HD];
  __shared__ float wm[4][kMaxGroup], wl[4][kMaxGroup];
  __shared__ float hm[kMaxGroup], hl[kMaxGroup];
  __shared__ __align__(16) uint4 os4[kOWords * 2][32];  // O projection input
  // The arguments past the preloaded ones that the prologue needs, read at
  // once with one wait: left to itself the compiler read each where first
  // used, a wait each (six dependent scalar round trips before the first
  // K/V load).
  asm volatile("" ::"s"(qn_w), "s"(kn_w), "s"(w_dt), "s"(rope.cos), "s"(rope.sin), "s"(rope.dt),
               "s"(rope.ld), "s"(rope.n_pos), "s"(rope.rot), "s"(rope.use_rope), "s"(eps),
               "s"(k_cache), "s"(v_cache), "s"(cache_rows), "s"(window), "s"(sync), "s"(o_w),
               "s"(o_rows), "s"(max_splits));
  // (split, KV head, row) of this workgroup; the grid's split count; its
  // index and size for the O projection's barrier
  int sp, kvh, S, wgl, n_wg;
  int64_t b;
  bool active = true;
  if constexpr (XL) {
    const int L = static_cast<int>(blockIdx.x), q = L >> 3;
    S = xl_splits;
    sp = (S - 1) - q % S;
    const int P = (q / S) * kXcds + (L & (kXcds - 1));
    active = P < n_rows * nkv;
    b = active ? P / nkv : 0;
    kvh = active ? P % nkv : 0;
    wgl = L;
    n_wg = static_cast<int>(gridDim.x);
  } else {
    sp = blockIdx.x;
    kvh = blockIdx.y;
    b = blockIdx.z;
    S = static_cast<int>(gridDim.x);
    wgl = (static_cast<int>(b) * static_cast<int>(gridDim.y) + kvh) * static_cast<int>(gridDim.x) + sp;
    n_wg = static_cast<int>(gridDim.x * gridDim.y * gridDim.z);
  }
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int group = nq / nkv;
  // This pair's barrier words.
  uint32_t* const arrive = sync + kSyncLine * (1 + 2 * (b * nkv + kvh));
  uint32_t* const gen = arrive + kSyncLine;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  // O projection in the same launch (batch 1): a barrier over every workgroup
  // of the launch on the sync area's last 33 lines, then each workgroup
  // computes its rows of o from the whole attention output.
  uint32_t* const gsub = sync + kSyncLine * (1 + 2 * n_rows * nkv);
  uint32_t* const gflags = gsub + kSyncLine * (kBarGroups + 1);
  const uint32_t f0o = o_w && wv == 0 ? ld_coh32(&gflags[kSyncLine * (wgl % kBarGroups)]) : 0u;
  // This workgroup's O rows (as the standalone GEMV splits them: 32 lanes of
  // kOWords words per row, 2 rows per wave pass, kOPass passes), loaded once
  // the K/V chunks are in, so that they do not compete with them.
  const int o_rq = o_w ? (o_rows + n_wg - 1) / n_wg : 0;
  const int okl = lane & 31, osub = lane >> 5;
  uint32_t ow_w[kOPass][kOWords];
  float ow_a[kOPass];
  auto o_prefetch = [&]() {
#pragma unroll
    for (int p = 0; p < kOPass; ++p) {
      int r = wgl * o_rq + p * 8 + wv * 2 + osub;
      r = r < o_rows ? r : o_rows - 1;
      load_words<kOWords>(o_w + static_cast<int64_t>(r) * (32 * kOWords) + okl * kOWords, ow_w[p]);
      ow_a[p] = ld_f(o_alpha, o_alpha_dt, r);
    }
  };
  auto attend = [&]() {
  // The prologue's position-independent loads go out first, before the
  // position is read: q's heads (fused: also the new K/V row's elements and
  // the norm weights), as raw values from in-bounds addresses (heads past
  // the group read head 0 and are dropped), converted only once the
  // position-dependent loads (the RoPE rows, the first K/V chunk) are out
  // too.  A load under a condition or a dtype switch would get a wait of its
  // own right behind it: a chain of round trips before q is ready.
  uint16_t xq[kMaxGroup / 4][E];                  // fused: head wv + 4 i, dims lane + 64 e
  uint16_t xkv[E];                                // fused: the new K (wave 0) or V (wave 1) row
  AnyWord wqr[E], wkr[E];                         // fused: the norm weights
  uint16_t xqf[kMaxGroup * HD / kAttnThreads];    // not fused: q element tid + kAttnThreads k
  if constexpr (FUSED) {
    const uint16_t* row = src + b * ldq;
#pragma unroll
    for (int i = 0; i < kMaxGroup / 4; ++i) {
      const int hh = wv + 4 * i, hc = hh < group ? hh : 0;
#pragma unroll
      for (int e = 0; e < E; ++e) xq[i][e] = row[(kvh * group + hc) * HD + lane + 64 * e];
    }
#pragma unroll
    for (int e = 0; e < E; ++e) {
      xkv[e] = row[(nq + kvh + (wv == 1 ? nkv : 0)) * HD + lane + 64 * e];
      wqr[e] = ld_any_word(qn_w, w_dt, lane + 64 * e);
      wkr[e] = ld_any_word(kn_w, w_dt, lane + 64 * e);
    }
  } else {
    const uint16_t* qsrc = src + (b * nq + kvh * group) * HD;
#pragma unroll
    for (int k = 0; k < kMaxGroup * HD / kAttnThreads; ++k) {
      const int i = tid + kAttnThreads * k;
      xqf[k] = qsrc[i / HD < group ? i : i % HD];
    }
  }
  MA_ISSUE_FENCE();
  // the cache row and the position: two scalar loads issued together, then
  // one wait (the row map's from a valid address either way; left to the
  // compiler, the second load went out only after the first had returned)
  int64_t rmv, slv;
  ld_scalar_pair(row_map ? row_map + b : seqlen + b, seqlen + b, rmv, slv);
  // The pair's generation, read before this split can arrive (so it is the
  // value the last arriver will advance) and after the prologue's loads are
  // out; by every wave, though wave 0 alone uses it (under a wave condition
  // the load got its wait right behind it).
  const uint32_t g0 = __hip_atomic_load(gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int64_t pos = clamp64(slv, 0, max_len - 1);
  const int64_t crow = row_map ? clamp64(rmv, 0, cache_rows - 1) : b;
  const int64_t kv_len = pos + 1;
  const int64_t start = (window > 0 && kv_len > window) ? kv_len - window : 0;
  const int n_chunks = static_cast<int>(cdiv(kv_len - start, kSplit));
  // (32-bit divisions: the 64-bit ones are long scalar sequences on the
  // path to the first K/V load)
  const int cps = static_cast<int>((static_cast<uint32_t>(n_chunks) + S - 1) / static_cast<uint32_t>(S));
  const int n_spl = static_cast<int>((static_cast<uint32_t>(n_chunks) + cps - 1) / static_cast<uint32_t>(cps));
  const float scale2 = scale * 1.44269504088896341f;  // log2(e): maxima and sums in base 2
  const int c_beg = sp * cps;
  const int c_end = c_beg + cps < n_chunks ? c_beg + cps : n_chunks;
  const int64_t base = (crow * nkv + kvh) * max_len;
  const bool owns_pos = FUSED && sp == n_spl - 1;

  // K fragments: positions 32 wv + 16 pb + r16, dims 8 g + 32 ks.
  // V: load (i, e) covers the wave's positions 32 wv + 8 i .. +7: lane l
  // holds position 32 wv + 8 i + (l >> 3), dims 64 e + 8 (l & 7) .. +8.
  auto load_chunk = [&](int c, uint4 (&kf)[2][KS], uint4 (&vr)[4][E]) {
    const int64_t lo = start + static_cast<int64_t>(c) * kSplit;
    const int64_t hi = lo + kSplit < kv_len ? lo + kSplit : kv_len;
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
      int64_t t = lo + 32 * wv + 16 * pb + r16;
      t = t < hi ? t : hi - 1;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        kf[pb][ks] = *reinterpret_cast<const uint4*>(k_cache + (base + t) * HD + 8 * g + 32 * ks);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int64_t tv = lo + 32 * wv + 8 * i + (lane >> 3);
      tv = tv < hi ? tv : hi - 1;
#pragma unroll
      for (int e = 0; e < E; ++e)
        vr[i][e] = *reinterpret_cast<const uint4*>(v_cache + (base + tv) * HD + 64 * e + 8 * (lane & 7));
    }
  };
  uint4 kf[2][KS], vr[4][E];
  uint16_t new_kv[E] = {};  // FUSED owner split: the new K (wave 0) or V (wave 1) elements
  if constexpr (FUSED) {
    // Every load of the prologue is issued before any of them is used, and
    // before the first chunk's (memory counters complete in issue order, so
    // q would otherwise wait for the K/V chunk).
    RopeWords rw[E];
#pragma unroll
    for (int e = 0; e < E; ++e) rw[e] = rope_words(rope, b, pos, e, qn_w);  // qn_w: read above
    load_chunk(c_beg, kf, vr);
    float wq[E], wk[E];
    float2 cs[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      wq[e] = any_word_f(wqr[e], w_dt);
      wk[e] = any_word_f(wkr[e], w_dt);
      cs[e] = rope_of_words(rope, rw[e]);
    }
#pragma unroll
    for (int i = 0; i < kMaxGroup / 4; ++i) {
      const int hh = wv + 4 * i;
      if (hh < group) {  // (rows past the group only need zeros)
        float xf[E], yf[E];
#pragma unroll
        for (int e = 0; e < E; ++e) xf[e] = bf16_to_f32(xq[i][e]);
        norm_rope_lane<E>(yf, xf, wq, cs, rope, eps);
#pragma unroll
        for (int e = 0; e < E; ++e) qs[hh][lane + 64 * e] = f32_to_bf16(yf[e]);
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) qs[hh][lane + 64 * e] = uint16_t(0);
      }
    }
    if (owns_pos && wv < 2) {
      float xf[E], yf[E];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        new_kv[e] = xkv[e];  // wave 1: V is stored as is
        xf[e] = bf16_to_f32(xkv[e]);
      }
      if (wv == 0) {
        norm_rope_lane<E>(yf, xf, wk, cs, rope, eps);
#pragma unroll
        for (int e = 0; e < E; ++e) new_kv[e] = f32_to_bf16(yf[e]);
      }
#pragma unroll
      for (int e = 0; e < E; ++e) kvnew[wv][lane + 64 * e] = new_kv[e];
    }
  } else {
    load_chunk(c_beg, kf, vr);
#pragma unroll
    for (int k = 0; k < kMaxGroup * HD / kAttnThreads; ++k) {
      const int i = tid + kAttnThreads * k;
      qs[i / HD][i % HD] = i / HD < group ? xqf[k] : uint16_t(0);
    }
  }
  __syncthreads();
  // Splits past the last chunk ran the prologue too (its loads stay in one
  // block with their uses, so the compiler does not sink them behind the
  // position's wait), and stop here.
  if (sp >= n_spl) {
    if (o_w) o_prefetch();
    return;
  }
  uint4 qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) qf[ks] = *reinterpret_cast<const uint4*>(&qs[r16][8 * g + 32 * ks]);

  // Each wave keeps its own running softmax state over its 32 positions of
  // every chunk (head r16's max and sum, in the 4 lanes holding that head), so
  // a chunk needs no workgroup barrier; the waves' states are combined once,
  // after the last chunk.  V^T of a chunk sits in the wave's own columns of
  // vt (positions 32 wv .. +31), which only that wave writes and reads.
  float mrun = -INFINITY, lrun = 0.f;
  f32x4a_t oacc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) oacc[nb] = f32x4a_t{0.f, 0.f, 0.f, 0.f};
  for (int c = c_beg; c < c_end; ++c) {
    const int64_t lo = start + static_cast<int64_t>(c) * kSplit;
    const int64_t hi = lo + kSplit < kv_len ? lo + kSplit : kv_len;
    if constexpr (FUSED) {  // the position written by this launch: the new K/V
#pragma unroll
      for (int pb = 0; pb < 2; ++pb) {
        const bool nk = owns_pos && lo + 32 * wv + 16 * pb + r16 == pos;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const uint4 v = *reinterpret_cast<const uint4*>(&kvnew[0][8 * g + 32 * ks]);
          kf[pb][ks] = make_uint4(sel32(nk, v.x, kf[pb][ks].x), sel32(nk, v.y, kf[pb][ks].y),
                                  sel32(nk, v.z, kf[pb][ks].z), sel32(nk, v.w, kf[pb][ks].w));
        }
      }
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const uint4 v = *reinterpret_cast<const uint4*>(&kvnew[1][64 * e + 8 * (lane & 7)]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool nv = owns_pos && lo + 32 * wv + 8 * i + (lane >> 3) == pos;
          vr[i][e] = make_uint4(sel32(nv, v.x, vr[i][e].x), sel32(nv, v.y, vr[i][e].y),
                                sel32(nv, v.z, vr[i][e].z), sel32(nv, v.w, vr[i][e].w));
        }
      }
    }
    // V^T in position pairs: lanes l and l ^ 8 hold positions 2m and 2m + 1
    // of the same 8 dims (one DPP rotate by 8 within each 16-lane row swaps
    // them); the even one writes the pairs of dims 0..3 of its 8, the odd one
    // dims 4..7.
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const bool odd = (lane >> 3) & 1;
      const int d0 = 64 * e + 8 * (lane & 7) + (odd ? 4 : 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t u[4] = {vr[i][e].x, vr[i][e].y, vr[i][e].z, vr[i][e].w};
        uint32_t o[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] = __builtin_amdgcn_update_dpp(0, u[k], 0x128, 0xF, 0xF, false);
        const int m = 16 * wv + 4 * i + (lane >> 4);
        // dims d0 .. d0+3: words 2 (odd) .. +1 of this lane's (and the partner's) 4
        const uint32_t a0 = odd ? o[2] : u[0], a1 = odd ? o[3] : u[1];  // position 2m
        const uint32_t b0 = odd ? u[2] : o[0], b1 = odd ? u[3] : o[1];  // position 2m + 1
        vt[d0][m] = (a0 & 0xffffu) | (b0 << 16);
        vt[d0 + 1][m] = (a0 >> 16) | (b0 & 0xffff0000u);
        vt[d0 + 2][m] = (a1 & 0xffffu) | (b1 << 16);
        vt[d0 + 3][m] = (a1 >> 16) | (b1 & 0xffff0000u);
      }
    }
    // Scores and this wave's per-head maximum.
    // (in the base-2 domain: scores times log2(e), so that every exponential
    // of the softmax and of the merges is one v_exp_f32)
    float s[2][4];
    const int span = static_cast<int>(hi - lo);
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
      f32x4a_t acc = mfma_att(kf[pb][0], qf[0], f32x4a_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
      for (int ks = 1; ks < KS; ++ks) acc = mfma_att(kf[pb][ks], qf[ks], acc);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        s[pb][i] = 32 * wv + 16 * pb + 4 * g + i < span ? acc[i] * scale2 : -INFINITY;
    }
    if (c + 1 < c_end) load_chunk(c + 1, kf, vr);  // in flight during softmax and P.V
    float mx = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                     fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(mrun, mx);
    const float r = m_new == -INFINITY ? 1.f : exp2_fast(mrun - m_new);  // 0 on the first valid chunk
    float p[2][4], ls = 0.f;
#pragma unroll
    for (int pb = 0; pb < 2; ++pb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[pb][i] = s[pb][i] == -INFINITY ? 0.f : exp2_fast(s[pb][i] - m_new);
        ls += p[pb][i];
      }
    ls += __shfl_xor(ls, 16, 64);
    ls += __shfl_xor(ls, 32, 64);
    lrun = lrun * r + ls;
    mrun = m_new;
    // P in bf16 as the A fragment: k = positions 4g..4g+3 of block 0, then of block 1.
    const uint4 pa = make_uint4(pack_bf16x2_rn(p[0][0], p[0][1]), pack_bf16x2_rn(p[0][2], p[0][3]),
                                pack_bf16x2_rn(p[1][0], p[1][1]), pack_bf16x2_rn(p[1][2], p[1][3]));
    // rescale of head 4g + i: held by lane 4g + i
    float rr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) rr[i] = __shfl(r, 4 * g + i, 64);
    const int mp = 16 * wv + 2 * g;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int d = 16 * nb + r16;
      const uint2 b0 = *reinterpret_cast<const uint2*>(&vt[d][mp]);
      const uint2 b1 = *reinterpret_cast<const uint2*>(&vt[d][mp + 8]);
#pragma unroll
      for (int i = 0; i < 4; ++i) oacc[nb][i] *= rr[i];
      oacc[nb] = mfma_att(pa, make_uint4(b0.x, b0.y, b1.x, b1.y), oacc[nb]);
    }
    }
  if (o_w) o_prefetch();  // after the K/V stream, in flight through the merge and the barrier
  // The new K/V go to the cache last (after every read of the cache).
  if (owns_pos && wv < 2) {
#pragma unroll
    for (int e = 0; e < E; ++e) (wv == 0 ? k_cache : v_cache)[(base + pos) * HD + lane + 64 * e] = new_kv[e];
  }
  // Combine the waves' states in a fixed order, through LDS that V no longer
  // needs: head h's max M = max_w m_w, sum = sum_w l_w exp(m_w - M), output
  // sum_w acc_w exp(m_w - M).
  static_assert(sizeof(vt) >= 4 * kMaxGroup * HD * sizeof(float), "reduction buffer");
  float (*ow)[kMaxGroup][HD] = reinterpret_cast<float (*)[kMaxGroup][HD]>(&vt[0][0]);
  __syncthreads();  // every wave's last P.V has read its vt columns
  if (g == 0) {
    wm[wv][r16] = mrun;
    wl[wv][r16] = lrun;
  }
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (4 * g + i < group) ow[wv][4 * g + i][16 * nb + r16] = oacc[nb][i];
  __syncthreads();
  if (tid < kMaxGroup) {
    const float M = fmaxf(fmaxf(wm[0][tid], wm[1][tid]), fmaxf(wm[2][tid], wm[3][tid]));
    float L = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float sc = wm[w][tid] == -INFINITY ? 0.f : exp2_fast(wm[w][tid] - M);
      L += wl[w][tid] * sc;
      wm[w][tid] = sc;  // from here on: wave w's scale for head tid
    }
    hm[tid] = M;
    hl[tid] = L;
  }
  __syncthreads();
  const int64_t pidx = (b * nkv + kvh) * max_splits + sp;
  const int64_t n_part = static_cast<int64_t>(n_rows) * nkv * max_splits * kMaxGroup;
  const CoherentBuf acc_buf(part_acc, static_cast<uint32_t>(n_part * HD * 4));
  const CoherentBuf ml_buf(part_ml, static_cast<uint32_t>(n_part * 8));
  for (int item = tid; item < group * IPH; item += kAttnThreads) {
    const int hh = item / IPH, dq = item % IPH;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float4 q = *reinterpret_cast<const float4*>(&ow[w][hh][4 * dq]);
      const float sc = wm[w][hh];
      o.x += q.x * sc;
      o.y += q.y * sc;
      o.z += q.z * sc;
      o.w += q.w * sc;
    }
    if (n_spl == 1) {
      const float inv = 1.f / hl[hh];
      uint2 r;
      r.x = pack_bf16x2_rn(o.x * inv, o.y * inv);
      r.y = pack_bf16x2_rn(o.z * inv, o.w * inv);
      store_out(out + (b * nq + kvh * group + hh) * HD + 4 * dq, r, o_w != nullptr);
    } else if constexpr (XL) {  // read back through this XCD's L2 only
      *reinterpret_cast<float4*>(part_acc + (pidx * kMaxGroup + hh) * HD + 4 * dq) = o;
    } else {
      acc_buf.st4(static_cast<uint32_t>(((pidx * kMaxGroup + hh) * HD + 4 * dq) * 4), o);
    }
  }
  if (n_spl == 1) return;
  if (tid < group) {
    if constexpr (XL)
      *reinterpret_cast<float2*>(part_ml + (pidx * kMaxGroup + tid) * 2) = make_float2(hm[tid], hl[tid]);
    else
      ml_buf.st2(static_cast<uint32_t>((pidx * kMaxGroup + tid) * 8), make_float2(hm[tid], hl[tid]));
  }
  // Barrier among the n_spl splits of this (row, KV head), once this split's
  // partials have completed (no device-scope fence: on this GPU that writes
  // back the whole L2).
  if constexpr (XL) MA_STORES_DONE();
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if constexpr (XL) {
    // n_spl <= S <= 63 flags, one lane each
    uint32_t* const flags = arrive + 1;
    const uint32_t tag = g0 + 1u;
    if (wv == 0) {
      if (lane == 0) st_l2_32(&flags[sp], tag);
      bool timed_out = false;
      for (;;) {
        MA_POLL_RELOAD();
        const bool seen = lane >= n_spl || ld_coh32(&flags[lane]) == tag;
        if (__builtin_amdgcn_ballot_w64(!seen) == 0 || timed_out) break;
        __builtin_amdgcn_s_sleep(1);
        timed_out = (__builtin_amdgcn_s_memrealtime() - t0) > kAttnSpin;
      }
      if (timed_out && lane == 0) st_coh32(sync + 2, 1u);
      if (sp == 0 && lane == 0) st_coh32(gen, tag);
    }
  } else if (tid == 0) {
    if (atomicAdd(arrive, 1u) == static_cast<uint32_t>(n_spl - 1)) {
      __hip_atomic_store(arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(gen, g0 + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      bool timed_out = false;
      while (__hip_atomic_load(gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == g0 && !timed_out) {
        __builtin_amdgcn_s_sleep(1);
        timed_out = (__builtin_amdgcn_s_memrealtime() - t0) > kAttnSpin;
      }
      if (timed_out) __hip_atomic_store(sync + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  // Merge this split's slice.  Item (head, 4 dims) is shared by TPI adjacent
  // lanes (the power of two >= n_spl, at most a wave); lane j folds splits j,
  // j + TPI, ... (kCombineChunk per round, loads issued together) into a
  // running (max, sum, acc) state, and the TPI states combine through lane
  // exchanges in a fixed order.
  const int64_t p0 = (b * nkv + kvh) * max_splits;
  const int n_items = group * IPH;
  const int ipw = (n_items + n_spl - 1) / n_spl;
  const int it_lo = sp * ipw, it_hi = it_lo + ipw < n_items ? it_lo + ipw : n_items;
  int tpi = 1;
  while (tpi < n_spl && tpi < 64) tpi *= 2;
  for (int ib = it_lo; ib < it_hi; ib += kAttnThreads / tpi) {
    const int item = ib + tid / tpi, j = tid % tpi;
    const bool live = item < it_hi;
    const int hh = live ? item / IPH : 0, dq = item % IPH;
    float mx = -INFINITY, den = 0.f, n0 = 0.f, n1 = 0.f, n2 = 0.f, n3 = 0.f;
    for (int s0 = 0; s0 < n_spl; s0 += kCombineChunk * tpi) {  // uniform over the wave
      float2 ml[kCombineChunk];
      float4 ac[kCombineChunk];
#pragma unroll
      for (int u = 0; u < kCombineChunk; ++u) {  // absent splits load nothing
        const int s = s0 + u * tpi + j;
        ml[u] = make_float2(-INFINITY, 0.f);
        ac[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (s < n_spl) {
          const uint32_t q = static_cast<uint32_t>((p0 + s) * kMaxGroup + hh);
          ml[u] = ml_buf.ld2(q * 8);
          ac[u] = acc_buf.ld4((q * HD + 4 * dq) * 4);
        }
      }
      MA_ISSUE_FENCE();
#pragma unroll
      for (int u = 0; u < kCombineChunk; ++u) {
        if (s0 + u * tpi < n_spl) {  // uniform: some lane of every item has this split
          const bool ok = s0 + u * tpi + j < n_spl;
          const float m = ok ? ml[u].x : -INFINITY;
          const float mn = fmaxf(mx, m);
          const float r = mx == -INFINITY ? 0.f : exp2_fast(mx - mn);
          const float w = ok ? exp2_fast(m - mn) : 0.f;
          den = den * r + w * ml[u].y;
          n0 = n0 * r + w * ac[u].x;
          n1 = n1 * r + w * ac[u].y;
          n2 = n2 * r + w * ac[u].z;
          n3 = n3 * r + w * ac[u].w;
          mx = mn;
        }
      }
    }
    for (int off = 1; off < tpi; off <<= 1) {  // lanes without splits hold mx = -inf
      const float mo = __shfl_xor(mx, off, 64), dn = __shfl_xor(den, off, 64);
      const float o0 = __shfl_xor(n0, off, 64), o1 = __shfl_xor(n1, off, 64);
      const float o2 = __shfl_xor(n2, off, 64), o3 = __shfl_xor(n3, off, 64);
      const float mn = fmaxf(mx, mo);
      const float r = mx == -INFINITY ? 0.f : exp2_fast(mx - mn);
      const float ro = mo == -INFINITY ? 0.f : exp2_fast(mo - mn);
      den = den * r + dn * ro;
      n0 = n0 * r + o0 * ro;
      n1 = n1 * r + o1 * ro;
      n2 = n2 * r + o2 * ro;
      n3 = n3 * r + o3 * ro;
      mx = mn;
    }
    if (live && j == 0) {
      uint2 r;
      r.x = pack_bf16x2_rn(n0 / den, n1 / den);
      r.y = pack_bf16x2_rn(n2 / den, n3 / den);
      store_out(out + (b * nq + kvh * group + hh) * HD + 4 * dq, r, o_w != nullptr);
    }
  }
  };
  if (active)
    attend();
  else if (o_w)
    o_prefetch();
  if (!o_w) return;

  // O projection: o_out = ternary_gemv(attention output, o_w, o_alpha) --
  // reference kernels/ternary_gemv.py (the o_proj of MapleAttention,
  // model.py:368-414) -- with the standalone fast GEMV's per-lane arithmetic
  // in the same order (so the same bits), once every workgroup's slice of
  // the attention output is out.
  __builtin_amdgcn_s_waitcnt(0);  // this workgroup's output stores have completed
  __syncthreads();
  bool o_timed_out = false;
  if (wv == 0) o_timed_out = grid_barrier_flags(gsub, gflags, f0o, n_wg, wgl, lane, t0);
  __syncthreads();
  {  // entry (i, half, l) of os4 = values 8 half .. + 8 of word l * kOWords + i
    const int w = tid >> 1, half = tid & 1;
    const uint64_t* p = reinterpret_cast<const uint64_t*>(out + static_cast<int64_t>(b) * nq * HD +
                                                          w * 16 + 8 * half);
    const uint64_t v0 = ld_coh64(p), v1 = ld_coh64(p + 1);
    os4[(w % kOWords) * 2 + half][w / kOWords] =
        make_uint4(static_cast<uint32_t>(v0), static_cast<uint32_t>(v0 >> 32),
                   static_cast<uint32_t>(v1), static_cast<uint32_t>(v1 >> 32));
  }
  __syncthreads();
  uint32_t xh[kOWords][8];
  float c = 0.f;
#pragma unroll
  for (int i = 0; i < kOWords; ++i) {
    const uint4 a0 = os4[i * 2][okl], a1 = os4[i * 2 + 1][okl];
    const uint32_t u[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    float xs[16];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      xs[2 * q] = __uint_as_float(u[q] << 16);
      xs[2 * q + 1] = __uint_as_float(u[q] & 0xffff0000u);
    }
    c += prep_word_pairs(xs, xh[i]);
  }
  const ExpandConsts kc;
#pragma unroll
  for (int p = 0; p < kOPass; ++p) {
    float acc[2] = {0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kOWords; ++i) {
      uint32_t e[8];
      expand_word(ow_w[p][i], e, kc);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j & 1] = dot2(e[j], xh[i][j], acc[j & 1]);
    }
    const float d = group_sum<32>(((acc[0] + acc[1]) - c) * ow_a[p]);
    const int rl = p * 8 + wv * 2 + osub;
    const int r = wgl * o_rq + rl;
    if (okl == 0 && rl < o_rq && r < o_rows) o_out[r] = f32_to_bf16(d);
  }
  if (o_timed_out && tid == 0) st_coh32(sync + 2, 1u);
}

// Sync area: line 0 (word 2: timeout), then per (row, KV head) an arrival
// counter line (word 0: the counter; words 1 .. 63: the XCD-local form's
// per-split flags) and a generation line, then the O projection's grid
// barrier (16 group-counter lines, one unused line, 16 group-flag lines).
size_t sync_bytes(int64_t batch, int nkv) {
  return (1 + 2 * static_cast<size_t>(batch) * nkv + 2 * kBarGroups + 1) * kSyncLine * sizeof(uint32_t);
}

int64_t max_splits_for(int64_t max_len) { return cdiv(max_len, kSplit); }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int check_rope(const RopeSrc& r, int head_dim, const char* what) {
  if (r.rot < 0 || r.rot > head_dim || r.rot % 2)
    return fail(MA_EVALUE, "%s: rotary_dim %d must be even and <= head_dim", what, r.rot);
  if (r.use_rope && r.rot > 0) {
    if (!r.cos || !r.sin) return fail(MA_EVALUE, "%s: cos/sin missing", what);
    if (r.dt != MA_F32 && r.dt != MA_BF16 && r.dt != MA_F16)
      return fail(MA_ETYPE, "%s: cos/sin dtype %d unsupported", what, r.dt);
    if (r.n_pos < 0 || r.ld < r.rot) return fail(MA_EVALUE, "%s: bad cos/sin layout", what);
  }
  return MA_OK;
}

int check_heads(int64_t batch, int nq, int nkv, int head_dim, int64_t max_len, int64_t cache_rows,
                const void* row_map, const char* what) {
  if (head_dim != 64 && head_dim != 128)
    return fail(MA_EVALUE, "%s: head_dim %d unsupported (64 or 128)", what, head_dim);
  if (batch < 0 || nq < 1 || nkv < 1 || nq % nkv || nq / nkv > kMaxGroup || max_len < 1)
    return fail(MA_EVALUE, "%s: bad sizes", what);
  if (!row_map && cache_rows < batch)
    return fail(MA_EVALUE, "%s: cache has %lld rows for batch %lld", what,
                static_cast<long long>(cache_rows), static_cast<long long>(batch));
  if (cache_rows < 1) return fail(MA_EVALUE, "%s: empty cache", what);
  return MA_OK;
}

}  // namespace ma

using namespace ma;

extern "C" int ma_qk_norm_rope_store(const void* qkv, int64_t ldq, int64_t batch, int n_heads,
                                     int n_kv_heads, int head_dim, const void* q_norm_w,
                                     const void* k_norm_w, int w_dtype, const void* cos,
                                     const void* sin, int cs_dtype, int64_t ld_cs, int64_t n_pos,
                                     int rotary_dim, int use_rope, float eps,
                                     const int64_t* seqlen, const int64_t* row_map,
                                     void* k_cache, void* v_cache, int64_t cache_rows,
                                     int64_t max_len, void* q_out, void* stream) {
  const char* what = "qk_norm_rope_store";
  if (int rc = check_heads(batch, n_heads, n_kv_heads, head_dim, max_len, cache_rows, row_map, what))
    return rc;
  const RopeSrc rope{cos, sin, cs_dtype, ld_cs, n_pos, rotary_dim, use_rope};
  if (int rc = check_rope(rope, head_dim, what)) return rc;
  if (w_dtype != MA_F32 && w_dtype != MA_BF16 && w_dtype != MA_F16)
    return fail(MA_ETYPE, "%s: norm weight dtype %d unsupported", what, w_dtype);
  if (ldq < static_cast<int64_t>(n_heads + 2 * n_kv_heads) * head_dim)
    return fail(MA_EVALUE, "%s: qkv row stride too small", what);
  if (batch == 0) return MA_OK;
  dim3 grid(static_cast<unsigned>(n_heads + 2 * n_kv_heads), static_cast<unsigned>(batch));
#define MA_QK_ARGS                                                                               \
  static_cast<const uint16_t*>(qkv), ldq, q_norm_w, k_norm_w, w_dtype, rope, eps,                \
      static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), \
      seqlen, row_map, cache_rows, n_heads, n_kv_heads, max_len
  if (head_dim == 128)
    hipLaunchKernelGGL(k_qk_norm_rope_store<128>, grid, dim3(64), 0, static_cast<hipStream_t>(stream),
                       MA_QK_ARGS);
  else
    hipLaunchKernelGGL(k_qk_norm_rope_store<64>, grid, dim3(64), 0, static_cast<hipStream_t>(stream),
                       MA_QK_ARGS);
#undef MA_QK_ARGS
  return check_launch(what);
}

extern "C" size_t ma_gqa_workspace_bytes(int64_t batch, int n_kv_heads, int64_t max_len, int head_dim) {
  if (batch < 0 || n_kv_heads < 1 || max_len < 1 || (head_dim != 64 && head_dim != 128)) return 0;
  const size_t parts = static_cast<size_t>(batch) * n_kv_heads * max_splits_for(max_len) * kMaxGroup;
  return sync_bytes(batch, n_kv_heads) + parts * (head_dim + 2) * sizeof(float);
}

// Workgroups of one attention launch.
static int64_t attn_grid_splits(int64_t batch, int nkv, int64_t max_len, int64_t window) {
  const int64_t span = window > 0 && window < max_len ? window : max_len;
  int64_t grid_splits = cdiv(kTargetGroups, batch * nkv);
  if (grid_splits > cdiv(span, kSplit)) grid_splits = cdiv(span, kSplit);
  return grid_splits;
}

// The splits of one (row, KV head) wait on each other, so they must fit on the
// device at once: their number is capped at the kernel's resident capacity
// (compute units x occupancy).  Workgroups are dispatched in index order and a
// (row, KV head)'s splits are consecutive, so every earlier pair has all of
// its splits placed and finishes; with the O projection in the launch the
// whole grid meets at one barrier and must be resident.
template <int HD, bool XL>
static const void* attn_kernel(bool fused) {
  return fused ? reinterpret_cast<const void*>(&k_decode_attn<true, HD, XL>)
               : reinterpret_cast<const void*>(&k_decode_attn<false, HD, XL>);
}

static int attn_capacity(bool fused, int head_dim, int64_t* cap, bool xl = false) {
  const void* k = head_dim == 128 ? (xl ? attn_kernel<128, true>(fused) : attn_kernel<128, false>(fused))
                                  : (xl ? attn_kernel<64, true>(fused) : attn_kernel<64, false>(fused));
  return resident_capacity(k, kAttnThreads, cap);
}

// The XCD-local form (XL in k_decode_attn): chosen when the pair's splits
// need merging, their flags fit the pair's arrival line, one XCD holds a
// pair's splits at once (the whole grid when the O projection's barrier spans
// it) and the GPU hands workgroups to XCDs round robin.  MAPLE_AMD_ATTN=grid
// keeps the cross-XCD form (for A/B timing).
static bool attn_xcd_form(bool fused, int hd, int64_t n_pairs, int64_t splits, bool with_o, hipStream_t s) {
  if (splits < 2 || splits > kSyncLine - 1) return false;
  const char* force = getenv("MAPLE_AMD_ATTN");
  if (force && strcmp(force, "grid") == 0) return false;
  int64_t cap = 0;
  if (attn_capacity(fused, hd, &cap, true) != MA_OK) return false;
  const int64_t n_wg = kXcds * splits * cdiv(n_pairs, kXcds);
  if (kXcds * splits > cap || (with_o && n_wg > cap)) return false;
  bool ok = false;
  return xcd_round_robin(s, &ok) == MA_OK && ok;
}

extern "C" int ma_decode_attn_o_supported(int64_t batch, int n_heads, int n_kv_heads, int head_dim,
                                          int64_t max_len, int64_t window, int64_t o_rows) {
  if (batch != 1 || n_kv_heads < 1 || max_len < 1 ||
      static_cast<int64_t>(n_heads) * head_dim != 32 * kOWords * 16)
    return 0;
  if (head_dim != 64 && head_dim != 128) return 0;
  const int64_t n_wg = attn_grid_splits(batch, n_kv_heads, max_len, window) * n_kv_heads;
  int64_t cap = 0;
  if (attn_capacity(true, head_dim, &cap) != MA_OK || n_wg > cap) return 0;
  return n_wg >= kBarGroups && o_rows >= 1 && o_rows <= n_wg * 8 * kOPass;
}

extern "C" int ma_decode_attn_form(int64_t batch, int n_kv_heads, int head_dim, int64_t max_len, int64_t window,
                                   int fused, int with_o) {
  if (batch < 1 || n_kv_heads < 1 || max_len < 1 || (head_dim != 64 && head_dim != 128)) return -1;
  const int64_t splits = attn_grid_splits(batch, n_kv_heads, max_len, window);
  return attn_xcd_form(fused != 0, head_dim, batch * n_kv_heads, splits, with_o != 0, nullptr) ? 1 : 0;
}

// Shared launch of k_decode_attn for the two entry points below.
static int launch_attn(bool fused, const void* src, int64_t ldq, const void* qn_w,
                       const void* kn_w, int w_dt, const RopeSrc& rope, float eps,
                       void* k_cache, void* v_cache, int64_t cache_rows, int64_t max_len,
                       const int64_t* seqlen, const int64_t* row_map, int64_t batch, int nq,
                       int nkv, int hd, int64_t window, float scale, void* out, void* workspace,
                       size_t workspace_bytes, const uint32_t* o_w, const void* o_alpha,
                       int o_alpha_dt, int64_t o_rows, void* o_out, hipStream_t s,
                       const char* what) {
  if (!workspace || workspace_bytes < ma_gqa_workspace_bytes(batch, nkv, max_len, hd))
    return fail(MA_EVALUE, "%s: workspace too small", what);
  if (!aligned16(workspace) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out) ||
      (!fused && !aligned16(src)))
    return fail(MA_EVALUE, "%s: buffers must be 16-byte aligned", what);
  const int64_t max_splits = max_splits_for(max_len);
  if (batch * nkv * max_splits * kMaxGroup * hd * 4 >= (int64_t{1} << 32))
    return fail(MA_EVALUE, "%s: batch x kv heads x max_len too large for one launch", what);
  int64_t grid_splits = attn_grid_splits(batch, nkv, max_len, window);
  int64_t capacity = 0;
  if (int rc = attn_capacity(fused, hd, &capacity)) return rc;
  if (grid_splits > capacity) grid_splits = capacity;
  auto* sync = static_cast<uint32_t*>(workspace);
  float* acc = reinterpret_cast<float*>(static_cast<char*>(workspace) + sync_bytes(batch, nkv));
  float* ml = acc + static_cast<size_t>(batch) * nkv * max_splits * kMaxGroup * hd;
  const bool xl = attn_xcd_form(fused, hd, batch * nkv, grid_splits, o_w != nullptr, s);
  const dim3 grid = xl ? dim3(static_cast<unsigned>(kXcds * grid_splits * cdiv(batch * nkv, kXcds)))
                       : dim3(static_cast<unsigned>(grid_splits), static_cast<unsigned>(nkv),
                              static_cast<unsigned>(batch));
  if (o_w) {
    const int64_t n_wg = static_cast<int64_t>(grid.x) * grid.y * grid.z;
    if (batch != 1 || static_cast<int64_t>(nq) * hd != 32 * kOWords * 16)
      return fail(MA_EVALUE, "%s: the O projection in the launch needs batch 1 and n_heads x head_dim = %d",
                  what, 32 * kOWords * 16);
    if (n_wg > capacity)
      return fail(MA_ERUNTIME, "%s: the O projection's %lld workgroups wait on each other but the device holds %lld",
                  what, static_cast<long long>(n_wg), static_cast<long long>(capacity));
    if (n_wg < kBarGroups || o_rows < 1 || o_rows > n_wg * 8 * kOPass)
      return fail(MA_EVALUE, "%s: O projection of %lld rows over %lld workgroups unsupported", what,
                  static_cast<long long>(o_rows), static_cast<long long>(n_wg));
    if (!o_alpha || !o_out || !aligned16(o_w))
      return fail(MA_EVALUE, "%s: O projection needs 16-byte aligned weights, alpha and output", what);
    if (o_alpha_dt != MA_F32 && o_alpha_dt != MA_BF16)
      return fail(MA_ETYPE, "%s: O projection alpha dtype %d", what, o_alpha_dt);
  }
#define MA_ATTN_ARGS                                                                            \
  seqlen, row_map, static_cast<const uint16_t*>(src), ldq, nq, nkv, static_cast<int>(batch),   \
      static_cast<int>(grid_splits), max_len, qn_w, kn_w, w_dt, rope, eps,                      \
      static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), cache_rows, window,     \
      scale, static_cast<int>(max_splits), sync, acc, ml, static_cast<uint16_t*>(out), o_w,     \
      o_alpha, o_alpha_dt, static_cast<int>(o_rows), static_cast<uint16_t*>(o_out)
#define MA_ATTN_LAUNCH(F, H)                                                                      \
  do {                                                                                          \
    if (xl)                                                                                     \
      hipLaunchKernelGGL((k_decode_attn<F, H, true>), grid, dim3(kAttnThreads), 0, s, MA_ATTN_ARGS); \
    else                                                                                        \
      hipLaunchKernelGGL((k_decode_attn<F, H, false>), grid, dim3(kAttnThreads), 0, s, MA_ATTN_ARGS); \
  } while (0)
  if (fused && hd == 128)
    MA_ATTN_LAUNCH(true, 128);
  else if (fused)
    MA_ATTN_LAUNCH(true, 64);
  else if (hd == 128)
    MA_ATTN_LAUNCH(false, 128);
  else
    MA_ATTN_LAUNCH(false, 64);
#undef MA_ATTN_LAUNCH
#undef MA_ATTN_ARGS
  return check_launch(what);
}

extern "C" int ma_decode_gqa_attn(const void* q, int64_t batch, int n_heads, int n_kv_heads,
                                  int head_dim, const void* k_cache, const void* v_cache,
                                  int64_t cache_rows, int64_t max_len, const int64_t* seqlen,
                                  const int64_t* row_map, int64_t window, float scale, void* out,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  const char* what = "decode_gqa_attn";
  if (int rc = check_heads(batch, n_heads, n_kv_heads, head_dim, max_len, cache_rows, row_map, what))
    return rc;
  if (batch == 0) return MA_OK;
  const RopeSrc none{nullptr, nullptr, MA_F32, 0, 0, 0, 0};
  return launch_attn(false, q, 0, nullptr, nullptr, MA_F32, none, 0.f,
                     const_cast<void*>(k_cache), const_cast<void*>(v_cache), cache_rows, max_len,
                     seqlen, row_map, batch, n_heads, n_kv_heads, head_dim, window, scale, out, workspace,
                     workspace_bytes, nullptr, nullptr, 0, 0, nullptr,
                     static_cast<hipStream_t>(stream), what);
}

extern "C" int ma_decode_attn_fused(const void* qkv, int64_t ldq, int64_t batch, int n_heads,
                                    int n_kv_heads, int head_dim, const void* q_norm_w,
                                    const void* k_norm_w, int w_dtype, const void* cos,
                                    const void* sin, int cs_dtype, int64_t ld_cs, int64_t n_pos,
                                    int rotary_dim, int use_rope, float eps,
                                    const int64_t* seqlen, const int64_t* row_map, void* k_cache,
                                    void* v_cache, int64_t cache_rows, int64_t max_len,
                                    int64_t window, float scale, void* out, void* workspace,
                                    size_t workspace_bytes, const uint32_t* o_w,
                                    const void* o_alpha, int o_alpha_dtype, int64_t o_rows,
                                    void* o_out, void* stream) {
  const char* what = "decode_attn_fused";
  if (int rc = check_heads(batch, n_heads, n_kv_heads, head_dim, max_len, cache_rows, row_map, what))
    return rc;
  const RopeSrc rope{cos, sin, cs_dtype, ld_cs, n_pos, rotary_dim, use_rope};
  if (int rc = check_rope(rope, head_dim, what)) return rc;
  if (w_dtype != MA_F32 && w_dtype != MA_BF16 && w_dtype != MA_F16)
    return fail(MA_ETYPE, "%s: norm weight dtype %d unsupported", what, w_dtype);
  if (ldq < static_cast<int64_t>(n_heads + 2 * n_kv_heads) * head_dim)
    return fail(MA_EVALUE, "%s: qkv row stride too small", what);
  if (batch == 0) return MA_OK;
  return launch_attn(true, qkv, ldq, q_norm_w, k_norm_w, w_dtype, rope, eps, k_cache, v_cache,
                     cache_rows, max_len, seqlen, row_map, batch, n_heads, n_kv_heads, head_dim, window,
                     scale, out, workspace, workspace_bytes, o_w, o_alpha, o_alpha_dtype, o_rows,
                     o_out, static_cast<hipStream_t>(stream), what);
}
