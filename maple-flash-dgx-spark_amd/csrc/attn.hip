// Decode attention for q_len = 1 (gfx950): QK RMSNorm + partial RoPE + KV
// write, and split-sequence GQA whose partials are merged by the last split
// to finish (a ticket per (row, KV head)), so one launch does the whole
// attention.  A fused entry point also does the QK-norm/RoPE/KV write inside
// the same launch.
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
#include "common.h"

namespace ma {

constexpr int kHeadDim = 64;                // head_dim of the synthetic decoder
constexpr int kSplit = 128;                 // positions per workgroup = threads
constexpr int kMaxGroup = 16;               // query heads per KV head
constexpr int kWRow = kHeadDim + 4;         // LDS row of interleaved V pairs in
                                            // words, padded: rows 4 banks apart
constexpr size_t kCounterAlign = 256;
constexpr int kCombineChunk = 12;           // splits whose partials load together
constexpr int kTargetGroups = 1024;         // workgroups an attention launch aims for

// Device-coherent (agent-scope) 8-byte store / load of two floats: visible to
// workgroups on every XCD once the store has completed, without a fence.
__device__ __forceinline__ void st_coherent2(float* p, float a, float b) {
  const uint64_t v = static_cast<uint64_t>(__float_as_uint(a)) |
                     (static_cast<uint64_t>(__float_as_uint(b)) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 ld_coherent2(const float* p) {
  const uint64_t v = __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<float*>(p)),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__uint_as_float(static_cast<uint32_t>(v)),
                     __uint_as_float(static_cast<uint32_t>(v >> 32)));
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

// cos/sin for lane d of the row used at position ``pos`` of batch row b,
// rounded to bf16 (the activation dtype) as the reference's table gather does.
__device__ __forceinline__ float2 rope_coeffs(const RopeSrc& r, int64_t b, int64_t pos) {
  if (!r.use_rope || r.rot <= 0) return make_float2(1.f, 0.f);
  const int d = threadIdx.x & 63;
  const int64_t row = r.n_pos > 0 ? (pos < r.n_pos ? pos : r.n_pos - 1) : b;
  const int dd = d < r.rot ? d : 0;
  return make_float2(bf16_to_f32(f32_to_bf16(ld_f(r.cos, r.dt, row * r.ld + dd))),
                     bf16_to_f32(f32_to_bf16(ld_f(r.sin, r.dt, row * r.ld + dd))));
}

// RMSNorm of one head held one dim per lane (wave-wide), then rotate-half
// RoPE on the first ``rot`` dims with this lane's coefficients ``cs``.
__device__ __forceinline__ float norm_rope_lane(float x, float w, float2 cs, const RopeSrc& r,
                                                float eps) {
  const int d = threadIdx.x & 63;
  const float ss = group_sum<64>(x * x);
  float y = x * rsqrtf(ss / kHeadDim + eps) * w;
  if (r.use_rope && r.rot > 0) {
    const int half = r.rot / 2;
    const float other = __shfl(y, d < half ? d + half : d - half, 64);
    if (d < r.rot) y = d < half ? y * cs.x - other * cs.y : y * cs.x + other * cs.y;
  }
  return y;
}

__device__ __forceinline__ int64_t clamp64(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

// One wave per (head slot, row): q heads [0, nq), k heads [nq, nq + nkv), v
// heads after that.  Lane d owns dimension d.
__global__ __launch_bounds__(64) void k_qk_norm_rope_store(
    const uint16_t* __restrict__ qkv, int64_t ldq, const void* __restrict__ q_w,
    const void* __restrict__ k_w, int w_dt, RopeSrc rope, float eps,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache, const int64_t* __restrict__ seqlen,
    const int64_t* __restrict__ row_map, int64_t cache_rows, int nq, int nkv, int64_t max_len) {
  const int d = threadIdx.x;
  const int hs = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int64_t pos = clamp64(seqlen[b], 0, max_len - 1);
  const int64_t crow = row_map ? clamp64(row_map[b], 0, cache_rows - 1) : b;
  const uint16_t* row = qkv + b * ldq;
  if (hs >= nq + nkv) {  // V: copy
    const int h = hs - nq - nkv;
    v_cache[((crow * nkv + h) * max_len + pos) * kHeadDim + d] = row[(nq + nkv + h) * kHeadDim + d];
    return;
  }
  const bool is_q = hs < nq;
  const float x = bf16_to_f32(row[hs * kHeadDim + d]);
  const float w = ld_f(is_q ? q_w : k_w, w_dt, d);
  const float2 cs = rope_coeffs(rope, b, pos);
  const uint16_t yb = f32_to_bf16(norm_rope_lane(x, w, cs, rope, eps));
  if (is_q)
    q_out[(b * nq + hs) * kHeadDim + d] = yb;
  else
    k_cache[((crow * nkv + (hs - nq)) * max_len + pos) * kHeadDim + d] = yb;
}

// Loads of the K and V rows of position t (clamped to hi - 1 when dead).
__device__ __forceinline__ void load_kv_rows(const uint16_t* __restrict__ k_cache,
                                             const uint16_t* __restrict__ v_cache, int64_t row,
                                             uint4 kr[8], uint4 vr[8]) {
  const uint4* kp = reinterpret_cast<const uint4*>(k_cache + row * kHeadDim);
  const uint4* vp = reinterpret_cast<const uint4*>(v_cache + row * kHeadDim);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    vr[i] = vp[i];
    kr[i] = kp[i];
  }
}

// One workgroup (128 threads, 2 waves) per (split, KV head, row); a split
// walks chunks of 128 positions (the grid holds about kTargetGroups
// workgroups; rows x KV heads x splits), thread t on position lo + t:
//   q:     FUSED normalises + ropes the group's q heads from the qkv row; the
//          split holding position seqlen[b] also makes the new K/V (used in
//          place of what it read, stored to the cache at the end).
//          Otherwise q is read.
//   chunk: V rows of positions 2m, 2m+1 (lanes t, t^1) are interleaved into
//          LDS as bf16 pairs W[m][d] = (v_2m[d], v_2m+1[d]); scores q.k *
//          scale (dot2 over dim pairs) -> LDS; the next chunk's K/V loads
//          are issued; online softmax per head (running max and sum, P
//          rounded to bf16); P.V by thread (head, 4 dims) with one dot2 per
//          position pair, the accumulator rescaled by exp(m_old - m_new).
//   end:   one split: normalise and store.  Several: write (acc, m, l)
//          partials with device-coherent stores; the last split of the (row,
//          KV head) to take a ticket merges them and resets the ticket.
template <bool FUSED>
__global__ __launch_bounds__(kSplit) void k_decode_attn(
    const uint16_t* __restrict__ src, int64_t ldq, const void* __restrict__ qn_w,
    const void* __restrict__ kn_w, int w_dt, RopeSrc rope, float eps,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache, int64_t cache_rows,
    int64_t max_len, const int64_t* __restrict__ seqlen, const int64_t* __restrict__ row_map,
    int nq, int nkv, int64_t window, float scale, int max_splits, uint32_t* __restrict__ tickets,
    float* __restrict__ part_acc, float* __restrict__ part_ml, uint16_t* __restrict__ out) {
  __shared__ __align__(16) uint32_t qs[kMaxGroup][kHeadDim / 2];
  __shared__ __align__(16) uint32_t vw[kSplit / 2][kWRow];
  __shared__ __align__(16) float sc[kMaxGroup][kSplit];
  __shared__ __align__(16) uint16_t pb[kMaxGroup][kSplit];
  __shared__ __align__(16) uint32_t kvnew[2][kHeadDim / 2];
  __shared__ float hm[kMaxGroup], hl[kMaxGroup], hr[kMaxGroup];
  __shared__ int s_last;
  const int sp = blockIdx.x, kvh = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  // wave index, made visibly wave-uniform so that branches on it stay scalar
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int group = nq / nkv;
  const int64_t pos = clamp64(seqlen[b], 0, max_len - 1);
  const int64_t kv_len = pos + 1;
  const int64_t start = (window > 0 && kv_len > window) ? kv_len - window : 0;
  const int n_chunks = static_cast<int>(cdiv(kv_len - start, kSplit));
  const int cps = static_cast<int>(cdiv(n_chunks, gridDim.x));  // chunks per split
  const int n_spl = static_cast<int>(cdiv(n_chunks, cps));
  if (sp >= n_spl) return;
  const int c_beg = sp * cps;
  const int c_end = c_beg + cps < n_chunks ? c_beg + cps : n_chunks;
  const int64_t crow = row_map ? clamp64(row_map[b], 0, cache_rows - 1) : b;
  const int64_t base = (crow * nkv + kvh) * max_len;
  const bool owns_pos = FUSED && sp == n_spl - 1;

  // First chunk's K/V rows: the longest latency.
  uint4 kr[8], vr[8];
  {
    const int64_t lo = start + static_cast<int64_t>(c_beg) * kSplit;
    const int64_t hi = lo + kSplit < kv_len ? lo + kSplit : kv_len;
    const int64_t t = lo + tid;
    load_kv_rows(k_cache, v_cache, base + (t < hi ? t : hi - 1), kr, vr);
  }
  uint16_t new_kv = 0;  // FUSED owner split: this wave's new K (wave 0) or V (wave 1)
  if constexpr (FUSED) {
    // Every load of the prologue is issued before any of them is used.
    const uint16_t* row = src + b * ldq;
    uint16_t xq[kMaxGroup / 2];
#pragma unroll
    for (int i = 0; i < kMaxGroup / 2; ++i) {
      const int hh = wv + 2 * i;
      xq[i] = hh < group ? row[(kvh * group + hh) * kHeadDim + lane] : uint16_t(0);
    }
    const uint16_t xkv = owns_pos ? row[(nq + kvh + (wv ? nkv : 0)) * kHeadDim + lane] : uint16_t(0);
    const float wq = ld_f(qn_w, w_dt, lane);
    const float wk = ld_f(kn_w, w_dt, lane);
    const float2 cs = rope_coeffs(rope, b, pos);
#pragma unroll
    for (int i = 0; i < kMaxGroup / 2; ++i) {
      const int hh = wv + 2 * i;
      if (hh < group) {
        const float y = norm_rope_lane(bf16_to_f32(xq[i]), wq, cs, rope, eps);
        reinterpret_cast<uint16_t*>(qs[hh])[lane] = f32_to_bf16(y);
      }
    }
    if (owns_pos) {
      new_kv = xkv;  // wave 1: V is stored as is
      if (wv == 0) new_kv = f32_to_bf16(norm_rope_lane(bf16_to_f32(xkv), wk, cs, rope, eps));
      reinterpret_cast<uint16_t*>(kvnew[wv])[lane] = new_kv;
    }
  } else {
    const uint32_t* qsrc = reinterpret_cast<const uint32_t*>(src + (b * nq + kvh * group) * kHeadDim);
    for (int i = tid; i < group * (kHeadDim / 2); i += kSplit)
      qs[i / (kHeadDim / 2)][i % (kHeadDim / 2)] = qsrc[i];
  }
  if (tid < group) {
    hm[tid] = -INFINITY;
    hl[tid] = 0.f;
  }
  __syncthreads();

  float o[kMaxGroup / 8][4] = {};  // thread items: (head, 4 dims), up to 2 per thread
  for (int c = c_beg; c < c_end; ++c) {
    const int64_t lo = start + static_cast<int64_t>(c) * kSplit;
    const int64_t hi = lo + kSplit < kv_len ? lo + kSplit : kv_len;
    const int64_t t = lo + tid;
    const bool live = t < hi;
    if constexpr (FUSED) {  // the position written by this launch: use the new K/V
      const bool use_new = owns_pos && t == pos;
#pragma unroll
      for (int i = 0; i < 8; ++i) {  // selects, so that kr/vr stay in registers
        const uint4 nk = *reinterpret_cast<const uint4*>(&kvnew[0][4 * i]);
        const uint4 nv = *reinterpret_cast<const uint4*>(&kvnew[1][4 * i]);
        kr[i].x = use_new ? nk.x : kr[i].x;
        kr[i].y = use_new ? nk.y : kr[i].y;
        kr[i].z = use_new ? nk.z : kr[i].z;
        kr[i].w = use_new ? nk.w : kr[i].w;
        vr[i].x = use_new ? nv.x : vr[i].x;
        vr[i].y = use_new ? nv.y : vr[i].y;
        vr[i].z = use_new ? nv.z : vr[i].z;
        vr[i].w = use_new ? nv.w : vr[i].w;
      }
    }
    // Interleave V with the neighbouring position: the even lane of a pair
    // builds dims 0..31, the odd lane dims 32..63.
    {
      uint32_t v[32];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        v[4 * i] = vr[i].x;
        v[4 * i + 1] = vr[i].y;
        v[4 * i + 2] = vr[i].z;
        v[4 * i + 3] = vr[i].w;
      }
      const bool odd = tid & 1;
      uint32_t w[32];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint32_t mine = odd ? v[16 + j] : v[j];
        const uint32_t send = odd ? v[j] : v[16 + j];
        const uint32_t other = __builtin_amdgcn_update_dpp(0, send, 0xB1, 0xF, 0xF, false);
        const uint32_t e = odd ? other : mine, od = odd ? mine : other;  // positions 2m, 2m+1
        w[2 * j] = (e & 0xffffu) | (od << 16);
        w[2 * j + 1] = (e >> 16) | (od & 0xffff0000u);
      }
      uint32_t* dst = &vw[tid >> 1][odd ? kHeadDim / 2 : 0];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        *reinterpret_cast<uint4*>(dst + 4 * i) =
            make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
    }
    for (int hh = 0; hh < group; ++hh) {
      float a0 = 0.f, a1 = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint4 qq = *reinterpret_cast<const uint4*>(&qs[hh][4 * i]);
        a0 = dot2(kr[i].x, qq.x, a0);
        a1 = dot2(kr[i].y, qq.y, a1);
        a0 = dot2(kr[i].z, qq.z, a0);
        a1 = dot2(kr[i].w, qq.w, a1);
      }
      sc[hh][tid] = live ? (a0 + a1) * scale : -INFINITY;
    }
    __syncthreads();
    if (c + 1 < c_end) {  // next chunk's rows, in flight during softmax and P.V
      const int64_t lo2 = lo + kSplit;
      const int64_t hi2 = lo2 + kSplit < kv_len ? lo2 + kSplit : kv_len;
      const int64_t t2 = lo2 + tid;
      load_kv_rows(k_cache, v_cache, base + (t2 < hi2 ? t2 : hi2 - 1), kr, vr);
    }
    // Online softmax: wave w takes heads w, w + 2, ...; lane owns positions
    // lane and lane + 64.  Position lo is always live, so the max is finite.
    for (int hh = wv; hh < group; hh += 2) {
      const float v0 = sc[hh][lane], v1 = sc[hh][lane + 64];
      const float m_old = hm[hh];
      const float m = fmaxf(m_old, wave_max(fmaxf(v0, v1)));
      const float p0 = v0 == -INFINITY ? 0.f : expf(v0 - m);
      const float p1 = v1 == -INFINITY ? 0.f : expf(v1 - m);
      const float l = group_sum<64>(p0 + p1);
      pb[hh][lane] = f32_to_bf16(p0);  // P in bf16 for P.V
      pb[hh][lane + 64] = f32_to_bf16(p1);
      if (lane == 0) {
        const float r = expf(m_old - m);  // 0 on the first chunk
        hm[hh] = m;
        hl[hh] = hl[hh] * r + l;
        hr[hh] = r;
      }
    }
    __syncthreads();
    // P.V: thread (head hh, dims 4dq..4dq+3), one dot2 per position pair.
    // Dead positions have P = 0 and a finite (duplicated) V row.
    const int npairs = (static_cast<int>(hi - lo) + 1) >> 1;
#pragma unroll
    for (int k = 0; k < kMaxGroup / 8; ++k) {
      const int item = tid + kSplit * k;
      if (item < group * 16) {
        const int hh = item >> 4, dq = item & 15;
        const uint32_t* pw = reinterpret_cast<const uint32_t*>(pb[hh]);
        const float r = hr[hh];
        float o0 = o[k][0] * r, o1 = o[k][1] * r, o2 = o[k][2] * r, o3 = o[k][3] * r;
#pragma unroll 4
        for (int m = 0; m < npairs; ++m) {
          const uint32_t pp = pw[m];
          const uint4 vv = *reinterpret_cast<const uint4*>(&vw[m][4 * dq]);
          o0 = dot2(vv.x, pp, o0);
          o1 = dot2(vv.y, pp, o1);
          o2 = dot2(vv.z, pp, o2);
          o3 = dot2(vv.w, pp, o3);
        }
        o[k][0] = o0;
        o[k][1] = o1;
        o[k][2] = o2;
        o[k][3] = o3;
      }
    }
    __syncthreads();  // vw / sc / pb are rewritten by the next chunk
  }
  // The new K/V go to the cache last: a store to the cache ahead of the reads
  // of kr makes the compiler keep kr in scratch memory.
  if (owns_pos) (wv == 0 ? k_cache : v_cache)[(base + pos) * kHeadDim + lane] = new_kv;
  const int64_t pidx = (b * nkv + kvh) * max_splits + sp;
#pragma unroll
  for (int k = 0; k < kMaxGroup / 8; ++k) {
    const int item = tid + kSplit * k;
    if (item < group * 16) {
      const int hh = item >> 4, dq = item & 15;
      if (n_spl == 1) {
        const float inv = 1.f / hl[hh];
        uint2 r;
        r.x = pack_bf16x2_rn(o[k][0] * inv, o[k][1] * inv);
        r.y = pack_bf16x2_rn(o[k][2] * inv, o[k][3] * inv);
        *reinterpret_cast<uint2*>(out + (b * nq + kvh * group + hh) * kHeadDim + 4 * dq) = r;
      } else {
        float* pa = part_acc + (pidx * kMaxGroup + hh) * kHeadDim + 4 * dq;
        st_coherent2(pa, o[k][0], o[k][1]);
        st_coherent2(pa + 2, o[k][2], o[k][3]);
      }
    }
  }
  if (n_spl == 1) return;
  if (tid < group) st_coherent2(part_ml + (pidx * kMaxGroup + tid) * 2, hm[tid], hl[tid]);
  // The partials were written with device-coherent stores; wait until they
  // have all completed, then take a ticket.  (No device-scope fence: on this
  // GPU that writes back the whole L2, which thousands of splits cannot
  // afford.)
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  uint32_t* ticket = tickets + b * nkv + kvh;
  if (tid == 0) s_last = atomicAdd(ticket, 1u) == static_cast<uint32_t>(n_spl - 1);
  __syncthreads();
  if (!s_last) return;
  // Merge: one pass with a running max, kCombineChunk splits' loads at a time.
  const int64_t p0 = (b * nkv + kvh) * max_splits;
  for (int item = tid; item < group * 16; item += kSplit) {
    const int hh = item >> 4, dq = item & 15;
    float mx = -INFINITY, den = 0.f, n0 = 0.f, n1 = 0.f, n2 = 0.f, n3 = 0.f;
    for (int s0 = 0; s0 < n_spl; s0 += kCombineChunk) {
      float2 ml[kCombineChunk], a01[kCombineChunk], a23[kCombineChunk];
#pragma unroll
      for (int u = 0; u < kCombineChunk; ++u) {
        const int s = s0 + u < n_spl ? s0 + u : n_spl - 1;
        const int64_t q = (p0 + s) * kMaxGroup + hh;
        ml[u] = ld_coherent2(part_ml + q * 2);
        a01[u] = ld_coherent2(part_acc + q * kHeadDim + 4 * dq);
        a23[u] = ld_coherent2(part_acc + q * kHeadDim + 4 * dq + 2);
      }
      MA_ISSUE_FENCE();
#pragma unroll
      for (int u = 0; u < kCombineChunk; ++u) {  // no early exit: arrays stay in registers
        const bool ok = s0 + u < n_spl;  // u = 0 always is, so mx is finite after it
        const float m = ok ? ml[u].x : -INFINITY;
        const float mn = fmaxf(mx, m);
        const float r = expf(mx - mn), w = ok ? expf(m - mn) : 0.f;
        den = den * r + w * ml[u].y;
        n0 = n0 * r + w * a01[u].x;
        n1 = n1 * r + w * a01[u].y;
        n2 = n2 * r + w * a23[u].x;
        n3 = n3 * r + w * a23[u].y;
        mx = mn;
      }
    }
    uint2 r;
    r.x = pack_bf16x2_rn(n0 / den, n1 / den);
    r.y = pack_bf16x2_rn(n2 / den, n3 / den);
    *reinterpret_cast<uint2*>(out + (b * nq + kvh * group + hh) * kHeadDim + 4 * dq) = r;
  }
  if (tid == 0) atomicExch(ticket, 0u);
}

size_t ticket_bytes(int64_t batch, int nkv) {
  const size_t n = static_cast<size_t>(batch) * nkv * sizeof(uint32_t);
  return (n + kCounterAlign - 1) / kCounterAlign * kCounterAlign;
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
  if (head_dim != kHeadDim)
    return fail(MA_EVALUE, "%s: head_dim %d unsupported (64)", what, head_dim);
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
  hipLaunchKernelGGL(k_qk_norm_rope_store, grid, dim3(64), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(qkv), ldq, q_norm_w, k_norm_w, w_dtype, rope,
                     eps, static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_cache),
                     static_cast<uint16_t*>(v_cache), seqlen, row_map, cache_rows, n_heads,
                     n_kv_heads, max_len);
  return check_launch(what);
}

extern "C" size_t ma_gqa_workspace_bytes(int64_t batch, int n_kv_heads, int64_t max_len) {
  if (batch < 0 || n_kv_heads < 1 || max_len < 1) return 0;
  const size_t parts = static_cast<size_t>(batch) * n_kv_heads * max_splits_for(max_len) * kMaxGroup;
  return ticket_bytes(batch, n_kv_heads) + parts * (kHeadDim + 2) * sizeof(float);
}

// Shared launch of k_decode_attn for the two entry points below.
static int launch_attn(bool fused, const void* src, int64_t ldq, const void* qn_w,
                       const void* kn_w, int w_dt, const RopeSrc& rope, float eps,
                       void* k_cache, void* v_cache, int64_t cache_rows, int64_t max_len,
                       const int64_t* seqlen, const int64_t* row_map, int64_t batch, int nq,
                       int nkv, int64_t window, float scale, void* out, void* workspace,
                       size_t workspace_bytes, hipStream_t s, const char* what) {
  if (!workspace || workspace_bytes < ma_gqa_workspace_bytes(batch, nkv, max_len))
    return fail(MA_EVALUE, "%s: workspace too small", what);
  if (!aligned16(workspace) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out) ||
      (!fused && !aligned16(src)))
    return fail(MA_EVALUE, "%s: buffers must be 16-byte aligned", what);
  const int64_t max_splits = max_splits_for(max_len);
  const int64_t span = window > 0 && window < max_len ? window : max_len;
  const int64_t pairs = batch * nkv;
  int64_t grid_splits = cdiv(kTargetGroups, pairs);
  if (grid_splits > cdiv(span, kSplit)) grid_splits = cdiv(span, kSplit);
  auto* tickets = static_cast<uint32_t*>(workspace);
  float* acc = reinterpret_cast<float*>(static_cast<char*>(workspace) + ticket_bytes(batch, nkv));
  float* ml = acc + static_cast<size_t>(batch) * nkv * max_splits * kMaxGroup * kHeadDim;
  dim3 grid(static_cast<unsigned>(grid_splits), static_cast<unsigned>(nkv),
            static_cast<unsigned>(batch));
#define MA_ATTN_ARGS                                                                            \
  static_cast<const uint16_t*>(src), ldq, qn_w, kn_w, w_dt, rope, eps,                          \
      static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), cache_rows, max_len,    \
      seqlen, row_map, nq, nkv, window, scale, static_cast<int>(max_splits), tickets, acc, ml, \
      static_cast<uint16_t*>(out)
  if (fused)
    hipLaunchKernelGGL(k_decode_attn<true>, grid, dim3(kSplit), 0, s, MA_ATTN_ARGS);
  else
    hipLaunchKernelGGL(k_decode_attn<false>, grid, dim3(kSplit), 0, s, MA_ATTN_ARGS);
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
                     seqlen, row_map, batch, n_heads, n_kv_heads, window, scale, out, workspace,
                     workspace_bytes, static_cast<hipStream_t>(stream), what);
}

extern "C" int ma_decode_attn_fused(const void* qkv, int64_t ldq, int64_t batch, int n_heads,
                                    int n_kv_heads, int head_dim, const void* q_norm_w,
                                    const void* k_norm_w, int w_dtype, const void* cos,
                                    const void* sin, int cs_dtype, int64_t ld_cs, int64_t n_pos,
                                    int rotary_dim, int use_rope, float eps,
                                    const int64_t* seqlen, const int64_t* row_map, void* k_cache,
                                    void* v_cache, int64_t cache_rows, int64_t max_len,
                                    int64_t window, float scale, void* out, void* workspace,
                                    size_t workspace_bytes, void* stream) {
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
                     cache_rows, max_len, seqlen, row_map, batch, n_heads, n_kv_heads, window,
                     scale, out, workspace, workspace_bytes, static_cast<hipStream_t>(stream), what);
}
