// Decode attention for q_len = 1 (gfx950): QK RMSNorm + partial RoPE + KV
// write, then split-sequence GQA and a log-sum-exp combine.
//
// Semantics of reference src/maple_run/kernels/decode_attn.py:
//   apply_qkv_decode (:15-163, :362-439): per head, x * rsqrt(mean(x^2) + eps)
//     * w; rotate-half RoPE on the first rotary_dim dims with cos/sin taken
//     from a float32 table rounded to the activation dtype (model.py:94-109);
//     K and V stored at position seqlen[b] of cache row b.
//   decode_gqa_attn (:166-359): over positions [start, min(seqlen[b] + 1,
//     max_len)), start = kv_len - window for a sliding window; scores
//     q.k * scale, online softmax, P rounded to bf16 before P.V, float32
//     accumulation, splits merged with exp(m_s - max) weights.
// Positions at or beyond max_len are clamped to the last slot so nothing is
// ever written or read outside the cache.
#include "common.h"

namespace ma {

constexpr int kHeadDim = 64;       // head_dim of the synthetic decoder
constexpr int kSplitTokens = 256;  // positions per GQA workgroup
constexpr int kMaxGroup = 16;      // query heads per KV head

// One wave per (head slot, row): q heads [0, nq), k heads [nq, nq + nkv),
// v heads after that.  Lane d owns dimension d (head_dim 64).
__global__ __launch_bounds__(64) void k_qk_norm_rope_store(
    const uint16_t* __restrict__ qkv, int64_t ldq, const float* __restrict__ q_w,
    const float* __restrict__ k_w, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, int64_t n_pos, int rot, int use_rope,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache, const int64_t* __restrict__ seqlen, int nq, int nkv,
    int64_t max_len, float eps) {
  const int d = threadIdx.x;
  const int hs = blockIdx.x;
  const int64_t b = blockIdx.y;
  int64_t pos = seqlen[b];
  pos = pos < 0 ? 0 : (pos >= max_len ? max_len - 1 : pos);
  const uint16_t* row = qkv + b * ldq;
  if (hs >= nq + nkv) {  // V: copy
    const int h = hs - nq - nkv;
    v_cache[((b * nkv + h) * max_len + pos) * kHeadDim + d] = row[(nq + nkv + h) * kHeadDim + d];
    return;
  }
  const bool is_q = hs < nq;
  const int h = is_q ? hs : hs - nq;
  const float x = bf16_to_f32(row[hs * kHeadDim + d]);
  const float ss = group_sum<64>(x * x);
  const float rstd = rsqrtf(ss / kHeadDim + eps);
  float y = x * rstd * (is_q ? q_w[d] : k_w[d]);
  if (use_rope && d < rot) {
    const int half = rot / 2;
    const int64_t p = pos < n_pos ? pos : n_pos - 1;
    // cos/sin rounded to the activation dtype, as the reference's table gather.
    const float c = bf16_to_f32(f32_to_bf16(cos_t[p * rot + d]));
    const float s = bf16_to_f32(f32_to_bf16(sin_t[p * rot + d]));
    const float other = __shfl(y, d < half ? d + half : d - half, 64);
    y = d < half ? y * c - other * s : y * c + other * s;
  }
  const uint16_t yb = f32_to_bf16(y);
  if (is_q)
    q_out[(b * nq + h) * kHeadDim + d] = yb;
  else
    k_cache[((b * nkv + h) * max_len + pos) * kHeadDim + d] = yb;
}

// One workgroup (256 threads) per (KV head, split, row).  Phase 1: thread t
// scores position lo + t against the group's query heads (q in LDS, K row
// from global) and stages its V row in LDS.  Phase 2: per-head max / exp /
// sum over the split (P rounded to bf16).  Phase 3: thread (head, dim pair)
// accumulates P.V from LDS.  Writes unnormalised (acc, m, l) partials.
__global__ __launch_bounds__(256) void k_gqa_split(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_cache,
    const uint16_t* __restrict__ v_cache, const int64_t* __restrict__ seqlen, int nq, int nkv,
    int64_t max_len, int64_t window, float scale, int splits, float* __restrict__ part_acc,
    float* __restrict__ part_m, float* __restrict__ part_l) {
  __shared__ __align__(16) uint32_t qs[kMaxGroup][kHeadDim / 2];
  __shared__ __align__(16) uint32_t vs[kSplitTokens][kHeadDim / 2];
  __shared__ float sc[kMaxGroup][kSplitTokens];
  __shared__ float hm[kMaxGroup], hl[kMaxGroup];
  const int kvh = blockIdx.x, sp = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int group = nq / nkv;
  int64_t kv_len = seqlen[b] + 1;
  kv_len = kv_len < 1 ? 1 : (kv_len > max_len ? max_len : kv_len);
  const int64_t start = (window > 0 && kv_len > window) ? kv_len - window : 0;
  const int64_t lo = start + static_cast<int64_t>(sp) * kSplitTokens;
  const int64_t hi = lo + kSplitTokens < kv_len ? lo + kSplitTokens : kv_len;
  const int64_t base = (b * nkv + kvh) * max_len;
  const int64_t pidx = (b * nkv + kvh) * splits + sp;
  if (lo >= hi) {  // empty split: l = 0 is dropped by the combine
    if (tid < group) {
      part_m[pidx * kMaxGroup + tid] = -1e30f;
      part_l[pidx * kMaxGroup + tid] = 0.f;
    }
    return;
  }
  for (int i = tid; i < group * (kHeadDim / 2); i += 256)
    qs[i / (kHeadDim / 2)][i % (kHeadDim / 2)] =
        reinterpret_cast<const uint32_t*>(q + (b * nq + kvh * group) * kHeadDim)[i];
  // Phase 1: scores and V staging, one position per thread.
  const int64_t t = lo + tid;
  const bool live = t < hi;
  const int64_t tt = live ? t : hi - 1;
  uint4 kr[8], vr[8];
  const uint4* kp = reinterpret_cast<const uint4*>(k_cache + (base + tt) * kHeadDim);
  const uint4* vp = reinterpret_cast<const uint4*>(v_cache + (base + tt) * kHeadDim);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    kr[i] = kp[i];
    vr[i] = vp[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 8; ++i) *reinterpret_cast<uint4*>(&vs[tid][4 * i]) = vr[i];
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
  // Phase 2: wave w takes heads w, w + 4, ...; 4 positions per lane.
  for (int hh = wv; hh < group; hh += 4) {
    float v4[4], m = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v4[i] = sc[hh][lane + 64 * i];
      m = fmaxf(m, v4[i]);
    }
    m = wave_max(m);
    float l = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = v4[i] == -INFINITY ? 0.f : expf(v4[i] - m);
      l += p;
      sc[hh][lane + 64 * i] = bf16_to_f32(f32_to_bf16(p));  // P in bf16 for P.V
    }
    l = group_sum<64>(l);
    if (lane == 0) {
      hm[hh] = m;
      hl[hh] = l;
    }
  }
  __syncthreads();
  // Phase 3: thread (head hh, dims 2dp, 2dp+1).
  const int npos = static_cast<int>(hi - lo);
  for (int item = tid; item < group * (kHeadDim / 2); item += 256) {
    const int hh = item / (kHeadDim / 2), dp = item % (kHeadDim / 2);
    float o0 = 0.f, o1 = 0.f;
#pragma unroll 8
    for (int j = 0; j < npos; ++j) {
      const float p = sc[hh][j];
      const uint32_t vv = vs[j][dp];
      o0 += p * __uint_as_float(vv << 16);
      o1 += p * __uint_as_float(vv & 0xffff0000u);
    }
    float* acc = part_acc + (pidx * kMaxGroup + hh) * kHeadDim;
    acc[2 * dp] = o0;
    acc[2 * dp + 1] = o1;
  }
  if (tid < group) {
    part_m[pidx * kMaxGroup + tid] = hm[tid];
    part_l[pidx * kMaxGroup + tid] = hl[tid];
  }
}

// out[b, h, d] = sum_s e^(m_s - M) acc_s / sum_s e^(m_s - M) l_s, stored bf16.
__global__ __launch_bounds__(64) void k_gqa_combine(const float* __restrict__ part_acc,
                                                    const float* __restrict__ part_m,
                                                    const float* __restrict__ part_l, int nq,
                                                    int nkv, int splits,
                                                    uint16_t* __restrict__ out) {
  const int h = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int d = threadIdx.x;
  const int group = nq / nkv;
  const int kvh = h / group, hh = h % group;
  float mx = -1e30f;
  for (int s = 0; s < splits; ++s) {
    const int64_t pidx = (b * nkv + kvh) * splits + s;
    if (part_l[pidx * kMaxGroup + hh] > 0.f) mx = fmaxf(mx, part_m[pidx * kMaxGroup + hh]);
  }
  float num = 0.f, den = 0.f;
  for (int s = 0; s < splits; ++s) {
    const int64_t pidx = (b * nkv + kvh) * splits + s;
    const float l = part_l[pidx * kMaxGroup + hh];
    if (l > 0.f) {
      const float w = expf(part_m[pidx * kMaxGroup + hh] - mx);
      num += w * part_acc[(pidx * kMaxGroup + hh) * kHeadDim + d];
      den += w * l;
    }
  }
  out[(b * nq + h) * kHeadDim + d] = f32_to_bf16(num / den);
}

}  // namespace ma

using namespace ma;

extern "C" int ma_qk_norm_rope_store(const void* qkv, int64_t ldq, int64_t batch, int n_heads,
                                     int n_kv_heads, int head_dim, const float* q_norm_w,
                                     const float* k_norm_w, const float* cos_table,
                                     const float* sin_table, int64_t n_pos, int rotary_dim,
                                     int use_rope, float eps, const int64_t* seqlen,
                                     void* k_cache, void* v_cache, int64_t max_len,
                                     void* q_out, void* stream) {
  if (head_dim != kHeadDim)
    return fail(MA_EVALUE, "qk_norm_rope_store: head_dim %d unsupported (64)", head_dim);
  if (batch < 0 || n_heads < 1 || n_kv_heads < 1 || n_heads % n_kv_heads || max_len < 1 ||
      rotary_dim < 0 || rotary_dim > head_dim || rotary_dim % 2 || (use_rope && n_pos < 1))
    return fail(MA_EVALUE, "qk_norm_rope_store: bad sizes");
  if (batch == 0) return MA_OK;
  dim3 grid(static_cast<unsigned>(n_heads + 2 * n_kv_heads), static_cast<unsigned>(batch));
  hipLaunchKernelGGL(k_qk_norm_rope_store, grid, dim3(64), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(qkv), ldq, q_norm_w, k_norm_w, cos_table,
                     sin_table, n_pos, rotary_dim, use_rope, static_cast<uint16_t*>(q_out),
                     static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), seqlen,
                     n_heads, n_kv_heads, max_len, eps);
  return check_launch("qk_norm_rope_store");
}

extern "C" size_t ma_gqa_workspace_bytes(int64_t batch, int n_kv_heads, int64_t max_len) {
  const int64_t splits = cdiv(max_len, kSplitTokens);
  const int64_t parts = (batch > 0 ? batch : 0) * n_kv_heads * splits * kMaxGroup;
  return static_cast<size_t>(parts) * (kHeadDim + 2) * sizeof(float);
}

extern "C" int ma_decode_gqa_attn(const void* q, int64_t batch, int n_heads, int n_kv_heads,
                                  int head_dim, const void* k_cache, const void* v_cache,
                                  const int64_t* seqlen, int64_t max_len, int64_t window,
                                  float scale, void* out, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  if (head_dim != kHeadDim)
    return fail(MA_EVALUE, "decode_gqa_attn: head_dim %d unsupported (64)", head_dim);
  if (batch < 0 || n_kv_heads < 1 || n_heads % n_kv_heads || n_heads / n_kv_heads > kMaxGroup ||
      max_len < 1)
    return fail(MA_EVALUE, "decode_gqa_attn: bad sizes");
  if (batch == 0) return MA_OK;
  if (!workspace || workspace_bytes < ma_gqa_workspace_bytes(batch, n_kv_heads, max_len))
    return fail(MA_EVALUE, "decode_gqa_attn: workspace too small");
  const int splits = static_cast<int>(cdiv(window > 0 && window < max_len ? window : max_len, kSplitTokens));
  const int64_t parts = batch * n_kv_heads * cdiv(max_len, kSplitTokens) * kMaxGroup;
  float* acc = static_cast<float*>(workspace);
  float* pm = acc + parts * kHeadDim;
  float* pl = pm + parts;
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 g1(static_cast<unsigned>(n_kv_heads), static_cast<unsigned>(splits), static_cast<unsigned>(batch));
  hipLaunchKernelGGL(k_gqa_split, g1, dim3(256), 0, s, static_cast<const uint16_t*>(q),
                     static_cast<const uint16_t*>(k_cache), static_cast<const uint16_t*>(v_cache),
                     seqlen, n_heads, n_kv_heads, max_len, window, scale, splits, acc, pm, pl);
  dim3 g2(static_cast<unsigned>(n_heads), static_cast<unsigned>(batch));
  hipLaunchKernelGGL(k_gqa_combine, g2, dim3(64), 0, s, acc, pm, pl, n_heads, n_kv_heads, splits,
                     static_cast<uint16_t*>(out));
  return check_launch("decode_gqa_attn");
}
