// Fused top-k / temperature / nucleus sampling over the vocabulary (gfx950).
//
// Semantics of the reference's two-launch sampler
// (src/maple_run/kernels/sampler.py:24-103): the top_k largest logits of a row
// (descending, ties at the lower index), p = exp((v - v_max) / T) normalised
// over them, the nucleus drop (a token stays while the mass before it is at
// most top_p), then the inverse CDF at u * (kept mass) for the caller's
// uniform u in [0, 1): the first token whose inclusive prefix exceeds it.
//
// Selection is exact, by keys: key = (order-preserving bits of the float32
// value) << 32 | (0xffffffff - index), so one unsigned 64-bit compare orders
// by value and then by lower index, and every key of a row is distinct.
//
//   k_sample_partial  grid (ceil(vocab / 4096), rows), 256 threads: the
//                     chunk's top_k keys, sorted, into the workspace.
//   k_sample_final    grid (rows), 256 threads: the row's top_k from the
//                     chunk lists, then one wave does softmax, nucleus and
//                     the CDF inversion (top_k <= 64 = one lane per token).
//
// Block top-k (both kernels): the k-th largest of the 256 per-thread maxima
// (a bitonic sort of 256 keys in LDS) is a lower bound T on the k-th largest
// key of the block, because those k maxima are k distinct keys >= T.  Only
// the keys >= T can be in the top k, and only the k threads whose maximum is
// >= T hold any, so at most k x (keys per thread) candidates are compacted
// into LDS and bitonic-sorted; the first k are the answer.
#include "common.h"

namespace ma {

constexpr int kSampleThreads = 256;
constexpr int kSampleChunk = 4096;  // vocabulary entries per partial workgroup
constexpr int kSamplePer = kSampleChunk / kSampleThreads;
constexpr int kSampleMaxK = 64;
constexpr int kSampleFinalPer = 16;  // candidate keys per thread in the final pass

__device__ __forceinline__ uint64_t sample_key(float v, uint32_t idx) {
  const uint32_t b = __float_as_uint(v);
  const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return (static_cast<uint64_t>(o) << 32) | (0xffffffffu - idx);
}

__device__ __forceinline__ float key_value(uint64_t k) {
  const uint32_t o = static_cast<uint32_t>(k >> 32);
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

__device__ __forceinline__ uint32_t key_index(uint64_t k) {
  return 0xffffffffu - static_cast<uint32_t>(k);
}

// Sort s[0, n) descending (n a power of two, at most 4 x kSampleThreads).
__device__ void bitonic_desc(uint64_t* s, int n) {
  const int tid = threadIdx.x;
  for (int size = 2; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < n; i += kSampleThreads) {
        const int j = i ^ stride;
        if (j > i) {
          const uint64_t a = s[i], b = s[j];
          const bool desc = (i & size) == 0;
          if (desc ? (a < b) : (a > b)) {
            s[i] = b;
            s[j] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

struct TopkLds {
  uint64_t tmax[kSampleThreads];
  uint64_t cand[kSampleMaxK * kSampleFinalPer];
  int wsum[kSampleThreads / 64];
};

// The block's k largest keys (key 0 = empty, never selected) into
// L.cand[0, k), descending; entries past the block's non-empty keys are 0.
template <int N>
__device__ void block_topk(const uint64_t (&key)[N], int k, TopkLds& L) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  uint64_t m = 0;
#pragma unroll
  for (int i = 0; i < N; ++i) m = key[i] > m ? key[i] : m;
  L.tmax[tid] = m;
  __syncthreads();
  bitonic_desc(L.tmax, kSampleThreads);
  const uint64_t t = L.tmax[k - 1];
  int c = 0;
#pragma unroll
  for (int i = 0; i < N; ++i) c += (key[i] != 0 && key[i] >= t) ? 1 : 0;
  int inc = c;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(inc, off, 64);
    if (lane >= off) inc += u;
  }
  if (lane == 63) L.wsum[wv] = inc;
  __syncthreads();
  int base = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kSampleThreads / 64; ++w) {
    base += w < wv ? L.wsum[w] : 0;
    total += L.wsum[w];
  }
  int pos = base + inc - c;
#pragma unroll
  for (int i = 0; i < N; ++i)
    if (key[i] != 0 && key[i] >= t) L.cand[pos++] = key[i];
  int n = 1;
  while (n < total || n < k) n <<= 1;
  for (int i = total + tid; i < n; i += kSampleThreads) L.cand[i] = 0;
  __syncthreads();
  bitonic_desc(L.cand, n);
}

template <int DT>
__global__ __launch_bounds__(kSampleThreads) void k_sample_partial(const void* __restrict__ logits,
                                                                   int64_t vocab, int64_t ld, int k,
                                                                   uint64_t* __restrict__ cand) {
  __shared__ TopkLds L;
  const int chunk = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  const int64_t n_chunks = gridDim.x;
  uint64_t key[kSamplePer];
#pragma unroll
  for (int i = 0; i < kSamplePer; ++i) {
    const int64_t e = static_cast<int64_t>(chunk) * kSampleChunk + i * kSampleThreads + tid;
    key[i] = e < vocab ? sample_key(ld_t<DT>(logits, row * ld + e), static_cast<uint32_t>(e)) : 0;
  }
  block_topk(key, k, L);
  uint64_t* out = cand + (row * n_chunks + chunk) * k;
  for (int i = tid; i < k; i += kSampleThreads) out[i] = L.cand[i];
}

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_scan_f(float v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float u = __shfl_up(v, off, 64);
    if (lane >= off) v += u;
  }
  return v;
}

__global__ __launch_bounds__(kSampleThreads) void k_sample_final(const uint64_t* __restrict__ cand,
                                                                 int n_cand, int k,
                                                                 const float* __restrict__ uniform,
                                                                 float inv_t, float top_p,
                                                                 int64_t* __restrict__ out) {
  __shared__ TopkLds L;
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  const uint64_t* c = cand + static_cast<int64_t>(row) * n_cand;
  uint64_t key[kSampleFinalPer];
#pragma unroll
  for (int i = 0; i < kSampleFinalPer; ++i) {
    const int j = i * kSampleThreads + tid;
    key[i] = j < n_cand ? c[j] : 0;
  }
  block_topk(key, k, L);
  if (tid >= 64) return;
  const uint64_t mine = lane < k ? L.cand[lane] : 0;
  const bool valid = mine != 0;
  const float vmax = key_value(L.cand[0]);
  float p = valid ? __expf((key_value(mine) - vmax) * inv_t) : 0.0f;
  p = p / wave_sum_f(p);
  const float cum = wave_scan_f(p);
  p = (cum - p <= top_p) ? p : 0.0f;
  const float total = wave_sum_f(p);
  const float cum2 = wave_scan_f(p);
  const float u = uniform[row] * total;
  const uint64_t below = __ballot(lane < k && cum2 <= u);
  int pick = __popcll(below);
  pick = pick < k - 1 ? pick : k - 1;
  const uint64_t chosen = __shfl(mine, pick, 64);
  if (lane == 0) out[row] = chosen != 0 ? static_cast<int64_t>(key_index(chosen)) : 0;
}

static int64_t sample_chunks(int64_t vocab) { return (vocab + kSampleChunk - 1) / kSampleChunk; }

}  // namespace ma

using namespace ma;

extern "C" size_t ma_sampler_workspace_bytes(int64_t rows, int64_t vocab, int top_k) {
  if (rows < 0 || vocab < 1 || top_k < 1) return 0;
  return static_cast<size_t>(rows) * sample_chunks(vocab) * top_k * sizeof(uint64_t);
}

extern "C" int ma_fused_sample(const void* logits, int dtype, int64_t rows, int64_t vocab,
                               int64_t ld, const float* uniform, int top_k, float inv_temperature,
                               float top_p, void* workspace, size_t ws_bytes, int64_t* out,
                               void* stream) {
  if (rows < 0 || vocab < 1 || ld < vocab) return fail(MA_EVALUE, "fused_sample: bad sizes");
  if (top_k < 1 || top_k > kSampleMaxK || top_k > vocab)
    return fail(MA_EVALUE, "fused_sample: top_k %d outside [1, min(%d, vocab)]", top_k, kSampleMaxK);
  if (!(inv_temperature > 0.0f && inv_temperature < INFINITY) || !(top_p > 0.0f && top_p <= 1.0f))
    return fail(MA_EVALUE, "fused_sample: needs a finite 1 / temperature > 0 and 0 < top_p <= 1");
  if (dtype != MA_BF16 && dtype != MA_F32 && dtype != MA_F16)
    return fail(MA_ETYPE, "fused_sample: dtype %d unsupported", dtype);
  const int64_t n_chunks = sample_chunks(vocab);
  const int64_t n_cand = n_chunks * top_k;
  if (n_cand > static_cast<int64_t>(kSampleThreads) * kSampleFinalPer)
    return fail(MA_EVALUE, "fused_sample: %lld chunk candidates exceed %d (vocab %lld, top_k %d)",
                static_cast<long long>(n_cand), kSampleThreads * kSampleFinalPer,
                static_cast<long long>(vocab), top_k);
  if (ws_bytes < ma_sampler_workspace_bytes(rows, vocab, top_k))
    return fail(MA_EVALUE, "fused_sample: workspace of %zu bytes, need %zu", ws_bytes,
                ma_sampler_workspace_bytes(rows, vocab, top_k));
  if (rows == 0) return MA_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint64_t* cand = static_cast<uint64_t*>(workspace);
  const dim3 g1(static_cast<unsigned>(n_chunks), static_cast<unsigned>(rows));
  if (dtype == MA_BF16)
    hipLaunchKernelGGL(k_sample_partial<MA_BF16>, g1, dim3(kSampleThreads), 0, s, logits, vocab, ld,
                       top_k, cand);
  else if (dtype == MA_F16)
    hipLaunchKernelGGL(k_sample_partial<MA_F16>, g1, dim3(kSampleThreads), 0, s, logits, vocab, ld,
                       top_k, cand);
  else
    hipLaunchKernelGGL(k_sample_partial<MA_F32>, g1, dim3(kSampleThreads), 0, s, logits, vocab, ld,
                       top_k, cand);
  int rc = check_launch("fused_sample partial");
  if (rc != MA_OK) return rc;
  hipLaunchKernelGGL(k_sample_final, dim3(static_cast<unsigned>(rows)), dim3(kSampleThreads), 0, s,
                     cand, static_cast<int>(n_cand), top_k, uniform, inv_temperature, top_p, out);
  return check_launch("fused_sample final");
}
