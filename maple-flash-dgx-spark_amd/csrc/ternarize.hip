// Row-wise ternarisation on the GPU (the converter's step), gfx950.
//
// Semantics of reference src/maple_run/pack.py:120-149 (ternarize): per row
// of K float32 values (K a multiple of 128), thr = threshold_scale *
// mean(|w|); mask = |w| > thr; alpha = sum(|w| * mask) / max(sum(mask), 1),
// cast to the weight dtype; codes sign(w) * mask + 1 packed 16 per uint32,
// least significant first (pack.py:17-45).
//
// The reference computes the mean and the sums with NumPy in float32, and the
// mask depends on thr to the last bit, so the sums here follow NumPy's
// float32 pairwise summation (the order np.sum / np.mean take over a
// contiguous last axis): a range of n > 128 values splits at n2 = n/2 -
// (n/2 mod 8) into two halves summed separately and then added; a range of 8
// <= n <= 128 values sums into eight accumulators r_j = a_j + a_{8+j} + ...
// (in order), combined as ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7)),
// then adds the n mod 8 rest in order; the result is added to 0.  With K a
// multiple of 128 every leaf range is a multiple of 8 long.  mean = sum /
// float32(K) and thr = float32(threshold_scale) * mean, both in float32.
//
// One workgroup per row: the row's |w| staged in LDS, the leaf accumulators
// computed in parallel (one lane per accumulator), then one lane walks the
// split tree in post order.
#include "common.h"

namespace ma {

constexpr int kTernThreads = 256;
constexpr int kTernMaxK = 8192;
constexpr int kTernMaxLeaves = 128;  // leaf ranges are >= 64 values long, so <= K / 64

struct PwRange {
  int off, n;
};

// The leaf ranges of the split tree of [0, K), left to right.
__device__ inline int pw_leaves(int K, PwRange* out) {
  PwRange st[32];
  int sp = 0, nl = 0;
  st[sp++] = PwRange{0, K};
  while (sp > 0) {
    const PwRange f = st[--sp];
    if (f.n <= 128) {
      out[nl++] = f;
      continue;
    }
    int n2 = f.n / 2;
    n2 -= n2 % 8;
    st[sp++] = PwRange{f.off + n2, f.n - n2};
    st[sp++] = PwRange{f.off, n2};
  }
  return nl;
}

// Sum of v(a[i]) over [0, K) in NumPy's pairwise order.  Called by every
// thread of the workgroup (it synchronises); every thread gets the sum.
// ``acc`` holds 8 floats per leaf; ``leaves``/``nl`` from pw_leaves.
template <typename F>
__device__ inline float pw_sum(const float* a, int K, const PwRange* leaves, int nl, float* acc, float* res,
                               F v) {
  for (int c = threadIdx.x; c < 8 * nl; c += blockDim.x) {
    const PwRange lf = leaves[c >> 3];
    const int j = c & 7;
    float r = v(a[lf.off + j]);
    for (int t = 8; t < lf.n; t += 8) r += v(a[lf.off + t + j]);
    acc[c] = r;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    struct Fr {
      int off, n;
      bool expanded;
    };
    Fr st[48];
    float vs[32];
    int sp = 0, vp = 0, li = 0;
    st[sp++] = Fr{0, K, false};
    while (sp > 0) {
      const Fr f = st[--sp];
      if (f.n <= 128) {
        const float* r = acc + 8 * li++;
        vs[vp++] = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
        continue;
      }
      if (f.expanded) {
        const float rt = vs[--vp];
        const float lt = vs[--vp];
        vs[vp++] = lt + rt;
        continue;
      }
      int n2 = f.n / 2;
      n2 -= n2 % 8;
      st[sp++] = Fr{f.off, f.n, true};
      st[sp++] = Fr{f.off + n2, f.n - n2, false};
      st[sp++] = Fr{f.off, n2, false};
    }
    *res = 0.f + vs[0];
  }
  __syncthreads();
  const float s = *res;
  __syncthreads();  // res and acc are reused by the next sum
  return s;
}

template <int DT>
__global__ __launch_bounds__(kTernThreads) void k_ternarize(const void* __restrict__ w, int64_t K, float tscale,
                                                            uint32_t* __restrict__ packed, void* __restrict__ alpha) {
  __shared__ float aw[kTernMaxK];
  __shared__ PwRange leaves[kTernMaxLeaves];
  __shared__ float acc[8 * kTernMaxLeaves];
  __shared__ float res;
  __shared__ int s_nl;
  const int64_t row = blockIdx.x;
  const int k = static_cast<int>(K);
  for (int i = threadIdx.x; i < k; i += blockDim.x) aw[i] = fabsf(ld_t<DT>(w, row * K + i));
  if (threadIdx.x == 0) s_nl = pw_leaves(k, leaves);
  __syncthreads();
  const int nl = s_nl;
  const float mean = pw_sum(aw, k, leaves, nl, acc, &res, [](float x) { return x; }) / static_cast<float>(k);
  const float thr = tscale * mean;
  const float num = pw_sum(aw, k, leaves, nl, acc, &res, [thr](float x) { return x > thr ? x : 0.f; });
  const float cnt = pw_sum(aw, k, leaves, nl, acc, &res, [thr](float x) { return x > thr ? 1.f : 0.f; });
  // codes: thread t packs word t (16 values), re-reading the signs from w
  for (int wd = threadIdx.x; wd < k / 16; wd += blockDim.x) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float x = ld_t<DT>(w, row * K + wd * 16 + j);
      const uint32_t code = fabsf(x) > thr ? (x > 0.f ? 2u : (x < 0.f ? 0u : 1u)) : 1u;
      word |= code << (2 * j);
    }
    packed[row * (K / 16) + wd] = word;
  }
  if (threadIdx.x == 0) st_f(alpha, DT, row, num / fmaxf(cnt, 1.f));
}

}  // namespace ma

using namespace ma;

// Reference: src/maple_run/pack.py:120-149 (ternarize), as the converter
// calls it on [..., N, K] weights flattened to rows.
extern "C" int ma_ternarize(const void* weight, int dtype, int64_t rows, int64_t k_in, float threshold_scale,
                            uint32_t* packed, void* row_alpha, void* stream) {
  if (!weight || !packed || !row_alpha) return fail(MA_EVALUE, "ternarize: null pointer");
  if (rows < 0 || k_in < 128 || k_in % 128 != 0 || k_in > kTernMaxK)
    return fail(MA_EVALUE, "ternarize: K must be a multiple of 128 in [128, %d]; got %lld", kTernMaxK,
                static_cast<long long>(k_in));
  if (dtype != MA_F32 && dtype != MA_BF16 && dtype != MA_F16)
    return fail(MA_ETYPE, "ternarize: weight dtype %d (float32, bfloat16 or float16)", dtype);
  if (rows == 0) return MA_OK;
  if (rows > 0x7fffffff) return fail(MA_EVALUE, "ternarize: too many rows");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(rows)), block(kTernThreads);
  if (dtype == MA_F32)
    hipLaunchKernelGGL(k_ternarize<MA_F32>, grid, block, 0, st, weight, k_in, threshold_scale, packed, row_alpha);
  else if (dtype == MA_BF16)
    hipLaunchKernelGGL(k_ternarize<MA_BF16>, grid, block, 0, st, weight, k_in, threshold_scale, packed, row_alpha);
  else
    hipLaunchKernelGGL(k_ternarize<MA_F16>, grid, block, 0, st, weight, k_in, threshold_scale, packed, row_alpha);
  return check_launch("ternarize");
}
