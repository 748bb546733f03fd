// Greedy token choice: argmax over each row of the logits (gfx950).
//
// Semantics of the reference's greedy step (src/maple_run/generate.py:146-148,
// torch.argmax over the vocabulary): the index of the largest value, the
// lowest such index on ties.  One 1024-thread workgroup per row; every thread
// scans 16-byte vectors (bf16 or float32) by their maxima, then (value, index) pairs meet
// through shuffles within waves and LDS across waves (rows that are not
// 16-byte aligned take a scalar loop).  NaN logits are
// not expected (the reference's output would be its own NaN handling).
#include "common.h"

namespace ma {

constexpr int kArgmaxThreads = 1024;

// Better = larger value, or equal value at a lower index.
__device__ __forceinline__ void take_better(float& v, int64_t& i, float v2, int64_t i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

// The PER values of a 16-byte vector (bf16: 8, float32: 4) as floats.
template <int DT>
__device__ __forceinline__ void vec_unpack(const uint4& q, float (&f)[DT == MA_BF16 ? 8 : 4]) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  if constexpr (DT == MA_BF16) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      f[2 * k] = __uint_as_float(w[k] << 16);
      f[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) f[k] = __uint_as_float(w[k]);
  }
}
template <int DT>
__device__ __forceinline__ float vec_max(const uint4& q) {
  float f[DT == MA_BF16 ? 8 : 4];
  vec_unpack<DT>(q, f);
  if constexpr (DT == MA_BF16)
    return fmaxf(fmaxf(fmaxf(f[0], f[1]), fmaxf(f[2], f[3])), fmaxf(fmaxf(f[4], f[5]), fmaxf(f[6], f[7])));
  else
    return fmaxf(fmaxf(f[0], f[1]), fmaxf(f[2], f[3]));
}

__device__ __forceinline__ void wave_argmax(float& v, int64_t& i) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float v2 = __shfl_xor(v, off, 64);
    const int64_t i2 = __shfl_xor(i, off, 64);
    take_better(v, i, v2, i2);
  }
}

template <int DT>
__global__ __launch_bounds__(kArgmaxThreads) void k_argmax_rows(const void* __restrict__ x,
                                                                int64_t n, int64_t ldx, int vec,
                                                                int64_t* __restrict__ out) {
  __shared__ float sv[kArgmaxThreads / 64];
  __shared__ int64_t si[kArgmaxThreads / 64];
  constexpr int PER = DT == MA_BF16 ? 8 : 4;  // elements per 16-byte vector
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  float best = -INFINITY;
  int64_t bi = n;  // past the end: loses every tie
  const int64_t nvec = vec ? n / PER : 0;  // rows not 16-byte aligned: scalar loop only
  const uint4* p = reinterpret_cast<const uint4*>(static_cast<const char*>(x) +
                                                  row * ldx * (DT == MA_BF16 ? 2 : 4));
  // Per 16-byte vector: its maximum (v_max3), one compare against the
  // thread's best; strict, so the thread keeps its first vector holding its
  // maximum, and the lowest index in that vector is found once at the end.
  int64_t bv = -1;
  constexpr uint32_t kNegInf4 = DT == MA_BF16 ? 0xff80ff80u : 0xff800000u;  // -inf in every element
  constexpr int U = 19;  // 1024 x 19 x 16 B = 304 KB in flight: one round for a 151936-token bf16 row
  for (int64_t v0 = tid; v0 < nvec; v0 += static_cast<int64_t>(kArgmaxThreads) * U) {
    uint4 q[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t vi = v0 + static_cast<int64_t>(kArgmaxThreads) * u;
      q[u] = vi < nvec ? p[vi] : make_uint4(kNegInf4, kNegInf4, kNegInf4, kNegInf4);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t vi = v0 + static_cast<int64_t>(kArgmaxThreads) * u;
      const float m = vec_max<DT>(q[u]);
      if (m > best && vi < nvec) {  // vectors past the row never win (and are never re-read)
        best = m;
        bv = vi;
      }
    }
  }
  if (bv >= 0 && bv < nvec) {  // the lowest index of the winning vector holding the maximum
    float f[PER];
    vec_unpack<DT>(p[bv], f);
    int e = PER - 1;
#pragma unroll
    for (int k = PER - 1; k >= 0; --k)
      if (f[k] == best) e = k;
    bi = bv * PER + e;
  }
  // Tail elements that do not fill a vector.
  for (int64_t k = nvec * PER + tid; k < n; k += kArgmaxThreads) {
    const float f = DT == MA_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(x)[row * ldx + k])
                                  : static_cast<const float*>(x)[row * ldx + k];
    take_better(best, bi, f, k);
  }
  wave_argmax(best, bi);
  if (lane == 0) {
    sv[wv] = best;
    si[wv] = bi;
  }
  __syncthreads();
  if (wv == 0) {
    float v = lane < kArgmaxThreads / 64 ? sv[lane] : -INFINITY;
    int64_t i = lane < kArgmaxThreads / 64 ? si[lane] : n;
    wave_argmax(v, i);
    if (lane == 0) out[row] = i < n ? i : 0;
  }
}

}  // namespace ma

using namespace ma;

extern "C" int ma_argmax_rows(const void* x, int x_dtype, int64_t rows, int64_t n, int64_t ldx,
                              int64_t* out, void* stream) {
  if (rows < 0 || n < 1 || ldx < n) return fail(MA_EVALUE, "argmax_rows: bad sizes");
  if (x_dtype != MA_BF16 && x_dtype != MA_F32)
    return fail(MA_ETYPE, "argmax_rows: dtype %d unsupported", x_dtype);
  const int per = x_dtype == MA_BF16 ? 8 : 4;
  const int vec = (reinterpret_cast<uintptr_t>(x) & 15) == 0 && ldx % per == 0;
  if (rows == 0) return MA_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (x_dtype == MA_BF16)
    hipLaunchKernelGGL(k_argmax_rows<MA_BF16>, dim3(static_cast<unsigned>(rows)),
                       dim3(kArgmaxThreads), 0, s, x, n, ldx, vec, out);
  else
    hipLaunchKernelGGL(k_argmax_rows<MA_F32>, dim3(static_cast<unsigned>(rows)),
                       dim3(kArgmaxThreads), 0, s, x, n, ldx, vec, out);
  return check_launch("argmax_rows");
}
