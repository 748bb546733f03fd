// Greedy token choice: argmax over each row of the logits (gfx950).
//
// Semantics of the reference's greedy step (src/maple_run/generate.py:146-148,
// torch.argmax over the vocabulary): the index of the largest value, the
// lowest such index on ties.  One 1024-thread workgroup per row; every thread
// scans 16-byte vectors (bf16 or float32), then (value, index) pairs meet
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
  constexpr int U = 20;  // 1024 x 20 x 16 B = 320 KB in flight: one round for a 151936-token bf16 row
  for (int64_t v0 = tid; v0 < nvec; v0 += static_cast<int64_t>(kArgmaxThreads) * U) {
    uint4 q[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t vi = v0 + static_cast<int64_t>(kArgmaxThreads) * u;
      q[u] = vi < nvec ? p[vi] : make_uint4(0xff80ff80u, 0xff80ff80u, 0xff800000u, 0xff800000u);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t vi = v0 + static_cast<int64_t>(kArgmaxThreads) * u;
      if (vi >= nvec) continue;
      const uint32_t w[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
#pragma unroll
      for (int e = 0; e < PER; ++e) {
        float f;
        if constexpr (DT == MA_BF16)
          f = __uint_as_float((e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16));
        else
          f = __uint_as_float(w[e]);
        if (f > best) {  // strict: within a thread indices only grow
          best = f;
          bi = vi * PER + e;
        }
      }
    }
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
