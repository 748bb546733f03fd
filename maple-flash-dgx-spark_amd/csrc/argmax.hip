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
#include "grid_sync.h"

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
    if (lane == 0) out[row] = i < n && v != -INFINITY ? i : 0;  // every value -inf: index 0, as torch
  }
}

// Split form (ma_argmax_rows_ws): kSplitChunk-vector chunks of a row, one
// 256-thread workgroup each (every load of a chunk in flight at once), so a
// row is read by many CUs instead of one.  Each workgroup stores its chunk's
// (value, index) -- the larger value, the lower index on ties, as above --
// with the device-coherent policy, then takes a ticket on the row's counter;
// the workgroup that takes the last one reduces the row's partials in chunk
// order, writes out[row] and clears the counter (the workspace starts and
// ends every call zero; calls on one workspace must not overlap).  The last
// chunk also takes the elements past the last whole vector.
constexpr int kSplitThreads = 256, kSplitU = 5, kSplitChunk = kSplitThreads * kSplitU;
constexpr int kSplitMaxChunks = 64;  // per row (rows of up to 64 x 1280 vectors)
constexpr size_t kSplitRowBytes = 256 + kSplitMaxChunks * 16;  // counter line + partials

template <int DT>
__global__ __launch_bounds__(kSplitThreads) void k_argmax_split(const void* __restrict__ x, int64_t n,
                                                                int64_t ldx, int64_t* __restrict__ out,
                                                                uint8_t* __restrict__ ws) {
  __shared__ float sv[kSplitThreads / 64];
  __shared__ int64_t si[kSplitThreads / 64];
  __shared__ int last;
  constexpr int PER = DT == MA_BF16 ? 8 : 4;
  const int64_t row = blockIdx.y;
  const int g = blockIdx.x, G = gridDim.x;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t nvec = n / PER;
  const uint4* p = reinterpret_cast<const uint4*>(static_cast<const char*>(x) +
                                                  row * ldx * (DT == MA_BF16 ? 2 : 4));
  constexpr uint32_t kNegInf4 = DT == MA_BF16 ? 0xff80ff80u : 0xff800000u;
  const int64_t c0 = static_cast<int64_t>(g) * kSplitChunk;
  uint4 q[kSplitU];
#pragma unroll
  for (int u = 0; u < kSplitU; ++u) {
    const int64_t vi = c0 + tid + kSplitThreads * u;
    q[u] = vi < nvec ? p[vi] : make_uint4(kNegInf4, kNegInf4, kNegInf4, kNegInf4);
  }
  float best = -INFINITY;
  int64_t bv = -1;
#pragma unroll
  for (int u = 0; u < kSplitU; ++u) {
    const int64_t vi = c0 + tid + kSplitThreads * u;
    const float m = vec_max<DT>(q[u]);
    if (m > best && vi < nvec) {
      best = m;
      bv = vi;
    }
  }
  int64_t bi = n;
  if (bv >= 0) {  // the lowest index of the winning vector holding the maximum
    float f[PER];
    vec_unpack<DT>(p[bv], f);
    int e = PER - 1;
#pragma unroll
    for (int k = PER - 1; k >= 0; --k)
      if (f[k] == best) e = k;
    bi = bv * PER + e;
  }
  if (g == G - 1) {
    for (int64_t k = nvec * PER + tid; k < n; k += kSplitThreads) {
      const float f = DT == MA_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(x)[row * ldx + k])
                                    : static_cast<const float*>(x)[row * ldx + k];
      take_better(best, bi, f, k);
    }
  }
  wave_argmax(best, bi);
  if (lane == 0) {
    sv[wv] = best;
    si[wv] = bi;
  }
  __syncthreads();
  uint8_t* const rw = ws + row * kSplitRowBytes;
  uint32_t* const counter = reinterpret_cast<uint32_t*>(rw);
  uint64_t* const part = reinterpret_cast<uint64_t*>(rw + 256);  // [chunk] (index, value bits)
  if (tid == 0) {
    float v = sv[0];
    int64_t i = si[0];
    for (int w = 1; w < kSplitThreads / 64; ++w) take_better(v, i, sv[w], si[w]);
    st_coh64(&part[2 * g], static_cast<uint64_t>(i));
    st_coh64(&part[2 * g + 1], __float_as_uint(v));
    __builtin_amdgcn_s_waitcnt(0);  // the partial has completed before the ticket
    last = atomicAdd(counter, 1u) == static_cast<uint32_t>(G - 1);
  }
  __syncthreads();
  if (!last || wv != 0) return;
  float v = -INFINITY;
  int64_t i = n;
  for (int c = lane; c < G; c += 64) {  // lane order within a chunk round, then the exchanges
    const float vc = __uint_as_float(static_cast<uint32_t>(ld_coh64(&part[2 * c + 1])));
    const int64_t ic = static_cast<int64_t>(ld_coh64(&part[2 * c]));
    take_better(v, i, vc, ic);
  }
  wave_argmax(v, i);
  if (lane == 0) {
    out[row] = i < n && v != -INFINITY ? i : 0;  // every value -inf: index 0, as torch
    st_coh32(counter, 0u);
  }
}

}  // namespace ma

using namespace ma;

extern "C" size_t ma_argmax_workspace_bytes(int64_t rows) {
  return rows > 0 ? static_cast<size_t>(rows) * kSplitRowBytes : 0;
}

extern "C" int ma_argmax_rows_ws(const void* x, int x_dtype, int64_t rows, int64_t n, int64_t ldx,
                                 int64_t* out, void* workspace, size_t workspace_bytes, void* stream) {
  if (rows < 0 || n < 1 || ldx < n) return fail(MA_EVALUE, "argmax_rows_ws: bad sizes");
  if (x_dtype != MA_BF16 && x_dtype != MA_F32)
    return fail(MA_ETYPE, "argmax_rows_ws: dtype %d unsupported", x_dtype);
  if (rows == 0) return MA_OK;
  const int per = x_dtype == MA_BF16 ? 8 : 4;
  const int vec = (reinterpret_cast<uintptr_t>(x) & 15) == 0 && ldx % per == 0;
  const int64_t chunks = cdiv(n / per, kSplitChunk);
  // rows the split form does not take (not 16-byte aligned, or too long):
  // the one-workgroup form
  if (!vec || chunks < 1 || chunks > kSplitMaxChunks) return ma_argmax_rows(x, x_dtype, rows, n, ldx, out, stream);
  if (!workspace || workspace_bytes < ma_argmax_workspace_bytes(rows) ||
      (reinterpret_cast<uintptr_t>(workspace) & 255))
    return fail(MA_EVALUE, "argmax_rows_ws: workspace must be %zu bytes, 256-byte aligned",
                ma_argmax_workspace_bytes(rows));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(rows));
  if (x_dtype == MA_BF16)
    hipLaunchKernelGGL(k_argmax_split<MA_BF16>, grid, dim3(kSplitThreads), 0, s, x, n, ldx, out,
                       static_cast<uint8_t*>(workspace));
  else
    hipLaunchKernelGGL(k_argmax_split<MA_F32>, grid, dim3(kSplitThreads), 0, s, x, n, ldx, out,
                       static_cast<uint8_t*>(workspace));
  return check_launch("argmax_rows_ws");
}

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
