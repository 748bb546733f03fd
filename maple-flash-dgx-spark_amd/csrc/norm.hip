// RMSNorm, residual-add + RMSNorm and the MoE top-k combine (gfx950).
//
// Semantics: reference src/maple_run/kernels/fused_norm.py
//   rms_norm        :10-28   y = x * rsqrt(mean(x^2) + eps) * w, float32 math
//   add_rms_norm    :31-56   s = x + y; residual = s, normed = rms_norm(s)
//   moe_reduce_add  :59-96   y = sum_j w_j * expert_out_j (+ residual)
#include "common.h"

namespace ma {

__global__ __launch_bounds__(256) void k_rms_norm(const void* __restrict__ x, int x_dt,
                                                  int64_t n, const void* __restrict__ w,
                                                  int w_dt, float eps, void* __restrict__ y) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += 256) {
    const float v = ld_f(x, x_dt, row * n + i);
    ss += v * v;
  }
  const float rstd = rsqrtf(block_sum256(ss, red) / static_cast<float>(n) + eps);
  for (int64_t i = threadIdx.x; i < n; i += 256)
    st_f(y, x_dt, row * n + i, ld_f(x, x_dt, row * n + i) * rstd * ld_f(w, w_dt, i));
}

__global__ __launch_bounds__(256) void k_add_rms_norm(const void* __restrict__ x,
                                                      const void* __restrict__ y, int dt,
                                                      int64_t n, const void* __restrict__ w,
                                                      int w_dt, float eps,
                                                      void* __restrict__ res,
                                                      void* __restrict__ normed) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += 256) {
    const float s = ld_f(x, dt, row * n + i) + ld_f(y, dt, row * n + i);
    ss += s * s;
    st_f(res, dt, row * n + i, s);
  }
  const float rstd = rsqrtf(block_sum256(ss, red) / static_cast<float>(n) + eps);
  for (int64_t i = threadIdx.x; i < n; i += 256) {
    const float s = ld_f(x, dt, row * n + i) + ld_f(y, dt, row * n + i);
    st_f(normed, dt, row * n + i, s * rstd * ld_f(w, w_dt, i));
  }
}

// bf16 rows, n % 8 == 0 and n <= 2048 * CH: thread t owns 16-byte chunks
// t, t + 256, ...; every load is issued before the reduction.  ADD: x + y
// first, written to ``res`` (rounded); the norm uses the float32 sum.
template <int CH, bool ADD, int WDT>
__global__ __launch_bounds__(256) void k_norm_fast(const uint16_t* __restrict__ x,
                                                   const uint16_t* __restrict__ y, int64_t n,
                                                   const void* __restrict__ w, float eps,
                                                   uint16_t* __restrict__ res,
                                                   uint16_t* __restrict__ out) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int nch = static_cast<int>(n >> 3);
  uint4 xv[CH], yv[CH];
  float wv[CH][8];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = threadIdx.x + 256 * c;
    const int cc = ch < nch ? ch : nch - 1;
    xv[c] = reinterpret_cast<const uint4*>(x + row * n)[cc];
    if constexpr (ADD) yv[c] = reinterpret_cast<const uint4*>(y + row * n)[cc];
#pragma unroll
    for (int e = 0; e < 8; ++e) wv[c][e] = ld_t<WDT>(w, cc * 8 + e);
  }
  MA_ISSUE_FENCE();
  float v[CH][8], ss = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const bool live = threadIdx.x + 256 * c < nch;
    const uint32_t* xw = reinterpret_cast<const uint32_t*>(&xv[c]);
    const uint32_t* yw = reinterpret_cast<const uint32_t*>(&yv[c]);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float lo = __uint_as_float(xw[e] << 16), hi = __uint_as_float(xw[e] & 0xffff0000u);
      if constexpr (ADD) {
        lo += __uint_as_float(yw[e] << 16);
        hi += __uint_as_float(yw[e] & 0xffff0000u);
      }
      v[c][2 * e] = lo;
      v[c][2 * e + 1] = hi;
      if (live) ss += lo * lo + hi * hi;
    }
  }
  const float rstd = rsqrtf(block_sum256(ss, red) / static_cast<float>(n) + eps);
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = threadIdx.x + 256 * c;
    if (ch >= nch) continue;
    uint4 o, r;
    uint32_t* ow = reinterpret_cast<uint32_t*>(&o);
    uint32_t* rw = reinterpret_cast<uint32_t*>(&r);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      ow[e] = pack_bf16x2_rn(v[c][2 * e] * rstd * wv[c][2 * e], v[c][2 * e + 1] * rstd * wv[c][2 * e + 1]);
      if constexpr (ADD) rw[e] = pack_bf16x2_rn(v[c][2 * e], v[c][2 * e + 1]);
    }
    reinterpret_cast<uint4*>(out + row * n)[ch] = o;
    if constexpr (ADD) reinterpret_cast<uint4*>(res + row * n)[ch] = r;
  }
}

__global__ __launch_bounds__(256) void k_moe_reduce(const void* __restrict__ eo, int dt,
                                                    int64_t topk, int64_t n,
                                                    const float* __restrict__ wts,
                                                    const void* __restrict__ res, int res_dt,
                                                    void* __restrict__ y) {
  const int64_t t = blockIdx.y;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  float acc = 0.f;
  for (int64_t j = 0; j < topk; ++j) acc += wts[t * topk + j] * ld_f(eo, dt, (t * topk + j) * n + i);
  if (res) acc += ld_f(res, res_dt, t * n + i);
  st_f(y, dt, t * n + i, acc);
}

}  // namespace ma

using namespace ma;

// Fast-path launch for bf16 rows; returns false if the shape does not fit.
static bool launch_norm_fast(const void* x, const void* y, int64_t rows, int64_t n,
                             const void* w, int w_dtype, float eps, void* res, void* out,
                             hipStream_t s) {
  if (n % 8 || n > 8192 || (w_dtype != MA_F32 && w_dtype != MA_BF16)) return false;
  auto aligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (!aligned(x) || !aligned(out) || (y && (!aligned(y) || !aligned(res)))) return false;
  const int ch = n <= 2048 ? 1 : (n <= 4096 ? 2 : 4);
  const dim3 grid(static_cast<unsigned>(rows));
  const auto* xs = static_cast<const uint16_t*>(x);
  const auto* ys = static_cast<const uint16_t*>(y);
  auto* rs = static_cast<uint16_t*>(res);
  auto* os = static_cast<uint16_t*>(out);
#define MA_NORM_LAUNCH(CH, ADD, WDT) \
  hipLaunchKernelGGL((k_norm_fast<CH, ADD, WDT>), grid, dim3(256), 0, s, xs, ys, n, w, eps, rs, os)
#define MA_NORM_W(CH, ADD)                                     \
  if (w_dtype == MA_F32) MA_NORM_LAUNCH(CH, ADD, MA_F32); \
  else MA_NORM_LAUNCH(CH, ADD, MA_BF16)
#define MA_NORM_ADD(CH)      \
  if (y) { MA_NORM_W(CH, true); } \
  else { MA_NORM_W(CH, false); }
  if (ch == 1) { MA_NORM_ADD(1) }
  else if (ch == 2) { MA_NORM_ADD(2) }
  else { MA_NORM_ADD(4) }
#undef MA_NORM_ADD
#undef MA_NORM_W
#undef MA_NORM_LAUNCH
  return true;
}

extern "C" int ma_rms_norm(const void* x, int x_dtype, int64_t rows, int64_t n,
                           const void* weight, int w_dtype, float eps, void* y, void* stream) {
  if (rows < 0 || n < 1) return fail(MA_EVALUE, "rms_norm: bad sizes");
  if (rows == 0) return MA_OK;
  if (x_dtype == MA_BF16 &&
      launch_norm_fast(x, nullptr, rows, n, weight, w_dtype, eps, nullptr, y,
                       static_cast<hipStream_t>(stream)))
    return check_launch("rms_norm");
  hipLaunchKernelGGL(k_rms_norm, dim3(static_cast<unsigned>(rows)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, x_dtype, n, weight, w_dtype, eps, y);
  return check_launch("rms_norm");
}

extern "C" int ma_add_rms_norm(const void* x, const void* y, int dtype, int64_t rows, int64_t n,
                               const void* weight, int w_dtype, float eps, void* residual,
                               void* normed, void* stream) {
  if (rows < 0 || n < 1) return fail(MA_EVALUE, "add_rms_norm: bad sizes");
  if (rows == 0) return MA_OK;
  if (dtype == MA_BF16 &&
      launch_norm_fast(x, y, rows, n, weight, w_dtype, eps, residual, normed,
                       static_cast<hipStream_t>(stream)))
    return check_launch("add_rms_norm");
  hipLaunchKernelGGL(k_add_rms_norm, dim3(static_cast<unsigned>(rows)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, y, dtype, n, weight, w_dtype, eps,
                     residual, normed);
  return check_launch("add_rms_norm");
}

extern "C" int ma_moe_reduce_add(const void* expert_out, int eo_dtype, int64_t tokens,
                                 int64_t top_k, int64_t n, const float* topk_weight,
                                 const void* residual, int residual_dtype, void* y,
                                 void* stream) {
  if (tokens < 0 || top_k < 1 || n < 0) return fail(MA_EVALUE, "moe_reduce_add: bad sizes");
  if (tokens == 0 || n == 0) return MA_OK;
  dim3 grid(static_cast<unsigned>(cdiv(n, 256)), static_cast<unsigned>(tokens));
  hipLaunchKernelGGL(k_moe_reduce, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     expert_out, eo_dtype, top_k, n, topk_weight, residual, residual_dtype, y);
  return check_launch("moe_reduce_add");
}
