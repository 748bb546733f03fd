// RMSNorm, residual-add + RMSNorm and the MoE top-k combine (gfx950).
//
// Semantics: reference src/maple_run/kernels/fused_norm.py
//   rms_norm        :10-28   y = x * rsqrt(mean(x^2) + eps) * w, float32 math
//   add_rms_norm    :31-56   s = x + y; residual = s, normed = rms_norm(s)
//   moe_reduce_add  :59-96   y = sum_j w_j * expert_out_j (+ residual)
#include "common.h"

namespace ma {

// Block-wide sum over 256 threads; every thread gets the total.
__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = group_sum<64>(v);
  const int wv = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wv] = v;
  __syncthreads();
  const float t = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  return t;
}

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

extern "C" int ma_rms_norm(const void* x, int x_dtype, int64_t rows, int64_t n,
                           const void* weight, int w_dtype, float eps, void* y, void* stream) {
  if (rows < 0 || n < 1) return fail(MA_EVALUE, "rms_norm: bad sizes");
  if (rows == 0) return MA_OK;
  hipLaunchKernelGGL(k_rms_norm, dim3(static_cast<unsigned>(rows)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, x_dtype, n, weight, w_dtype, eps, y);
  return check_launch("rms_norm");
}

extern "C" int ma_add_rms_norm(const void* x, const void* y, int dtype, int64_t rows, int64_t n,
                               const void* weight, int w_dtype, float eps, void* residual,
                               void* normed, void* stream) {
  if (rows < 0 || n < 1) return fail(MA_EVALUE, "add_rms_norm: bad sizes");
  if (rows == 0) return MA_OK;
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
