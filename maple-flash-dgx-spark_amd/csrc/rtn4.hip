// 4-bit affine RTN lm_head GEMV and embedding gather (gfx950).
//
// Semantics of reference src/maple_run/kernels/rtn4.py: y[b, n] =
// sum_g sum_{k in g} (q[n,k] * s[n,g] + b[n,g]) * x[b,k] with float32
// accumulation (:84-167, :170-282); rtn4_embedding returns the dequantised
// float32 rows (:27-47).
//
// Fast GEMV (bf16 x, [N, K/8] codes, a lane's KW words inside one group):
// code j (low half) and j + 4 (high half) of a word are lined up by one shift
// in mantissa bits 3..6 of bf16 1.0, giving 1 + q/16; against x' = 16 x the
// dot is sum (16 + q) x, so per lane
//   contribution = s_g * (acc - 16 X) + b_g * X,   X = sum of the lane's x,
// which is the factored per-group form of the reference's batched kernel
// (rtn4.py:197-208) evaluated in float32.  A word costs 4 shifts, 4 and/or
// and 4 v_dot2_f32_bf16.
#include "common.h"

namespace ma {

constexpr uint32_t kMaskQ4 = 0x00780078u;

template <int KW>
__device__ __forceinline__ void load_words_r(const uint32_t* __restrict__ p, uint32_t out[KW]) {
  if constexpr (KW % 4 == 0) {
#pragma unroll
    for (int i = 0; i < KW / 4; ++i) {
      const uint4 v = reinterpret_cast<const uint4*>(p)[i];
      out[4 * i + 0] = v.x;
      out[4 * i + 1] = v.y;
      out[4 * i + 2] = v.z;
      out[4 * i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < KW; ++i) out[i] = p[i];
  }
}

template <int KW, int LPR, int BT, int U, int SDT>
__global__ __launch_bounds__(64) void k_rtn4_fast(
    const uint16_t* __restrict__ x, int64_t batch, int64_t ldx,
    const uint32_t* __restrict__ w, int64_t n_out, int64_t n_groups, int64_t gw,
    const void* __restrict__ scales, const void* __restrict__ biases,
    uint16_t* __restrict__ y, int64_t ldy) {
  constexpr int NW = KW * LPR;
  constexpr int RPI = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int kl = lane % LPR, sub = lane / LPR;
  const int64_t g = (static_cast<int64_t>(kl) * KW) / gw;  // the lane's RTN group
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * (RPI * U);
  const int64_t b0 = static_cast<int64_t>(blockIdx.y) * BT;

  uint32_t wv[U][KW];
  float sc[U], bi[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    int64_t r = r0 + u * RPI + sub;
    r = r < n_out ? r : n_out - 1;
    load_words_r<KW>(w + r * NW + kl * KW, wv[u]);
    sc[u] = ld_t<SDT>(scales, r * n_groups + g);
    bi[u] = ld_t<SDT>(biases, r * n_groups + g);
  }
  uint4 xr[BT][KW];
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) {
    const int64_t b = b0 + bt < batch ? b0 + bt : batch - 1;
#pragma unroll
    for (int i = 0; i < KW; ++i)
      xr[bt][i] = reinterpret_cast<const uint4*>(x + b * ldx + static_cast<int64_t>(kl * KW + i) * 8)[0];
  }
  MA_ISSUE_FENCE();
  uint32_t xp[BT][KW][4];
  float xsum[BT];
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) {
    const bool valid = b0 + bt < batch;
    float sx = 0.f;
#pragma unroll
    for (int i = 0; i < KW; ++i) {
      const uint32_t u4[4] = {xr[bt][i].x, xr[bt][i].y, xr[bt][i].z, xr[bt][i].w};
      float xs[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        xs[2 * q] = valid ? __uint_as_float(u4[q] << 16) : 0.f;
        xs[2 * q + 1] = valid ? __uint_as_float(u4[q] & 0xffff0000u) : 0.f;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xp[bt][i][j] = pack_bf16x2(16.f * xs[j], 16.f * xs[j + 4]);
        sx += xs[j] + xs[j + 4];
      }
    }
    xsum[bt] = sx;
  }
  const uint32_t mq = kMaskQ4, one = kOneBf16x2;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float acc[BT][2];
#pragma unroll
    for (int bt = 0; bt < BT; ++bt) acc[bt][0] = acc[bt][1] = 0.f;
#pragma unroll
    for (int i = 0; i < KW; ++i) {
      const uint32_t wd = wv[u][i];
      const uint32_t e[4] = {and_or(wd << 3, mq, one), and_or(wd >> 1, mq, one),
                             and_or(wd >> 5, mq, one), and_or(wd >> 9, mq, one)};
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int bt = 0; bt < BT; ++bt) acc[bt][j & 1] = dot2(e[j], xp[bt][i][j], acc[bt][j & 1]);
    }
    const int64_t r = r0 + u * RPI + sub;
#pragma unroll
    for (int bt = 0; bt < BT; ++bt) {
      const float part = sc[u] * ((acc[bt][0] + acc[bt][1]) - 16.f * xsum[bt]) + bi[u] * xsum[bt];
      const float v = group_sum<LPR>(part);
      const int64_t b = b0 + bt;
      if (kl == 0 && r < n_out && b < batch) y[b * ldy + r] = f32_to_bf16(v);
    }
  }
}

// Generic: one wave per row; any dtype / layout / group size.
__global__ __launch_bounds__(256) void k_rtn4_generic(
    const void* __restrict__ x, int x_dt, int64_t batch, int64_t ldx,
    const uint32_t* __restrict__ w, int64_t n_out, int64_t nwords, int kn,
    const void* __restrict__ scales, int s_dt, const void* __restrict__ biases, int b_dt,
    int64_t group, void* __restrict__ y, int64_t ldy) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= n_out) return;
  const int64_t b = blockIdx.y;
  const int64_t n_groups = nwords * 8 / group;
  float acc = 0.f;
  for (int64_t wi = lane; wi < nwords; wi += 64) {
    const uint32_t word = kn ? w[wi * n_out + row] : w[row * nwords + wi];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t k = wi * 8 + i;
      const int64_t g = k / group;
      const float s = ld_f(scales, s_dt, kn ? g * n_out + row : row * n_groups + g);
      const float bb = ld_f(biases, b_dt, kn ? g * n_out + row : row * n_groups + g);
      const float q = static_cast<float>((word >> (4 * i)) & 15u);
      acc += (q * s + bb) * ld_f(x, x_dt, b * ldx + k);
    }
  }
  acc = group_sum<64>(acc);
  if (lane == 0) st_f(y, x_dt, b * ldy + row, acc);
}

__global__ __launch_bounds__(256) void k_rtn4_embed(
    const void* __restrict__ ids, int ids64, int64_t vocab, const uint32_t* __restrict__ w,
    int64_t nwords, const void* __restrict__ scales, int s_dt,
    const void* __restrict__ biases, int b_dt, int64_t group, float* __restrict__ out) {
  const int64_t i = blockIdx.x;
  int64_t id = ld_id(ids, ids64, i);
  id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);  // clamp: never read outside the table
  const int64_t n_groups = nwords * 8 / group;
  for (int64_t wi = threadIdx.x; wi < nwords; wi += 256) {
    const uint32_t word = w[id * nwords + wi];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t k = wi * 8 + j;
      const int64_t g = k / group;
      const float s = ld_f(scales, s_dt, id * n_groups + g);
      const float bb = ld_f(biases, b_dt, id * n_groups + g);
      out[i * nwords * 8 + k] = static_cast<float>((word >> (4 * j)) & 15u) * s + bb;
    }
  }
}

template <int BT>
static bool rtn4_fast_launch(const void* x, int64_t batch, int64_t ldx, const uint32_t* w,
                             int64_t n_out, int64_t nwords, const void* sc, const void* bs,
                             int s_dt, int64_t group, void* y, int64_t ldy, hipStream_t s) {
  const int64_t gw = group / 8;  // words per group
  const int64_t n_groups = nwords / gw;
#define MA_RTN4(L, K)                                                                        \
  if (nwords == (L) * (K) && gw % (K) == 0) {                                                \
    constexpr int U = 4;                                                                     \
    dim3 grid(static_cast<unsigned>(cdiv(n_out, (64 / L) * U)),                              \
              static_cast<unsigned>(cdiv(batch, BT)));                                       \
    if (s_dt == MA_BF16)                                                                     \
      hipLaunchKernelGGL((k_rtn4_fast<K, L, BT, U, MA_BF16>), grid, dim3(64), 0, s,          \
                         static_cast<const uint16_t*>(x), batch, ldx, w, n_out, n_groups, gw, \
                         sc, bs, static_cast<uint16_t*>(y), ldy);                            \
    else                                                                                     \
      hipLaunchKernelGGL((k_rtn4_fast<K, L, BT, U, MA_F32>), grid, dim3(64), 0, s,           \
                         static_cast<const uint16_t*>(x), batch, ldx, w, n_out, n_groups, gw, \
                         sc, bs, static_cast<uint16_t*>(y), ldy);                            \
    return true;                                                                             \
  }
  MA_RTN4(32, 8)
  MA_RTN4(32, 4)
  MA_RTN4(32, 2)
  MA_RTN4(16, 4)
  MA_RTN4(16, 2)
  MA_RTN4(8, 2)
#undef MA_RTN4
  return false;
}

}  // namespace ma

using namespace ma;

// Batched MFMA path (dense_mfma.hip) for batch >= 5.
int launch_rtn4_mfma(const uint16_t* x, int64_t batch, int64_t ldx, const uint32_t* w,
                     int64_t n_out, int64_t nwords, int64_t group, const void* scales,
                     const void* biases, int s_dt, uint16_t* y, int64_t ldy, hipStream_t s);

extern "C" int ma_rtn4_gemv(const void* x, int x_dtype, int64_t batch, int64_t ldx,
                            const uint32_t* packed, int64_t n_out, int64_t nwords, int packed_kn,
                            const void* scales, int scales_dtype, const void* biases,
                            int biases_dtype, int64_t group_size, void* y, int64_t ldy,
                            void* stream) {
  if (batch < 0 || n_out < 0 || nwords < 1 || group_size < 8 || group_size % 8 ||
      (nwords * 8) % group_size)
    return fail(MA_EVALUE, "rtn4_gemv: K=%lld is not a whole number of groups of %lld",
                (long long)(nwords * 8), (long long)group_size);
  if (batch == 0 || n_out == 0) return MA_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool fast = x_dtype == MA_BF16 && !packed_kn && scales_dtype == biases_dtype &&
                    (scales_dtype == MA_BF16 || scales_dtype == MA_F32) && (ldx % 8) == 0 &&
                    ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(packed)) & 15u) == 0;
  if (fast && batch >= 5 && (group_size == 64 || group_size == 128) && nwords % 16 == 0 &&
      (reinterpret_cast<uintptr_t>(y) & 15u) == 0)
    return launch_rtn4_mfma(static_cast<const uint16_t*>(x), batch, ldx, packed, n_out, nwords,
                            group_size, scales, biases, scales_dtype, static_cast<uint16_t*>(y),
                            ldy, s);
  if (fast) {
    bool done;
    if (batch >= 4)
      done = rtn4_fast_launch<4>(x, batch, ldx, packed, n_out, nwords, scales, biases, scales_dtype, group_size, y, ldy, s);
    else if (batch >= 2)
      done = rtn4_fast_launch<2>(x, batch, ldx, packed, n_out, nwords, scales, biases, scales_dtype, group_size, y, ldy, s);
    else
      done = rtn4_fast_launch<1>(x, batch, ldx, packed, n_out, nwords, scales, biases, scales_dtype, group_size, y, ldy, s);
    if (done) return check_launch("rtn4_gemv");
  }
  dim3 grid(static_cast<unsigned>(cdiv(n_out, 4)), static_cast<unsigned>(batch));
  hipLaunchKernelGGL(k_rtn4_generic, grid, dim3(256), 0, s, x, x_dtype, batch, ldx, packed, n_out,
                     nwords, packed_kn, scales, scales_dtype, biases, biases_dtype, group_size, y,
                     ldy);
  return check_launch("rtn4_gemv");
}

extern "C" int ma_rtn4_embedding(const void* ids, int ids_is_int64, int64_t n_ids,
                                 const uint32_t* packed, int64_t vocab, int64_t nwords,
                                 const void* scales, int scales_dtype, const void* biases,
                                 int biases_dtype, int64_t group_size, float* out, void* stream) {
  if (n_ids < 0 || vocab < 1 || nwords < 1 || group_size < 8 || (nwords * 8) % group_size)
    return fail(MA_EVALUE, "rtn4_embedding: bad sizes");
  if (n_ids == 0) return MA_OK;
  hipLaunchKernelGGL(k_rtn4_embed, dim3(static_cast<unsigned>(n_ids)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), ids, ids_is_int64, vocab, packed, nwords,
                     scales, scales_dtype, biases, biases_dtype, group_size, out);
  return check_launch("rtn4_embedding");
}
