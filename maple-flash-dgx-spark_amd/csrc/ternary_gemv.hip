// Packed ternary GEMV y = alpha * (T . x_hat), gfx950: entry point and the
// generic kernel (any float dtype, either code layout, any K).  The bf16 fast
// kernels are in tgemv_fast.h.
//
// Semantics follow reference src/maple_run/kernels/ternary_gemv.py:76-258:
// float32 accumulation over the exact ternary values, alpha applied once per
// row, optional fused input RMSNorm folded as acc * rsqrt(sum x^2 / K + eps)
// with x_hat = x * w_rms, output stored in x's dtype.
#include "tgemv_fast.h"

namespace ma {

template <int BT>
__global__ __launch_bounds__(256) void k_tgemv_generic(
    const void* __restrict__ x, int x_dt, int64_t batch, int64_t ldx,
    const uint32_t* __restrict__ w, int64_t n_out, int64_t nwords, int kn,
    const void* __restrict__ alpha, int alpha_dt,
    const void* __restrict__ rms_w, int rms_dt, float eps,
    void* __restrict__ y, int64_t ldy) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= n_out) return;  // uniform per wave
  const int64_t b0 = static_cast<int64_t>(blockIdx.y) * BT;
  const int64_t k_total = nwords * 16;
  const bool rms = rms_w != nullptr;
  float acc[BT], ss[BT];
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) acc[bt] = ss[bt] = 0.f;
  for (int64_t wi = lane; wi < nwords; wi += 64) {
    const uint32_t word = kn ? w[wi * n_out + row] : w[row * nwords + wi];
#pragma unroll 4
    for (int i = 0; i < 16; ++i) {
      const float v = static_cast<float>((word >> (2 * i)) & 3u) - 1.0f;
      const int64_t k = wi * 16 + i;
      const float rw = rms ? ld_f(rms_w, rms_dt, k) : 1.0f;
#pragma unroll
      for (int bt = 0; bt < BT; ++bt) {
        const int64_t b = b0 + bt;
        if (b < batch) {
          const float xv = ld_f(x, x_dt, b * ldx + k);
          ss[bt] += xv * xv;
          acc[bt] += v * (xv * rw);
        }
      }
    }
  }
  const float a = ld_f(alpha, alpha_dt, row);
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) {
    const float s = group_sum<64>(acc[bt]);
    const float q = group_sum<64>(ss[bt]);
    const int64_t b = b0 + bt;
    if (lane == 0 && b < batch) {
      float v = s;
      if (rms) v = v * rsqrtf(q / static_cast<float>(k_total) + eps);
      st_f(y, x_dt, b * ldy + row, v * a);
    }
  }
}

static bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Returns true when the fast kernel was launched.
bool tgemv_fast(const void* x, int x_dtype, int64_t batch, int64_t ldx, const uint32_t* w,
                int64_t n_out, int64_t nwords, int packed_kn, const void* alpha, int alpha_dt,
                const void* rms_w, int rms_dt, float eps, void* y, int64_t ldy, hipStream_t s) {
  if (x_dtype != MA_BF16 || packed_kn) return false;
  if (alpha_dt != MA_BF16 && alpha_dt != MA_F32) return false;
  if (rms_w && rms_dt != MA_F32) return false;
  int lpr = 0, kw = 0;
  if (!tgemv_fast_shape(nwords, lpr, kw)) return false;
  const uintptr_t walign = (kw % 4 == 0) ? 16 : (kw % 2 == 0) ? 8 : 4;
  if (!aligned(w, walign) || !aligned(x, 16) || (ldx % 8) != 0) return false;
  if (rms_w) {
    if (batch >= 2) return tgemv_fast_rms2(lpr, kw, x, batch, ldx, w, n_out, alpha, alpha_dt, rms_w, rms_dt, eps, y, ldy, s);
    return tgemv_fast_rms1(lpr, kw, x, batch, ldx, w, n_out, alpha, alpha_dt, rms_w, rms_dt, eps, y, ldy, s);
  }
  if (batch >= 4) return tgemv_fast_b4(lpr, kw, x, batch, ldx, w, n_out, alpha, alpha_dt, nullptr, 0, eps, y, ldy, s);
  if (batch >= 2) return tgemv_fast_b2(lpr, kw, x, batch, ldx, w, n_out, alpha, alpha_dt, nullptr, 0, eps, y, ldy, s);
  return tgemv_fast_b1(lpr, kw, x, batch, ldx, w, n_out, alpha, alpha_dt, nullptr, 0, eps, y, ldy, s);
}

void tgemv_generic(const void* x, int x_dtype, int64_t batch, int64_t ldx, const uint32_t* w,
                   int64_t n_out, int64_t nwords, int packed_kn, const void* alpha, int alpha_dt,
                   const void* rms_w, int rms_dt, float eps, void* y, int64_t ldy, hipStream_t s) {
  const int64_t bt = batch >= 4 ? 4 : 1;
  dim3 grid(static_cast<unsigned>(cdiv(n_out, 4)), static_cast<unsigned>(cdiv(batch, bt)));
  if (bt == 4)
    hipLaunchKernelGGL(k_tgemv_generic<4>, grid, dim3(256), 0, s, x, x_dtype, batch, ldx, w,
                       n_out, nwords, packed_kn, alpha, alpha_dt, rms_w, rms_dt, eps, y, ldy);
  else
    hipLaunchKernelGGL(k_tgemv_generic<1>, grid, dim3(256), 0, s, x, x_dtype, batch, ldx, w,
                       n_out, nwords, packed_kn, alpha, alpha_dt, rms_w, rms_dt, eps, y, ldy);
}

}  // namespace ma

// Batched MFMA path (dense_mfma.hip), batch >= kMfmaMinBatch.
int launch_tgemm_mfma(const uint16_t* x, int64_t batch, int64_t ldx, const uint32_t* w,
                      int64_t n_out, int64_t nwords, const void* alpha, int alpha_dt,
                      const void* rms_w, int rms_dt, float rms_eps, uint16_t* y, int64_t ldy,
                      hipStream_t s);
// Two-launch MFMA path (RMS-folded; x' operands built once per token into a
// workspace), taken by ma_ternary_gemv_ws from kXpMinBatch tokens.
size_t tgemm_xp_bytes(int64_t batch, int64_t nwords);
int launch_tgemm_xp(const uint16_t* x, int64_t batch, int64_t ldx, const uint32_t* w,
                    int64_t n_out, int64_t nwords, const void* alpha, int alpha_dt,
                    const void* rms_w, int rms_dt, float rms_eps, uint16_t* y, int64_t ldy,
                    void* workspace, hipStream_t s, const ma::CombineIn& cb);
constexpr int64_t kMfmaMinBatch = 5;
constexpr int64_t kXpMinBatch = 17;

static bool mfma_ok(const void* x, int x_dtype, int64_t batch, int64_t ldx, const uint32_t* packed,
                    int64_t nwords, int packed_kn, int alpha_dtype, const void* rms_weight,
                    int rms_dtype, const void* y) {
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  return batch >= kMfmaMinBatch && x_dtype == MA_BF16 && !packed_kn && nwords % 16 == 0 &&
         (alpha_dtype == MA_BF16 || alpha_dtype == MA_F32) &&
         (!rms_weight || rms_dtype == MA_F32 || rms_dtype == MA_BF16) && a16(x) && ldx % 8 == 0 &&
         a16(packed) && a16(y) && (!rms_weight || a16(rms_weight));
}

extern "C" int ma_ternary_gemv(const void* x, int x_dtype, int64_t batch, int64_t ldx,
                               const uint32_t* packed, int64_t n_out, int64_t nwords,
                               int packed_kn, const void* row_alpha, int alpha_dtype,
                               const void* rms_weight, int rms_dtype, float rms_eps, void* y,
                               int64_t ldy, void* stream) {
  using namespace ma;
  if (batch < 0 || n_out < 0 || nwords < 1)
    return fail(MA_EVALUE, "ternary_gemv: bad sizes batch=%lld n=%lld nwords=%lld",
                (long long)batch, (long long)n_out, (long long)nwords);
  if (batch == 0 || n_out == 0) return MA_OK;
  if (!x || !packed || !row_alpha || !y) return fail(MA_EVALUE, "ternary_gemv: null pointer");
  if (ldx < nwords * 16 || ldy < n_out)
    return fail(MA_EVALUE, "ternary_gemv: leading dimension too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (mfma_ok(x, x_dtype, batch, ldx, packed, nwords, packed_kn, alpha_dtype, rms_weight,
              rms_dtype, y))
    return launch_tgemm_mfma(static_cast<const uint16_t*>(x), batch, ldx, packed, n_out, nwords,
                             row_alpha, alpha_dtype, rms_weight, rms_dtype, rms_eps,
                             static_cast<uint16_t*>(y), ldy, s);
  if (!tgemv_fast(x, x_dtype, batch, ldx, packed, n_out, nwords, packed_kn, row_alpha,
                  alpha_dtype, rms_weight, rms_dtype, rms_eps, y, ldy, s))
    tgemv_generic(x, x_dtype, batch, ldx, packed, n_out, nwords, packed_kn, row_alpha,
                  alpha_dtype, rms_weight, rms_dtype, rms_eps, y, ldy, s);
  return check_launch("ternary_gemv");
}

extern "C" size_t ma_ternary_gemv_workspace_bytes(int64_t batch, int64_t nwords, int rms) {
  if (!rms || batch < kXpMinBatch || nwords < 1 || nwords % 16 != 0) return 0;
  return tgemm_xp_bytes(batch, nwords);
}

extern "C" int ma_ternary_gemv_ws(const void* x, int x_dtype, int64_t batch, int64_t ldx,
                                  const uint32_t* packed, int64_t n_out, int64_t nwords,
                                  int packed_kn, const void* row_alpha, int alpha_dtype,
                                  const void* rms_weight, int rms_dtype, float rms_eps, void* y,
                                  int64_t ldy, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  using namespace ma;
  if (batch < 0 || n_out < 0 || nwords < 1)
    return fail(MA_EVALUE, "ternary_gemv: bad sizes batch=%lld n=%lld nwords=%lld",
                (long long)batch, (long long)n_out, (long long)nwords);
  if (batch == 0 || n_out == 0) return MA_OK;
  if (!x || !packed || !row_alpha || !y) return fail(MA_EVALUE, "ternary_gemv: null pointer");
  if (ldx < nwords * 16 || ldy < n_out)
    return fail(MA_EVALUE, "ternary_gemv: leading dimension too small");
  if (!rms_weight || batch < kXpMinBatch ||
      !mfma_ok(x, x_dtype, batch, ldx, packed, nwords, packed_kn, alpha_dtype, rms_weight,
               rms_dtype, y))
    return ma_ternary_gemv(x, x_dtype, batch, ldx, packed, n_out, nwords, packed_kn, row_alpha,
                           alpha_dtype, rms_weight, rms_dtype, rms_eps, y, ldy, stream);
  const size_t need = tgemm_xp_bytes(batch, nwords);
  if (!workspace || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 255))
    return fail(MA_EVALUE,
                "ternary_gemv: workspace of %zu bytes (256-byte aligned) needed, got %zu at %p",
                need, workspace_bytes, workspace);
  return launch_tgemm_xp(static_cast<const uint16_t*>(x), batch, ldx, packed, n_out, nwords,
                         row_alpha, alpha_dtype, rms_weight, rms_dtype, rms_eps,
                         static_cast<uint16_t*>(y), ldy, workspace, static_cast<hipStream_t>(stream),
                         ma::CombineIn{});
}

extern "C" int ma_ternary_gemv_combine_ws(const void* slot_out, const int32_t* inverse,
                                          const float* topk_weight, int64_t top_k,
                                          const void* residual, void* x_out, int64_t batch,
                                          const uint32_t* packed, int64_t n_out, int64_t nwords,
                                          const void* row_alpha, int alpha_dtype,
                                          const void* rms_weight, int rms_dtype, float rms_eps,
                                          void* y, int64_t ldy, void* workspace,
                                          size_t workspace_bytes, void* stream) {
  using namespace ma;
  if (batch < 0 || n_out < 0 || nwords < 1)
    return fail(MA_EVALUE, "ternary_gemv_combine: bad sizes batch=%lld n=%lld nwords=%lld",
                (long long)batch, (long long)n_out, (long long)nwords);
  if (batch == 0 || n_out == 0) return MA_OK;
  if (!slot_out || !inverse || !topk_weight || !x_out || !packed || !row_alpha || !y || !rms_weight)
    return fail(MA_EVALUE, "ternary_gemv_combine: null pointer");
  if (top_k < 1 || top_k > 8) return fail(MA_EVALUE, "ternary_gemv_combine: top_k must be 1..8");
  if (ldy < n_out) return fail(MA_EVALUE, "ternary_gemv_combine: leading dimension too small");
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (batch < kXpMinBatch ||
      !mfma_ok(x_out, MA_BF16, batch, nwords * 16, packed, nwords, 0, alpha_dtype, rms_weight,
               rms_dtype, y) ||
      !a16(slot_out) || (residual && !a16(residual)))
    return fail(MA_EVALUE,
                "ternary_gemv_combine: needs >= %lld tokens, K a multiple of 256, bf16 rows and "
                "16-byte aligned buffers",
                (long long)kXpMinBatch);
  const size_t need = tgemm_xp_bytes(batch, nwords);
  if (!workspace || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 255))
    return fail(MA_EVALUE,
                "ternary_gemv_combine: workspace of %zu bytes (256-byte aligned) needed, got %zu at %p",
                need, workspace_bytes, workspace);
  const CombineIn cb{static_cast<const uint16_t*>(slot_out), inverse, topk_weight,
                     static_cast<int>(top_k), static_cast<const uint16_t*>(residual),
                     static_cast<uint16_t*>(x_out)};
  return launch_tgemm_xp(static_cast<const uint16_t*>(x_out), batch, nwords * 16, packed, n_out,
                         nwords, row_alpha, alpha_dtype, rms_weight, rms_dtype, rms_eps,
                         static_cast<uint16_t*>(y), ldy, workspace, static_cast<hipStream_t>(stream), cb);
}
