// Fast ternary GEMV instances: 2 activation row(s) per pass, fused RMSNorm.
#include "tgemv_fast.h"

namespace ma {
bool tgemv_fast_rms2(int lpr, int kw, const void* x, int64_t batch, int64_t ldx,
                     const uint32_t* w, int64_t n_out, const void* alpha, int alpha_dt,
                     const void* rms_w, int rms_dt, float eps, void* y, int64_t ldy,
                     hipStream_t s) {
  return tgemv_fast_variant<2, true>(lpr, kw, x, batch, ldx, w, n_out, alpha, alpha_dt,
                                      rms_w, rms_dt, eps, y, ldy, s);
}
}  // namespace ma
