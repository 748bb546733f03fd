// Token-to-expert dispatch: per-expert lists of (token, slot) pairs (gfx950).
// One 1024-thread workgroup runs the stable counting sort of dispatch.h.
#include "dispatch.h"

namespace ma {

constexpr int kDispatchWaves = 16;
constexpr int kDispatchMaxExperts = 512;  // 32 KB of LDS counters

__global__ __launch_bounds__(1024) void k_dispatch(const void* __restrict__ ids, int ids64,
                                                   int64_t n_pairs, int n_exp, int bits,
                                                   int32_t* __restrict__ counts,
                                                   int32_t* __restrict__ offsets,
                                                   int32_t* __restrict__ pair_ids,
                                                   int32_t* __restrict__ inverse) {
  // base[w][e]: pass 1 counts, then running write positions.
  __shared__ int32_t base[kDispatchWaves][kDispatchMaxExperts];
  __shared__ int32_t wave_tot[kDispatchWaves];
  dispatch_block<kDispatchWaves, kDispatchMaxExperts>(
      [&](int64_t q) { return static_cast<int>(ld_id(ids, ids64, q)); }, n_pairs, n_exp, bits,
      base, wave_tot, counts, offsets, pair_ids, inverse);
}

}  // namespace ma

using namespace ma;

extern "C" int ma_moe_dispatch(const void* ids, int ids_is_int64, int64_t n_pairs, int n_experts,
                               int32_t* counts, int32_t* offsets, int32_t* pair_ids,
                               int32_t* inverse, void* stream) {
  if (n_pairs < 0 || n_pairs > 0x7fffffff) return fail(MA_EVALUE, "moe_dispatch: bad n_pairs");
  if (n_experts < 1 || n_experts > kDispatchMaxExperts)
    return fail(MA_EVALUE, "moe_dispatch: n_experts must be in [1, %d]", kDispatchMaxExperts);
  int bits = 0;
  while ((1 << bits) < n_experts) ++bits;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), 0, s, ids, ids_is_int64, n_pairs,
                     n_experts, bits, counts, offsets, pair_ids, inverse);
  return check_launch("moe_dispatch");
}
