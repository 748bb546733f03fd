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

// Rows: output row r reads weight row r; with MAP, weight row src(r) =
// cid[r / cs] * cs + r % cs (cid NULL: src = r), clamped to [0, n_src), and
// the output goes to y[out_idx[src]] (out_idx NULL: y[r]), clamped to
// [0, n_dst) -- the FlashHead gathers and scatters; no index read from
// memory can send an access outside the buffers.  The per-row arithmetic is
// the same either way.
template <int KW, int LPR, int BT, int U, int SDT, bool MAP = false>
__global__ __launch_bounds__(64) void k_rtn4_fast(
    const uint16_t* __restrict__ x, int64_t batch, int64_t ldx,
    const uint32_t* __restrict__ w, int64_t n_out, int64_t n_groups, int64_t gw,
    const void* __restrict__ scales, const void* __restrict__ biases,
    uint16_t* __restrict__ y, int64_t ldy, const int32_t* __restrict__ cid = nullptr,
    int64_t cs = 1, const int32_t* __restrict__ out_idx = nullptr, int64_t n_src = 1,
    int64_t n_dst = 1) {
  constexpr int NW = KW * LPR;
  constexpr int RPI = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int kl = lane % LPR, sub = lane / LPR;
  const int64_t g = (static_cast<int64_t>(kl) * KW) / gw;  // the lane's RTN group
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * (RPI * U);
  const int64_t b0 = static_cast<int64_t>(blockIdx.y) * BT;

  uint32_t wv[U][KW];
  float sc[U], bi[U];
  int64_t src[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    int64_t r = r0 + u * RPI + sub;
    r = r < n_out ? r : n_out - 1;
    if constexpr (MAP) {
      r = cid ? static_cast<int64_t>(cid[r / cs]) * cs + r % cs : r;
      r = r < 0 ? 0 : (r >= n_src ? n_src - 1 : r);
    }
    src[u] = r;
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t r = src[u];
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
      int64_t o = r;
      if constexpr (MAP) {
        o = out_idx ? static_cast<int64_t>(out_idx[src[u]]) : r;
        o = o < 0 ? 0 : (o >= n_dst ? n_dst - 1 : o);
      }
      if (kl == 0 && r < n_out && b < batch) y[b * ldy + o] = f32_to_bf16(v);
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
    if (group % 8 == 0) {
      // one group per word: its scale and bias read once, as raw words from a
      // dtype-selected address (no dtype branch: a load converted in one
      // waits right there, and this loop issued sixteen such loads a word)
      const int64_t gi = id * n_groups + wi * 8 / group;
      const AnyWord sw = ld_any_word(scales, s_dt, gi), bw = ld_any_word(biases, b_dt, gi);
      const float s = any_word_f(sw, s_dt), bb = any_word_f(bw, b_dt);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        out[i * nwords * 8 + wi * 8 + j] = static_cast<float>((word >> (4 * j)) & 15u) * s + bb;
    } else {
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

// The same GEMV over mapped rows (batch rows on the grid's y, one at a time):
// MA_EVALUE-free launcher; false when no fast shape fits.
static bool rtn4_rows_launch(const void* x, int64_t batch, int64_t ldx, const uint32_t* w,
                             int64_t n_out, int64_t nwords, const void* sc, const void* bs, int s_dt,
                             int64_t group, void* y, int64_t ldy, const int32_t* cid, int64_t cs,
                             const int32_t* out_idx, int64_t n_src, int64_t n_dst, hipStream_t s) {
  const int64_t gw = group / 8;
  const int64_t n_groups = nwords / gw;
#define MA_RTN4_MAP(L, K)                                                                        \
  if (nwords == (L) * (K) && gw % (K) == 0) {                                                    \
    constexpr int U = 4;                                                                         \
    dim3 grid(static_cast<unsigned>(cdiv(n_out, (64 / L) * U)), static_cast<unsigned>(batch));   \
    if (s_dt == MA_BF16)                                                                         \
      hipLaunchKernelGGL((k_rtn4_fast<K, L, 1, U, MA_BF16, true>), grid, dim3(64), 0, s,         \
                         static_cast<const uint16_t*>(x), batch, ldx, w, n_out, n_groups, gw, sc, \
                         bs, static_cast<uint16_t*>(y), ldy, cid, cs, out_idx, n_src, n_dst);     \
    else                                                                                         \
      hipLaunchKernelGGL((k_rtn4_fast<K, L, 1, U, MA_F32, true>), grid, dim3(64), 0, s,          \
                         static_cast<const uint16_t*>(x), batch, ldx, w, n_out, n_groups, gw, sc, \
                         bs, static_cast<uint16_t*>(y), ldy, cid, cs, out_idx, n_src, n_dst);     \
    return true;                                                                                 \
  }
  MA_RTN4_MAP(32, 8)
  MA_RTN4_MAP(32, 4)
  MA_RTN4_MAP(32, 2)
  MA_RTN4_MAP(16, 4)
  MA_RTN4_MAP(16, 2)
  MA_RTN4_MAP(8, 2)
#undef MA_RTN4_MAP
  return false;
}

// ---------------------------------------------------------------------------
// FlashHead cluster selection (reference flash_head.py:345-351: torch.topk of
// the centroid scores): the n_probes largest of n_clusters bf16 scores, equal
// scores at the lower cluster index, written as ascending cluster ids.  One
// 1024-thread workgroup, thread t holding scores 8t .. 8t+7 (one 16-byte
// load).  A bf16 score's order-preserving key has 16 bits, so the radix
// select of the n_probes-th largest key takes two 8-bit digit passes over
// per-wave LDS histograms; then one workgroup scan places the keys above it
// and one the lowest-index keys equal to it.  Workgroups 1 .. fill the full
// vocabulary row of logits with -inf meanwhile.
constexpr int kSelThreads = 1024;
constexpr int kSelPer = 8;  // up to 8192 clusters
constexpr int kSelWaves = kSelThreads / 64;

__device__ __forceinline__ uint32_t score_key(uint32_t b) {  // bf16 bits -> 16-bit order key
  return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
}

// Exclusive prefix over the workgroup of per-thread counts (thread order);
// *total gets the sum.  Uses sh[kSelWaves].
__device__ __forceinline__ int block_excl_scan(int v, int* sh, int* total) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  int inc = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(inc, off, 64);
    if (lane >= off) inc += u;
  }
  if (lane == 63) sh[wv] = inc;
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kSelWaves; ++w) {
    base += w < wv ? sh[w] : 0;
    tot += sh[w];
  }
  __syncthreads();
  *total = tot;
  return base + inc - v;
}

__global__ __launch_bounds__(kSelThreads) void k_flash_select(const uint16_t* __restrict__ scores,
                                                              int n, int k, int32_t* __restrict__ ids,
                                                              uint16_t* __restrict__ full, int64_t vocab) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  if (blockIdx.x > 0) {  // fill: 8 bf16 of -inf per thread
    const int64_t i = (static_cast<int64_t>(blockIdx.x - 1) * kSelThreads + tid) * 8;
    if (i + 8 <= vocab) {
      *reinterpret_cast<uint4*>(full + i) = make_uint4(0xff80ff80u, 0xff80ff80u, 0xff80ff80u, 0xff80ff80u);
    } else {
      for (int64_t j = i; j < vocab; ++j) full[j] = 0xff80u;
    }
    return;
  }
  __shared__ int hist[kSelWaves][256];
  __shared__ int tot[256];
  __shared__ int sh[kSelWaves];
  __shared__ uint32_t s_prefix;
  __shared__ int s_need;
  uint32_t key[kSelPer];  // 16-bit order keys; indices past n are not valid
  bool valid[kSelPer];
  const int i0 = tid * kSelPer;
  if (i0 + kSelPer <= n && (n & 7) == 0) {
    const uint4 v = *reinterpret_cast<const uint4*>(scores + i0);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      key[2 * q] = score_key(w[q] & 0xffffu);
      key[2 * q + 1] = score_key(w[q] >> 16);
    }
  } else {
#pragma unroll
    for (int j = 0; j < kSelPer; ++j) key[j] = i0 + j < n ? score_key(scores[i0 + j]) : 0u;
  }
#pragma unroll
  for (int j = 0; j < kSelPer; ++j) valid[j] = i0 + j < n;
  uint32_t prefix = 0, mask = 0;
  int need = k;  // rank, from the top, of the wanted key among those matching the prefix
  for (int pass = 0; pass < 2; ++pass) {
    const int shift = 8 - 8 * pass;  // digits: key bits 15..8, then 7..0
    for (int i = tid; i < kSelWaves * 256; i += kSelThreads) (&hist[0][0])[i] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kSelPer; ++j)
      if (valid[j] && (key[j] & mask) == prefix) atomicAdd(&hist[wv][(key[j] >> shift) & 255u], 1);
    __syncthreads();
    if (tid < 256) {
      int c = 0;
#pragma unroll
      for (int w = 0; w < kSelWaves; ++w) c += hist[w][tid];
      tot[tid] = c;
    }
    __syncthreads();
    if (wv == 0) {
      int c4[4], own = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        c4[q] = tot[4 * lane + q];
        own += c4[q];
      }
      int suf = own;  // inclusive suffix over lanes >= lane
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int u = __shfl_down(suf, off, 64);
        if (lane + off < 64) suf += u;
      }
      // the digit d with (count above d) < need <= (count above d) + count(d)
      int hit_d = -1, hit_above = 0, above = suf - own;
#pragma unroll
      for (int q = 3; q >= 0; --q) {
        if (hit_d < 0 && above < need && need <= above + c4[q]) {
          hit_d = 4 * lane + q;
          hit_above = above;
        }
        above += c4[q];
      }
      const uint64_t hb = __ballot(hit_d >= 0);
      const int src = hb ? __builtin_ctzll(hb) : 0;
      const int d = __shfl(hit_d, src, 64), a = __shfl(hit_above, src, 64);
      if (lane == 0) {
        s_prefix = prefix | (static_cast<uint32_t>(d < 0 ? 0 : d) << shift);
        s_need = need - a;
      }
    }
    __syncthreads();
    prefix = s_prefix;
    need = s_need;
    mask |= 255u << shift;
  }
  // prefix is the k-th largest key: take every key above it and the lowest
  // `need` indices equal to it, in index order
  int ties = 0;
#pragma unroll
  for (int j = 0; j < kSelPer; ++j) ties += (valid[j] && key[j] == prefix) ? 1 : 0;
  int tie_total;
  int tie_rank = block_excl_scan(ties, sh, &tie_total);
  bool take[kSelPer];
  int cnt = 0;
#pragma unroll
  for (int j = 0; j < kSelPer; ++j) {
    const bool tie = valid[j] && key[j] == prefix;
    take[j] = (valid[j] && key[j] > prefix) || (tie && tie_rank < need);
    tie_rank += tie ? 1 : 0;
    cnt += take[j] ? 1 : 0;
  }
  int take_total;
  int pos = block_excl_scan(cnt, sh, &take_total);
#pragma unroll
  for (int j = 0; j < kSelPer; ++j)
    if (take[j]) {
      if (pos < k) ids[pos] = i0 + j;
      ++pos;
    }
}

}  // namespace ma

using namespace ma;

// Batched MFMA path (dense_mfma.hip) for batch >= 5, and its workspace form.
int launch_rtn4_mfma(const uint16_t* x, int64_t batch, int64_t ldx, const uint32_t* w,
                     int64_t n_out, int64_t nwords, int64_t group, const void* scales,
                     const void* biases, int s_dt, uint16_t* y, int64_t ldy, hipStream_t s);
int launch_rtn4_mfma_ws(const uint16_t* x, int64_t batch, int64_t ldx, const uint32_t* w,
                        int64_t n_out, int64_t nwords, int64_t group, const void* scales,
                        const void* biases, int s_dt, uint16_t* y, int64_t ldy, void* workspace,
                        hipStream_t s);
namespace ma {
size_t rtn4_ws_bytes(int64_t batch, int64_t nwords, int64_t group);
}  // namespace ma

// Whether a call takes the workspace form: the batched MFMA path (bf16 x,
// [N, K/8] codes, 16-byte aligned) in groups of 128 over a whole number of
// 32-row blocks.
static bool rtn4_ws_form(int x_dtype, int64_t batch, int64_t ldx, const void* x, const void* packed,
                         int64_t n_out, int64_t nwords, int packed_kn, int scales_dtype, int biases_dtype,
                         int64_t group_size, const void* y) {
  return x_dtype == MA_BF16 && !packed_kn && scales_dtype == biases_dtype &&
         (scales_dtype == MA_BF16 || scales_dtype == MA_F32) && (ldx % 8) == 0 && batch >= 5 &&
         group_size == 128 && nwords % 16 == 0 && n_out % 32 == 0 &&
         ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(packed) |
           reinterpret_cast<uintptr_t>(y)) & 15u) == 0;
}

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

extern "C" size_t ma_rtn4_gemv_workspace_bytes(int64_t batch, int64_t nwords, int64_t group_size) {
  if (batch < 5 || group_size != 128 || nwords < 16 || nwords % 16) return 0;
  return rtn4_ws_bytes(batch, nwords, group_size);
}

extern "C" int ma_rtn4_gemv_ws(const void* x, int x_dtype, int64_t batch, int64_t ldx,
                               const uint32_t* packed, int64_t n_out, int64_t nwords, int packed_kn,
                               const void* scales, int scales_dtype, const void* biases,
                               int biases_dtype, int64_t group_size, void* y, int64_t ldy,
                               void* workspace, size_t workspace_bytes, void* stream) {
  if (batch > 0 && n_out > 0 &&
      rtn4_ws_form(x_dtype, batch, ldx, x, packed, n_out, nwords, packed_kn, scales_dtype, biases_dtype,
                   group_size, y)) {
    if (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 255u) ||
        workspace_bytes < rtn4_ws_bytes(batch, nwords, group_size))
      return fail(MA_EVALUE, "rtn4_gemv_ws: workspace missing, misaligned or under %zu bytes",
                  rtn4_ws_bytes(batch, nwords, group_size));
    return launch_rtn4_mfma_ws(static_cast<const uint16_t*>(x), batch, ldx, packed, n_out, nwords, group_size,
                               scales, biases, scales_dtype, static_cast<uint16_t*>(y), ldy, workspace,
                               static_cast<hipStream_t>(stream));
  }
  return ma_rtn4_gemv(x, x_dtype, batch, ldx, packed, n_out, nwords, packed_kn, scales, scales_dtype, biases,
                      biases_dtype, group_size, y, ldy, stream);
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

extern "C" int ma_rtn4_indexed_gemv(const void* x, int x_dtype, int64_t batch, int64_t ldx,
                                    const uint32_t* packed, int64_t n_clusters, int64_t cluster_size,
                                    int64_t nwords, const void* scales, int scales_dtype,
                                    const void* biases, int biases_dtype, int64_t group_size,
                                    const int32_t* cluster_ids, int64_t n_probes, void* y, int64_t ldy,
                                    void* stream) {
  if (batch < 0 || n_clusters < 1 || cluster_size < 1 || n_probes < 0 || nwords < 1 ||
      group_size < 8 || group_size % 8 || (nwords * 8) % group_size || ldy < n_probes * cluster_size)
    return fail(MA_EVALUE, "rtn4_indexed_gemv: bad sizes");
  if (x_dtype != MA_BF16 || scales_dtype != biases_dtype || (scales_dtype != MA_BF16 && scales_dtype != MA_F32))
    return fail(MA_ETYPE, "rtn4_indexed_gemv: needs bf16 x and bf16 or float32 scales/biases of one dtype");
  if ((ldx % 8) || ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(packed)) & 15u))
    return fail(MA_EVALUE, "rtn4_indexed_gemv: x rows and codes must be 16-byte aligned");
  if (batch == 0 || n_probes == 0) return MA_OK;
  if (!rtn4_rows_launch(x, batch, ldx, packed, n_probes * cluster_size, nwords, scales, biases,
                        scales_dtype, group_size, y, ldy, cluster_ids, cluster_size, nullptr,
                        n_clusters * cluster_size, n_probes * cluster_size, static_cast<hipStream_t>(stream)))
    return fail(MA_EVALUE, "rtn4_indexed_gemv: %lld words per row with group %lld not built",
                (long long)nwords, (long long)group_size);
  return check_launch("rtn4_indexed_gemv");
}

extern "C" size_t ma_flash_head_workspace_bytes(int64_t n_clusters, int64_t n_probes) {
  if (n_clusters < 1 || n_probes < 1) return 0;
  return ((static_cast<size_t>(n_clusters) * 2 + 255) / 256) * 256 + static_cast<size_t>(n_probes) * 4;
}

extern "C" int ma_flash_head(const void* x, const uint32_t* centroids, const void* c_scales,
                             const void* c_biases, int c_dtype, int64_t n_clusters, int64_t c_group,
                             const uint32_t* head, const void* h_scales, const void* h_biases,
                             int h_dtype, int64_t cluster_size, int64_t h_group,
                             const int32_t* token_map, int64_t n_probes, const uint32_t* force_w,
                             const void* force_scales, const void* force_biases,
                             const int32_t* force_ids, int64_t n_force, int64_t nwords, int64_t vocab,
                             void* logits, int32_t* cluster_ids, void* workspace,
                             size_t workspace_bytes, void* stream) {
  const char* what = "flash_head";
  if (n_clusters < 1 || cluster_size < 1 || n_probes < 1 || n_probes > n_clusters ||
      n_clusters > static_cast<int64_t>(kSelThreads) * kSelPer || nwords < 1 || vocab < 1 || n_force < 0)
    return fail(MA_EVALUE, "%s: bad sizes (n_probes %lld of %lld clusters, at most %d clusters)", what,
                (long long)n_probes, (long long)n_clusters, kSelThreads * kSelPer);
  for (int64_t gsz : {c_group, h_group})
    if (gsz < 8 || gsz % 8 || (nwords * 8) % gsz) return fail(MA_EVALUE, "%s: bad group size %lld", what, (long long)gsz);
  if ((c_dtype != MA_BF16 && c_dtype != MA_F32) || (h_dtype != MA_BF16 && h_dtype != MA_F32))
    return fail(MA_ETYPE, "%s: scales/biases must be bf16 or float32", what);
  if (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(centroids) |
        reinterpret_cast<uintptr_t>(head) | reinterpret_cast<uintptr_t>(logits) |
        (force_w ? reinterpret_cast<uintptr_t>(force_w) : 0)) & 15u))
    return fail(MA_EVALUE, "%s: x, codes and logits must be 16-byte aligned", what);
  if (n_force > 0 && (!force_w || !force_scales || !force_biases || !force_ids))
    return fail(MA_EVALUE, "%s: force rows missing", what);
  if (!workspace || workspace_bytes < ma_flash_head_workspace_bytes(n_clusters, n_probes) ||
      (reinterpret_cast<uintptr_t>(workspace) & 255u))
    return fail(MA_EVALUE, "%s: workspace too small or not 256-byte aligned", what);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint16_t* scores = static_cast<uint16_t*>(workspace);
  int32_t* ids = cluster_ids ? cluster_ids
                             : reinterpret_cast<int32_t*>(static_cast<char*>(workspace) +
                                                          ((n_clusters * 2 + 255) / 256) * 256);
  // 1. centroid scores (the exact head's GEMV on the centroid rows), bf16
  if (!rtn4_fast_launch<1>(x, 1, nwords * 8, centroids, n_clusters, nwords, c_scales, c_biases, c_dtype,
                           c_group, scores, n_clusters, s))
    return fail(MA_EVALUE, "%s: %lld words per row with group %lld not built", what, (long long)nwords,
                (long long)c_group);
  // 2. the probed clusters; the rest of the grid fills the logits with -inf
  const unsigned fill = static_cast<unsigned>(cdiv(vocab, static_cast<int64_t>(kSelThreads) * 8));
  hipLaunchKernelGGL(k_flash_select, dim3(1 + fill), dim3(kSelThreads), 0, s, scores,
                     static_cast<int>(n_clusters), static_cast<int>(n_probes), ids,
                     static_cast<uint16_t*>(logits), vocab);
  // 3. exact logits of the probed clusters' tokens, scattered through token_map
  if (!rtn4_rows_launch(x, 1, nwords * 8, head, n_probes * cluster_size, nwords, h_scales, h_biases,
                        h_dtype, h_group, logits, vocab, ids, cluster_size, token_map,
                        n_clusters * cluster_size, vocab, s))
    return fail(MA_EVALUE, "%s: %lld words per row with group %lld not built", what, (long long)nwords,
                (long long)h_group);
  // 4. forced tokens (EOS and the like) from their own rows of the head
  if (n_force > 0 &&
      !rtn4_rows_launch(x, 1, nwords * 8, force_w, n_force, nwords, force_scales, force_biases, h_dtype,
                        h_group, logits, vocab, nullptr, 1, force_ids, n_force, vocab, s))
    return fail(MA_EVALUE, "%s: force rows not built", what);
  return check_launch(what);
}
