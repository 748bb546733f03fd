// One-launch MoE FFN layer for one token (decode batch 1), gfx950.
//
// Semantics: MapleSparseMoeBlock.__call__ (reference src/maple_run/model.py:
// 448-474) at T = 1: router_topk (kernels/router.py:39-126), the expert SwiGLU
// (kernels/ternary_expert.py:240-319, h stored bf16), each slot's down
// projection rounded to bf16 (ternary_expert.py:58-122), and the top-k
// weighted float32 combine with the residual (fused_norm.py:59-96), y stored
// bf16.  Optionally the add + RMSNorm ahead
// of it (kernels/fused_norm.py:31-56): s = a + b in float32, residual =
// bf16(s), x = bf16(s * rsqrt(mean(s^2) + eps) * w).
//
// A persistent grid of G workgroups (all resident) runs four phases with two
// hand-offs between workgroups, both through device-coherent memory and with
// nothing to clear between calls:
//   1. every workgroup stages x (after the optional add + RMSNorm); workgroup
//      e < E also computes router logit e and publishes it tagged with the
//      call's number;
//   2. every workgroup polls the E tagged logits until all are this call's,
//      and runs softmax + top-k itself;
//   3. it issues its SwiGLU and down-projection weight loads (known once the
//      ids are), computes its slice of the 8 x I SwiGLU outputs, publishes it;
//   grid barrier (per-group arrival counters; each group's last arriver
//   sets the group's flag, and every workgroup polls all group flags);
//   4. it stages h and finishes its rows of y.
// (Polling all of h directly instead of the barrier measured slower: every
// workgroup re-reading 12+ KB while the last outputs land loads the same
// coherent path the producers are writing through.)
// Every wait is bounded (about 0.2 s); on timeout the workspace error word is
// set and the kernel finishes with wrong values instead of hanging.
#include "moe_fused.h"
#include "topk.h"

namespace ma {

// Workspace layout: moe_fused.h.

// The expert of top-k slot s: with BALLOT (E <= 64, s the same in every lane
// of the wave) the one lane whose expert has rank s, in scalar registers;
// otherwise entry s of a slot table in LDS.
template <bool BALLOT>
__device__ __forceinline__ int slot_expert(uint32_t rank, int s, const int32_t* tbl) {
  if constexpr (BALLOT)
    return __builtin_ctzll(__ballot(rank == static_cast<uint32_t>(s)));
  else
    return tbl[s];
}

// Shapes: H = 16 * KWH * LPRH (SwiGLU rows split over LPRH lanes), I = 16 *
// KWI * LPRI (down rows over LPRI lanes), US SwiGLU iterations and UD down
// row iterations per wave, TK experts per token, PER = ceil(E / 64), W waves
// per workgroup, ADT the row scales' dtype (fixed at compile time: a run-time
// dtype switch among the weight loads delayed their issue by 4 us).
template <int KWH, int LPRH, int US, int KWI, int LPRI, int UD, int TK, int PER, int W, int ADT>
__global__ __launch_bounds__(64 * W) void k_moe_fused(
    const uint16_t* __restrict__ xa, uint32_t* __restrict__ ws, const uint16_t* __restrict__ gate_w,
    const uint16_t* __restrict__ residual, const uint16_t* __restrict__ xb, const void* __restrict__ norm_w,
    int n_exp, int norm_dt, float eps, const float* __restrict__ bias,
    const uint32_t* __restrict__ ug, const void* __restrict__ ug_alpha,
    const uint32_t* __restrict__ dn, const void* __restrict__ dn_alpha,
    uint16_t* __restrict__ y, int32_t* __restrict__ ids_out, float* __restrict__ wts_out,
    const uint32_t* __restrict__ nx_w, const void* __restrict__ nx_alpha,
    const float* __restrict__ nx_rms, float nx_eps, int nx_rows,
    uint16_t* __restrict__ nx_out) {
  constexpr int NWH = KWH * LPRH, H = 16 * NWH;
  constexpr int NWI = KWI * LPRI, I = 16 * NWI;
  constexpr int RPIH = 64 / LPRH, PPI = RPIH / 2;      // SwiGLU: up/gate pairs per wave pass
  constexpr int OPW = US * PPI;                        // SwiGLU outputs per wave
  constexpr int RPID = 64 / LPRI;                      // down rows per wave pass
  constexpr int RPB = RPID * UD;                       // y rows per workgroup
  constexpr int SPW = TK >= W ? TK / W : 1;
  constexpr int NTH = 64 * W;                          // threads per workgroup
  static_assert(TK % W == 0 || TK < W, "top-k split over waves");

  __shared__ __align__(16) uint32_t xs[NWH][8];
  __shared__ float cw[NWH];
  __shared__ __align__(16) uint32_t hs[TK][NWI][8];
  __shared__ float hc[TK][NWI];
  __shared__ int32_t s_ids[TK];
  __shared__ uint64_t s_key[64];
  __shared__ uint32_t s_cnt[W][64];
  __shared__ int32_t s_slot[W][TK];
  __shared__ float s_wts[TK];
  __shared__ float red[W], red2[W];
  __shared__ float part[W][RPB];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = gridDim.x, wg = blockIdx.x;
  uint32_t* const flags = ws + kLine * kFlags;
  uint64_t* const logits = reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(ws) + kLogitOff);
  uint16_t* const hbuf = reinterpret_cast<uint16_t*>(reinterpret_cast<char*>(ws) + kMoeWsHeader);
  // Calls made on this workspace so far (the h barrier moves the flags to f0
  // + 1 only once every workgroup has arrived, so every workgroup reads f0);
  // this call's logits carry the tag f0 + 1.
  // (f0 is first used once x is staged: used here, every wave waited for
  // this load before requesting x)
  uint32_t f0 = ld_coh32(&flags[kLine * (wg % kBarGroups)]);
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  bool timed_out = false;
  const bool router_wg = wg < n_exp;  // workgroup e < E computes router logit e

  // The residual of this workgroup's y rows, loaded now and used at the end
  // (pointers that are always valid, so no branch makes the load wait here).
  const int ro = wg * RPB + tid;
  const int roc = ro < H ? ro : H - 1;
  const uint16_t* const res_a = xb ? xa : (residual ? residual : xa);
  const uint16_t* const res_b = xb ? xb : xa;
  const uint32_t ra = res_a[roc], rb = res_b[roc];

  uint64_t tag = 0;  // this call's: (f0 + 1) << 32, formed below
  // ---- 1. x (optionally add + RMSNorm) staged as x' pairs; workgroup e also
  // takes the dot product with router row e (loaded alongside x)
  float dot = 0.f;
  {
    // thread t owns words t, t + NTH, ... (16 values each)
    constexpr int WPT = (NWH + NTH - 1) / NTH;
    float v[WPT][16], nw[WPT][16];
    uint4 gr[WPT][2];
    float ss = 0.f;
    // Every load first, as raw words (the norm weights from an address their
    // dtype selects, not from a dtype branch), then the arithmetic: a load
    // converted inside a branch gets its wait right behind it.
    const bool nf32 = norm_dt == MA_F32;
    uint4 xr[WPT][2], br[WPT][2], nr[WPT][4];
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      const int w = tid + NTH * i;
      const int wc = w < NWH ? w : NWH - 1;
      xr[i][0] = reinterpret_cast<const uint4*>(xa + wc * 16)[0];
      xr[i][1] = reinterpret_cast<const uint4*>(xa + wc * 16)[1];
      const uint4* gp = reinterpret_cast<const uint4*>(gate_w + static_cast<int64_t>(router_wg ? wg : 0) * H + wc * 16);
      gr[i][0] = gp[0];
      gr[i][1] = gp[1];
      br[i][0] = br[i][1] = make_uint4(0u, 0u, 0u, 0u);
      nr[i][0] = nr[i][1] = nr[i][2] = nr[i][3] = br[i][0];
      if (xb) {  // the addend and the norm weights (f32: 4 x 16 bytes per word; bf16: 2 x 16, loaded twice)
        br[i][0] = reinterpret_cast<const uint4*>(xb + wc * 16)[0];
        br[i][1] = reinterpret_cast<const uint4*>(xb + wc * 16)[1];
        const uint4* np = reinterpret_cast<const uint4*>(static_cast<const char*>(norm_w) + wc * (nf32 ? 64 : 32));
        nr[i][0] = np[0];
        nr[i][1] = np[1];
        nr[i][2] = np[nf32 ? 2 : 0];
        nr[i][3] = np[nf32 ? 3 : 1];
      }
    }
    // the other arguments read before the expert loads, at once
    asm volatile("" ::"s"(eps), "s"(bias), "s"(ug), "s"(ug_alpha), "s"(dn), "s"(dn_alpha), "s"(nx_w)
                 : "memory");
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      const int w = tid + NTH * i;
      const uint32_t u[8] = {xr[i][0].x, xr[i][0].y, xr[i][0].z, xr[i][0].w,
                             xr[i][1].x, xr[i][1].y, xr[i][1].z, xr[i][1].w};
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        v[i][2 * q] = __uint_as_float(u[q] << 16);
        v[i][2 * q + 1] = __uint_as_float(u[q] & 0xffff0000u);
      }
      if (xb) {
        const uint32_t ub[8] = {br[i][0].x, br[i][0].y, br[i][0].z, br[i][0].w,
                                br[i][1].x, br[i][1].y, br[i][1].z, br[i][1].w};
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          v[i][2 * q] += __uint_as_float(ub[q] << 16);
          v[i][2 * q + 1] += __uint_as_float(ub[q] & 0xffff0000u);
        }
        const uint32_t un[16] = {nr[i][0].x, nr[i][0].y, nr[i][0].z, nr[i][0].w, nr[i][1].x, nr[i][1].y,
                                 nr[i][1].z, nr[i][1].w, nr[i][2].x, nr[i][2].y, nr[i][2].z, nr[i][2].w,
                                 nr[i][3].x, nr[i][3].y, nr[i][3].z, nr[i][3].w};
#pragma unroll
        for (int q = 0; q < 16; ++q)
          nw[i][q] = nf32 ? __uint_as_float(un[q])
                          : (q & 1 ? __uint_as_float(un[q >> 1] & 0xffff0000u) : __uint_as_float(un[q >> 1] << 16));
      }
      if (w < NWH) {
#pragma unroll
        for (int q = 0; q < 16; ++q) ss += v[i][q] * v[i][q];
      }
    }
    if (xb) {
      ss = group_sum<64>(ss);
      if (lane == 0) red[wv] = ss;
      __syncthreads();
      float ssum = red[0];
#pragma unroll
      for (int w = 1; w < W; ++w) ssum += red[w];
      const float rstd = rsqrtf(ssum / static_cast<float>(H) + eps);
#pragma unroll
      for (int i = 0; i < WPT; ++i) {
#pragma unroll
        for (int q = 0; q < 16; ++q) v[i][q] = bf16_to_f32(f32_to_bf16(v[i][q] * rstd * nw[i][q]));
      }
    }
    // the router logit first (the bf16 x words against router row wg), so
    // that it goes out before this workgroup stages its x' pairs
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      if (tid + NTH * i < NWH) {
        const uint32_t g[8] = {gr[i][0].x, gr[i][0].y, gr[i][0].z, gr[i][0].w,
                               gr[i][1].x, gr[i][1].y, gr[i][1].z, gr[i][1].w};
#pragma unroll
        for (int j = 0; j < 8; ++j) dot = dot2(pack_bf16x2(v[i][2 * j], v[i][2 * j + 1]), g[j], dot);
      }
    }
    if (router_wg) {
      const float s = group_sum<64>(dot);
      if (lane == 0) red2[wv] = s;
    }
    __syncthreads();
    asm volatile("" : "+v"(f0));  // (keeps f0's uses from moving up)
    tag = static_cast<uint64_t>(f0 + 1u) << 32;
    if (router_wg && tid == 0) {
      float l = red2[0];
#pragma unroll
      for (int w = 1; w < W; ++w) l += red2[w];
      st_coh64(&logits[kLogitStride * wg], tag | __float_as_uint(l + (bias ? bias[wg] : 0.f)));
    }
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      const int w = tid + NTH * i;
      if (w < NWH) {
        uint32_t pr[8];
        cw[w] = prep_word_pairs(v[i], pr);
#pragma unroll
        for (int j = 0; j < 8; ++j) xs[w][j] = pr[j];
      }
    }
  }

  // ---- 2. top-k (router semantics of reference kernels/router.py:78-126),
  // once wave 0 of every workgroup has seen all E logits of this call (each
  // lane polls its tagged logit words until they carry this call's tag).  The
  // softmax is monotonic, so the experts are picked on the logits themselves,
  // the largest first and the lowest expert index among equal ones.
  //   E <= 64: every expert's rank is counted at once.  Wave 0 puts one
  //     64-bit key per expert in LDS (the logit's order-preserving bits over
  //     the complemented index, so all keys differ and ties go to the lower
  //     index); wave w counts, for every expert, how many of keys [64/W w,
  //     64/W (w + 1)) exceed its key; the W counts sum to the expert's rank,
  //     and slot s is the one expert of rank s (a ballot).
  //   E > 64: wave 0 takes TK rounds of one wave-wide integer max and one
  //     ballot, and hands the ids over through LDS.
  // Every wave ends with the slots' experts in scalar registers and issues
  // its weight loads at once; the routing weights (p / (sum p_top + 1e-20),
  // p the softmax over all E) follow while those loads are in flight.
  float lg[PER];  // wave 0: the logits of experts lane, lane + 64, ...
  if (wv == 0) {
    bool have[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      have[i] = lane + 64 * i >= n_exp;
      lg[i] = -INFINITY;
    }
    for (;;) {
      bool done = true;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        if (!have[i]) {
          const uint64_t v = ld_coh64(&logits[kLogitStride * (lane + 64 * i)]);
          have[i] = (v & 0xffffffff00000000ull) == tag;
          lg[i] = __uint_as_float(static_cast<uint32_t>(v));
          done = done && have[i];
        }
      }
      if (__all(done) || timed_out) break;
      __builtin_amdgcn_s_sleep(2);
      timed_out = (__builtin_amdgcn_s_memrealtime() - t0) > kGridSpin;
    }
    // experts past E get INT_MIN + 1 (below every logit)
    int key[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) key[i] = lane + 64 * i < n_exp ? float_order_key(lg[i]) : INT_MIN + 1;
    if constexpr (PER == 1) {
      s_key[lane] = (static_cast<uint64_t>(static_cast<uint32_t>(key[0]) ^ 0x80000000u) << 32) |
                    static_cast<uint32_t>(~lane);
    } else {
      int my_e = 0;
#pragma unroll
      for (int s = 0; s < TK; ++s) {
        int lk = key[0];
#pragma unroll
        for (int i = 1; i < PER; ++i) lk = max(lk, key[i]);
        const int mx = wave_max_ui(lk);
        int e_s = 0;
#pragma unroll
        for (int i = PER - 1; i >= 0; --i) {  // the lowest i with a hit wins: the lowest expert index
          const uint64_t hit = __ballot(key[i] == mx);
          if (hit) e_s = __builtin_ctzll(hit) + 64 * i;
        }
#pragma unroll
        for (int i = 0; i < PER; ++i)  // chosen experts drop below every key left
          if (lane + 64 * i == e_s) key[i] = INT_MIN;
        if (lane == s) my_e = e_s;
      }
      if (lane < TK) s_ids[lane] = my_e;
    }
  }
  __syncthreads();
  uint32_t rank = 0;  // E <= 64: the rank of this lane's expert
  if constexpr (PER == 1) {
    constexpr int KPW = 64 / W;
    static_assert(64 % W == 0, "keys per wave");
    const uint64_t mine = s_key[lane];
#pragma unroll
    for (int j = 0; j < KPW; ++j) rank += s_key[KPW * wv + j] > mine ? 1u : 0u;
    s_cnt[wv][lane] = rank;
    __syncthreads();
    rank = 0;
#pragma unroll
    for (int w = 0; w < W; ++w) rank += s_cnt[w][lane];
    // this wave's own slot table (one wave's LDS accesses complete in order)
    if (rank < static_cast<uint32_t>(TK)) s_slot[wv][rank] = lane;
  }
  const int32_t* const slot_tbl = PER == 1 ? s_slot[wv] : s_ids;
  const int my_e = slot_tbl[lane < TK ? lane : 0];  // lane s < TK: slot s's expert
  if (wv == 0 && wg == 0 && lane < TK) ids_out[lane] = my_e;

  // ---- 3. weights: SwiGLU rows of this wave's h outputs, then the down rows
  // of this workgroup's y rows (every load issued before any arithmetic)
  const int klh = lane % LPRH, subh = lane / LPRH, half = subh / PPI, pi = subh % PPI;
  const int o0 = (wg * W + wv) * OPW;  // this wave's first SwiGLU output
  uint32_t wu[US][KWH];
  float au[US];
#pragma unroll
  for (int u = 0; u < US; ++u) {
    int ug_i = o0 + u * PPI + pi;
    ug_i = ug_i < TK * I ? ug_i : TK * I - 1;
    const int s = ug_i / I, j = ug_i % I;
    const int64_t e = clamp_id(slot_expert<PER == 1 && PPI == 1>(rank, s, slot_tbl), n_exp);
    const int64_t row = e * (2 * I) + j + half * I;
    load_words_v<KWH>(ug + row * NWH + klh * KWH, wu[u]);
    au[u] = ld_t<ADT>(ug_alpha, row);
  }
  const int kld = lane % LPRI, subd = lane / LPRI;
  const int rbase = wg * RPB;
  uint32_t wd[SPW][UD][KWI];
  float ad[SPW][UD];
#pragma unroll
  for (int q = 0; q < SPW; ++q) {
    const int js = wv + W * q;
    const int jj = js < TK ? js : 0;  // idle waves (TK < waves) read slot 0 and add nothing
    const int64_t e = clamp_id(slot_expert<PER == 1>(rank, jj, slot_tbl), n_exp);
#pragma unroll
    for (int u = 0; u < UD; ++u) {
      int r = rbase + u * RPID + subd;
      r = r < H ? r : H - 1;
      load_words_v<KWI>(dn + (e * H + r) * NWI + kld * KWI, wd[q][u]);
      ad[q][u] = ld_t<ADT>(dn_alpha, e * H + r);
    }
  }
  // Next projection (optional): this workgroup's rows, issued after the
  // expert loads so that waiting for those never waits for these.  Lanes
  // split a row as the standalone GEMV does (LPRH lanes of KWH words), RPIH
  // rows per wave pass, NXP passes.
  constexpr int NXP = W == 4 ? 2 : 1;
  const int nx_rq = nx_w ? (nx_rows + G - 1) / G : 0;
  uint32_t nxw[NXP][KWH];
  uint32_t nxa_raw[NXP] = {};  // converted where used (ld_raw)
  if (nx_w) {
#pragma unroll
    for (int p = 0; p < NXP; ++p) {
      int r = wg * nx_rq + p * W * RPIH + wv * RPIH + subh;
      r = r < nx_rows ? r : nx_rows - 1;
      load_words_v<KWH>(nx_w + static_cast<int64_t>(r) * NWH + klh * KWH, nxw[p]);
      nxa_raw[p] = ld_raw<ADT>(nx_alpha, r);
    }
  }
  MA_ISSUE_FENCE();

  // routing weights, while the expert weights are in flight (read after the
  // barrier below): the softmax over all E logits with the max-subtracted
  // exp, then each chosen expert's probability over their sum + 1e-20 in slot
  // order
  if (wv == 0) {
    int mk = INT_MIN;
#pragma unroll
    for (int i = 0; i < PER; ++i) mk = max(mk, float_order_key(lg[i]));
    const float m = float_from_order_key(wave_max_ui(mk));
    float ex[PER], sum = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      ex[i] = lane + 64 * i < n_exp ? expf(lg[i] - m) : 0.f;
      sum += ex[i];
    }
    const float inv_sum = 1.0f / wave_sum_u(sum);
    float prob = 0.f;  // lane s < TK: the probability of the expert in slot s
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const float v = __shfl(ex[i] * inv_sum, my_e & 63, 64);
      if ((my_e >> 6) == i) prob = v;
    }
    float sel = 0.f;
#pragma unroll
    for (int s = 0; s < TK; ++s) sel += lane_bcast(prob, s);
    const float w = prob * (1.0f / (sel + 1e-20f));
    if (lane < TK) {
      s_wts[lane] = w;
      if (wg == 0) wts_out[lane] = w;
    }
  }

  // SwiGLU outputs of this wave
  {
    XSlice<KWH> xsl;
    slice_from_lds<KWH>(xs, cw, klh, xsl);
    const ExpandConsts kc;
    // output t = u * PPI + pi of this wave: its up row sums in lane group pi,
    // its gate row in group PPI + pi; lane t gathers both, then one SwiGLU
    // evaluation and one store for all of the wave's outputs
    float up_t = 0.f, gate_t = 0.f;
#pragma unroll
    for (int u = 0; u < US; ++u) {
      const float v = group_sum_last<LPRH>(slice_dot<KWH>(wu[u], xsl, kc) * au[u]);
#pragma unroll
      for (int q = 0; q < PPI; ++q) {
        const float up = lane_bcast(v, q * LPRH + LPRH - 1);
        const float gt = lane_bcast(v, (PPI + q) * LPRH + LPRH - 1);
        if (lane == u * PPI + q) {
          up_t = up;
          gate_t = gt;
        }
      }
    }
    const int ug_i = o0 + lane;
    if (lane < OPW && ug_i < TK * I) st_coh16(&hbuf[ug_i], f32_to_bf16(swiglu_act(up_t, gate_t)));
  }
  __builtin_amdgcn_s_waitcnt(0);  // this workgroup's h stores have completed
  __syncthreads();
  // ---- 4. barrier (all of h out), stage h, finish this workgroup's rows of y
  if (wv == 0) timed_out = grid_barrier_flags(ws + kLine * kSubB, flags, f0, G, wg, lane, t0) || timed_out;
  __syncthreads();
  {
    constexpr int HIT = (TK * NWI + NTH - 1) / NTH;  // h words per thread, all loads issued first
    const CoherentBuf hcb(hbuf, TK * I * 2);
    uint64_t d[HIT][4];
#pragma unroll
    for (int it = 0; it < HIT; ++it) {
      const int wi = tid + NTH * it;
      const int wc = wi < TK * NWI ? wi : TK * NWI - 1;
      const uint32_t off = static_cast<uint32_t>(((wc / NWI) * I + (wc % NWI) * 16) * 2);
      const uint4 q0 = hcb.ld4u(off), q1 = hcb.ld4u(off + 16);
      d[it][0] = (static_cast<uint64_t>(q0.y) << 32) | q0.x;
      d[it][1] = (static_cast<uint64_t>(q0.w) << 32) | q0.z;
      d[it][2] = (static_cast<uint64_t>(q1.y) << 32) | q1.x;
      d[it][3] = (static_cast<uint64_t>(q1.w) << 32) | q1.z;
    }
#pragma unroll
    for (int it = 0; it < HIT; ++it) {
      const int wi = tid + NTH * it;
      if (wi < TK * NWI) {
        const int s = wi / NWI, w = wi % NWI;
        float vv[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t lo = static_cast<uint32_t>(d[it][q]), hi = static_cast<uint32_t>(d[it][q] >> 32);
          vv[4 * q] = __uint_as_float(lo << 16);
          vv[4 * q + 1] = __uint_as_float(lo & 0xffff0000u);
          vv[4 * q + 2] = __uint_as_float(hi << 16);
          vv[4 * q + 3] = __uint_as_float(hi & 0xffff0000u);
        }
        uint32_t pr[8];
        hc[s][w] = prep_word_pairs(vv, pr);
#pragma unroll
        for (int j = 0; j < 8; ++j) hs[s][w][j] = pr[j];
      }
    }
  }
  __syncthreads();

  // down rows + weighted combine + residual
  {
    const ExpandConsts kc;
    float acc[UD];
#pragma unroll
    for (int u = 0; u < UD; ++u) acc[u] = 0.f;
#pragma unroll
    for (int q = 0; q < SPW; ++q) {
      const int js = wv + W * q;
      const int jj = js < TK ? js : 0;
      const float wjq = js < TK ? s_wts[jj] : 0.f;  // idle waves (TK < waves) add nothing
      XSlice<KWI> hsl;
      slice_from_lds<KWI>(hs[jj], hc[jj], kld, hsl);
#pragma unroll
      for (int u = 0; u < UD; ++u) {
        // each slot's down output is rounded to bf16 before the weighted sum,
        // as the reference's ternary_expert_gemv -> moe_reduce_add chain stores it
        const float eo = group_sum<LPRI>(slice_dot<KWI>(wd[q][u], hsl, kc) * ad[q][u]);
        acc[u] += wjq * bf16_to_f32(f32_to_bf16(eo));
      }
    }
#pragma unroll
    for (int u = 0; u < UD; ++u)
      if (kld == 0) part[wv][u * RPID + subd] = acc[u];
  }
  __syncthreads();
  if (tid < RPB && ro < H) {
    float v = xb ? bf16_to_f32(f32_to_bf16(__uint_as_float(ra << 16) + __uint_as_float(rb << 16)))
                 : residual ? __uint_as_float(ra << 16) : 0.f;
#pragma unroll
    for (int ww = 0; ww < W; ++ww) v += part[ww][tid];
    if (nx_w)
      st_coh16(&y[ro], f32_to_bf16(v));  // read back by every workgroup below
    else
      y[ro] = f32_to_bf16(v);
  }

  // ---- 5. next projection (optional), once every workgroup's rows of y are out
  float nxa[NXP];
#pragma unroll
  for (int p = 0; p < NXP; ++p) {
    uint32_t u = nxa_raw[p];
    asm volatile("" : "+v"(u));  // keeps the conversion here, not next to the load
    nxa[p] = from_raw<ADT>(u);
  }
  if (nx_w)
    timed_out = next_projection<KWH, LPRH, W, NXP>(y, nx_rms, nx_eps, nx_rows, nx_rq, nx_out, nxw, nxa, ws,
                                                   f0 + 1u, G, wg, tid, lane, wv, t0) ||
                timed_out;
  if (__ballot(timed_out) && lane == 0) st_coh32(&ws[2], 1u);
}

}  // namespace ma



using namespace ma;

namespace {

// Supported (hidden, intermediate, top_k) shapes and their grid (at least
// kBarGroups workgroups, and at least one per expert).
struct FusedShape {
  int hidden, inter, top_k, grid, waves;
};
// (2048, 768, 8): 8 waves, SwiGLU 24 outputs and down 8 rows per workgroup -> 256 groups.
// (2048, 512, 8): Maple-Preview (E = 256): 8 waves, SwiGLU 16 outputs and
//                 down 8 rows per workgroup -> 256 groups (one per expert).
// (256, 128, 2): 4 waves, SwiGLU 16 outputs, down 8 rows per workgroup -> 32 groups.
constexpr FusedShape kShapes[] = {{2048, 768, 8, 256, 8}, {2048, 512, 8, 256, 8}, {256, 128, 2, 32, 4}};
static_assert(kShapes[0].grid >= kBarGroups && kShapes[1].grid >= kBarGroups &&
                  kShapes[2].grid >= kBarGroups, "barrier groups");

const FusedShape* find_shape(int64_t hidden, int64_t inter, int64_t top_k) {
  for (const auto& s : kShapes)
    if (s.hidden == hidden && s.inter == inter && s.top_k == top_k) return &s;
  return nullptr;
}

size_t ws_bytes(int64_t, int, int64_t inter, int64_t top_k) {
  // the XCD form's layout lies past the grid form's (either may run on it)
  return top_k == 8 && inter <= 768 ? kXWsBytes : kMoeWsHeader + static_cast<size_t>(top_k * inter) * 2;
}

// The kernel instantiation a call launches (PER = 1 up to 64 experts, else 4).
template <int ADT>
const void* fused_kernel_t(int64_t hidden, int64_t inter, int64_t n_experts) {
  const bool p1 = n_experts <= 64;
  if (hidden == 2048 && inter == 768)
    return p1 ? reinterpret_cast<const void*>(&k_moe_fused<4, 32, 3, 3, 16, 2, 8, 1, 8, ADT>)
              : reinterpret_cast<const void*>(&k_moe_fused<4, 32, 3, 3, 16, 2, 8, 4, 8, ADT>);
  if (hidden == 2048)
    return p1 ? reinterpret_cast<const void*>(&k_moe_fused<4, 32, 2, 2, 16, 2, 8, 1, 8, ADT>)
              : reinterpret_cast<const void*>(&k_moe_fused<4, 32, 2, 2, 16, 2, 8, 4, 8, ADT>);
  return reinterpret_cast<const void*>(&k_moe_fused<1, 16, 2, 1, 8, 1, 2, 1, 4, ADT>);
}
const void* fused_kernel(int64_t hidden, int64_t inter, int64_t n_experts, int alpha_dtype) {
  return alpha_dtype == MA_F32 ? fused_kernel_t<MA_F32>(hidden, inter, n_experts)
                               : fused_kernel_t<MA_BF16>(hidden, inter, n_experts);
}

}  // namespace

// Whether every workgroup of the one-launch layer fits on the current device
// at once (its grid barrier needs that): *needed = the grid, *capacity =
// compute units x occupancy.  MA_EVALUE if the shape is not built.
extern "C" int ma_moe_fused_resident(int64_t n_experts, int64_t hidden, int64_t inter,
                                     int64_t top_k, int64_t* needed, int64_t* capacity) {
  const FusedShape* s = find_shape(hidden, inter, top_k);
  if (!s || !needed || !capacity) return fail(MA_EVALUE, "moe_fused_resident: shape not built");
  *needed = s->grid;
  return resident_capacity(fused_kernel(hidden, inter, n_experts, MA_BF16), 64 * s->waves, capacity);
}

extern "C" size_t ma_moe_fused_workspace_bytes(int64_t n_experts, int64_t hidden, int64_t inter,
                                               int64_t top_k) {
  const FusedShape* s = find_shape(hidden, inter, top_k);
  if (!s || n_experts < 1) return 0;
  return ws_bytes(n_experts, s->grid, inter, top_k);
}

static int moe_fused_impl(const void* x, const void* x_add, const void* norm_weight, int norm_dtype, float eps,
                          const void* residual, const void* gate_weight, const float* router_bias,
                          int64_t n_experts, int64_t hidden, int64_t inter, int64_t top_k, const uint32_t* up_gate,
                          const void* up_gate_alpha, const uint32_t* down, const void* down_alpha, int alpha_dtype,
                          void* y, int32_t* topk_ids, float* topk_weight, void* workspace, size_t workspace_bytes,
                          const uint32_t* next_w, const void* next_alpha, int next_alpha_dtype,
                          const float* next_rms, float next_eps, int64_t next_rows, void* next_out, void* stream,
                          const void* attn, const uint32_t* o_w, const void* o_alpha, const void* prefetch,
                          int64_t prefetch_bytes) {
  const FusedShape* s = find_shape(hidden, inter, top_k);
  if (!s)
    return fail(MA_EVALUE, "moe_fused: shape (hidden %lld, inter %lld, top_k %lld) not built",
                static_cast<long long>(hidden), static_cast<long long>(inter),
                static_cast<long long>(top_k));
  if (n_experts < top_k || n_experts > 256 || n_experts > static_cast<int64_t>(s->grid))
    return fail(MA_EVALUE, "moe_fused: %lld experts unsupported", static_cast<long long>(n_experts));
  if ((x_add || o_w) && !norm_weight) return fail(MA_EVALUE, "moe_fused: add without norm weight");
  if (alpha_dtype != MA_F32 && alpha_dtype != MA_BF16)
    return fail(MA_ETYPE, "moe_fused: row_alpha dtype %d (float32 or bfloat16)", alpha_dtype);
  if (norm_weight && norm_dtype != MA_F32 && norm_dtype != MA_BF16)
    return fail(MA_ETYPE, "moe_fused: norm weight dtype %d", norm_dtype);
  if (!workspace || workspace_bytes < ws_bytes(n_experts, s->grid, inter, top_k))
    return fail(MA_EVALUE, "moe_fused: workspace too small");
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (!a16(x) || (x_add && (!a16(x_add) || !a16(norm_weight))) || !a16(gate_weight) ||
      !a16(up_gate) || !a16(workspace))
    return fail(MA_EVALUE, "moe_fused: x, x_add, norm weight, weights and workspace must be 16-byte aligned");
  if (next_w) {
    // rows per workgroup pass: waves x rows per wave (2 at hidden 2048, 4 at 256), passes 8 / waves
    const int64_t max_rows = static_cast<int64_t>(s->grid) * 8 * (hidden == 2048 ? 2 : 4);
    if (!next_alpha || !next_rms || !next_out || next_rows < 1 || next_rows > max_rows)
      return fail(MA_EVALUE, "moe_fused: next projection needs alpha, rms weight, output and 1..%lld rows",
                  static_cast<long long>(max_rows));
    if (next_alpha_dtype != alpha_dtype)
      return fail(MA_ETYPE, "moe_fused: next projection alpha dtype %d differs from the experts' %d",
                  next_alpha_dtype, alpha_dtype);
    if (!a16(next_w) || !a16(next_rms) || !a16(y))
      return fail(MA_EVALUE, "moe_fused: next projection weights, rms weight and y must be 16-byte aligned");
  }
  int64_t capacity = 0;
  if (int rc = resident_capacity(fused_kernel(hidden, inter, n_experts, alpha_dtype), 64 * s->waves, &capacity))
    return rc;
  if (capacity < s->grid)
    return fail(MA_ERUNTIME, "moe_fused: its %d workgroups wait on each other but the device holds %lld at once",
                s->grid, static_cast<long long>(capacity));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (o_w && (!attn || !o_alpha || !a16(attn) || !a16(o_w)))
    return fail(MA_EVALUE, "moe_fused_o: the attention output and O weights (16-byte aligned) and row scales are needed");
  if (moe_xcd_supported(n_experts, hidden, inter, top_k, st))
    return moe_xcd_launch(x, x_add, norm_weight, norm_dtype, eps, residual, gate_weight, router_bias, n_experts,
                          hidden, inter, up_gate, up_gate_alpha, down, down_alpha, alpha_dtype, y, topk_ids,
                          topk_weight, workspace, next_w, next_alpha, next_rms, next_eps, next_rows, next_out, attn,
                          o_w, o_alpha, prefetch, prefetch_bytes, st);
  if (o_w)
    return fail(MA_EVALUE, "moe_fused_o: the O projection in the launch needs the XCD-split form (ma_moe_fused_form)");
#define MA_FUSED_ARGS                                                                            \
  static_cast<const uint16_t*>(x), static_cast<uint32_t*>(workspace),                           \
      static_cast<const uint16_t*>(gate_weight), static_cast<const uint16_t*>(residual),         \
      static_cast<const uint16_t*>(x_add), norm_weight, static_cast<int>(n_experts), norm_dtype, \
      eps, router_bias, up_gate, up_gate_alpha, down, down_alpha,                                \
      static_cast<uint16_t*>(y), topk_ids, topk_weight,                                          \
      next_w, next_alpha, next_rms, next_eps, static_cast<int>(next_rows),                        \
      static_cast<uint16_t*>(next_out)
  const dim3 grid(s->grid), block(64 * s->waves);
  const int per = n_experts <= 64 ? 1 : 4;
#define MA_FUSED_LAUNCH(ADT)                                                                      \
  if (hidden == 2048 && inter == 768) {                                                          \
    if (per == 1)                                                                                \
      hipLaunchKernelGGL((k_moe_fused<4, 32, 3, 3, 16, 2, 8, 1, 8, ADT>), grid, block, 0, st, MA_FUSED_ARGS); \
    else                                                                                         \
      hipLaunchKernelGGL((k_moe_fused<4, 32, 3, 3, 16, 2, 8, 4, 8, ADT>), grid, block, 0, st, MA_FUSED_ARGS); \
  } else if (hidden == 2048) {                                                                   \
    if (per == 1)                                                                                \
      hipLaunchKernelGGL((k_moe_fused<4, 32, 2, 2, 16, 2, 8, 1, 8, ADT>), grid, block, 0, st, MA_FUSED_ARGS); \
    else                                                                                         \
      hipLaunchKernelGGL((k_moe_fused<4, 32, 2, 2, 16, 2, 8, 4, 8, ADT>), grid, block, 0, st, MA_FUSED_ARGS); \
  } else {                                                                                       \
    hipLaunchKernelGGL((k_moe_fused<1, 16, 2, 1, 8, 1, 2, 1, 4, ADT>), grid, block, 0, st, MA_FUSED_ARGS); \
  }
  if (alpha_dtype == MA_F32) {
    MA_FUSED_LAUNCH(MA_F32)
  } else {
    MA_FUSED_LAUNCH(MA_BF16)
  }
#undef MA_FUSED_LAUNCH
#undef MA_FUSED_ARGS
  return check_launch("moe_fused");
}

extern "C" int ma_moe_fused(const void* x, const void* x_add, const void* norm_weight,
                            int norm_dtype, float eps, const void* residual,
                            const void* gate_weight, const float* router_bias, int64_t n_experts,
                            int64_t hidden, int64_t inter, int64_t top_k,
                            const uint32_t* up_gate, const void* up_gate_alpha,
                            const uint32_t* down, const void* down_alpha, int alpha_dtype, void* y,
                            int32_t* topk_ids, float* topk_weight, void* workspace,
                            size_t workspace_bytes, const uint32_t* next_w,
                            const void* next_alpha, int next_alpha_dtype, const float* next_rms,
                            float next_eps, int64_t next_rows, void* next_out, const void* prefetch,
                            int64_t prefetch_bytes, void* stream) {
  return moe_fused_impl(x, x_add, norm_weight, norm_dtype, eps, residual, gate_weight, router_bias, n_experts,
                        hidden, inter, top_k, up_gate, up_gate_alpha, down, down_alpha, alpha_dtype, y, topk_ids,
                        topk_weight, workspace, workspace_bytes, next_w, next_alpha, next_alpha_dtype, next_rms,
                        next_eps, next_rows, next_out, stream, nullptr, nullptr, nullptr, prefetch, prefetch_bytes);
}

extern "C" int ma_moe_fused_o(const void* x, const void* attn, const uint32_t* o_w, const void* o_alpha,
                              const void* norm_weight, int norm_dtype, float eps, const void* gate_weight,
                              const float* router_bias, int64_t n_experts, int64_t hidden, int64_t inter,
                              int64_t top_k, const uint32_t* up_gate, const void* up_gate_alpha,
                              const uint32_t* down, const void* down_alpha, int alpha_dtype, void* y,
                              int32_t* topk_ids, float* topk_weight, void* workspace, size_t workspace_bytes,
                              const uint32_t* next_w, const void* next_alpha, int next_alpha_dtype,
                              const float* next_rms, float next_eps, int64_t next_rows, void* next_out,
                              const void* prefetch, int64_t prefetch_bytes, void* stream) {
  if (!o_w) return fail(MA_EVALUE, "moe_fused_o: no O weights");
  return moe_fused_impl(x, nullptr, norm_weight, norm_dtype, eps, nullptr, gate_weight, router_bias, n_experts,
                        hidden, inter, top_k, up_gate, up_gate_alpha, down, down_alpha, alpha_dtype, y, topk_ids,
                        topk_weight, workspace, workspace_bytes, next_w, next_alpha, next_alpha_dtype, next_rms,
                        next_eps, next_rows, next_out, stream, attn, o_w, o_alpha, prefetch, prefetch_bytes);
}

extern "C" int ma_moe_fused_form(int64_t n_experts, int64_t hidden, int64_t inter, int64_t top_k) {
  if (!find_shape(hidden, inter, top_k)) return -1;
  return moe_xcd_supported(n_experts, hidden, inter, top_k, nullptr) ? 1 : 0;
}

extern "C" int ma_moe_fused_timed_out(const void* workspace, int* out, void* stream) {
  // Copies the error words to host memory: *out = 2 if the XCD-split form's
  // layout check aborted a call, else 1 if a wait timed out, else 0 (since
  // the workspace was zeroed); synchronises the stream.
  if (!workspace || !out) return fail(MA_EVALUE, "moe_fused_timed_out: null pointer");
  uint32_t v[3] = {0, 0, 0};  // words 2 (timeout), 3 (unused), 4 (layout)
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (hipMemcpyAsync(v, static_cast<const char*>(workspace) + 8, sizeof(v), hipMemcpyDeviceToHost, st) !=
          hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess)
    return fail(MA_ERUNTIME, "moe_fused_timed_out: copy failed");
  *out = v[2] ? 2 : (v[0] ? 1 : 0);
  return MA_OK;
}
