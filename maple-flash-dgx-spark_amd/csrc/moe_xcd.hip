// One-launch MoE FFN layer for one token, split by XCD (gfx950).
//
// Semantics: those of k_moe_fused (moe_fused.hip), i.e. MapleSparseMoeBlock.
// __call__ at T = 1 (reference src/maple_run/model.py:448-474): router_topk
// (kernels/router.py:39-126), the expert SwiGLU (kernels/ternary_expert.py:
// 240-319, h stored bf16), each slot's down projection rounded to bf16
// (ternary_expert.py:58-122), and the top-k weighted float32 combine in slot
// order with the residual (fused_norm.py:59-96), y stored bf16; optionally the
// add + RMSNorm ahead of it (fused_norm.py:31-56) and the next layer's
// RMS-folded projection after it.
//
// Why a second form.  The GPU has 8 XCDs, each with its own L2, and the
// hardware hands the workgroups of a launch to them in turn (workgroup i runs
// on XCD (i + o) mod 8, so i / 8 numbers the workgroups of one XCD 0..31).  A
// store seen through another XCD has to travel through memory: a round trip
// between workgroups on different XCDs costs ~1.2 us, while a plain store read
// back with an sc1 load by a workgroup of the same XCD (both through that
// XCD's L2) costs ~0.33 us.  With top-8 routing there are as many slots as
// XCDs, so XCD x takes slot x:
//   1. workgroups 0..7 of each XCD compute the 64 router logits (one per
//      wave) and publish them, tagged with the call's number, in the XCD's
//      own region; every workgroup polls its XCD's copy (L2 hits) and ranks
//      the experts (ties to the lower index), so it knows the expert of its
//      slot and issues that expert's SwiGLU and down rows at once;
//   2. workgroup j of XCD x computes outputs [24 j, 24 j + 24) of h_x and
//      publishes them as tagged bf16 words in the XCD's region; each
//      workgroup polls all of h_x there (3 KB from its L2), no barrier;
//   3. it computes rows [64 j, 64 j + 64) of slot x's down projection, rounds
//      each to bf16, scales it by the slot's routing weight and publishes it
//      as a tagged float with a device-coherent store;
//   4. workgroup g polls the 8 slots' values of rows [8 g, 8 g + 8) (one lane
//      each, the only hand-off between XCDs after the routing), adds them to
//      the residual in slot order and stores y;
//   5. with the next layer's projection in the launch, step 4 instead runs on
//      every XCD for all of y (workgroup j of the XCD polls the 8 slots'
//      values of rows [64 j, 64 j + 64)), so that each XCD hands its own copy
//      of y to its workgroups through its L2 (tagged words, no grid barrier)
//      and each workgroup then computes its rows of the projection.
// Tags: each workgroup keeps its own count of calls on the workspace (written
// only by itself at the end of a call); every call runs every workgroup, so
// all counts agree and this call's tag is the count + 1.  Nothing needs
// clearing between calls.  Every wait is bounded (200 us after the launch's
// start, below); on timeout the workspace error word is set and the kernel
// finishes with wrong values instead of hanging.
// Layout check: the kernel is right exactly when every XCD runs 32 of the
// workgroups with distinct numbers i / 8, i.e. (by pigeonhole) when each of
// the 256 (XCD, number) slots gets one workgroup.  Each workgroup stores the
// call's tag into its slot once its expert weight loads are issued: a plain
// store into its XCD's L2 (a device-coherent one at entry, acknowledged from
// memory, held the wave's first loads up by 0.15 us per layer: on this GPU a
// wait for a load also waits for every older store).  The waits are bounded
// at 200 us from the launch's start (below); a workgroup that ran out reads
// its own XCD's 32 slots at the end.  If the layout is wrong, some XCD
// misses a number, and the workgroups there that waited for that number's
// data find its slot empty: the sticky layout word is set for the host,
// which then turns the XCD-split forms off on the device
// (ma_xcd_forms_disable).  A healthy call pays one store for it.
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "moe_fused.h"

namespace ma {

constexpr int kXcdWgs = 32;  // workgroups per XCD
// Every wait of this kernel ends 200 us (of the 100 MHz counter) after the
// launch's start at the latest -- a hundred times the longest hand-off of a
// healthy call -- and once one has run out the later ones are skipped, so a
// call whose workgroups cannot meet ends within about 200 us, flagged.
// (MAPLE_AMD_WAIT_BOUND_US sets another bound, for tests.)
constexpr uint64_t kXWaitTicks = 20000;
// Prefetch: 16-byte units per prefetching lane (7 waves x 32 workgroups of
// an XCD x 2 = 28,672 units = 448 KB, more than a router of 64 x 2048 bf16)
constexpr int kPfPerLane = 2;
constexpr int kXHasO = 0x100;  // k_moe_xcd's mode: the O projection in front

// Shapes: H = 16 * KWH * LPRH with LPRH = 32 (one up/gate row pair per
// SwiGLU pass), I = 16 * KWI * LPRI, US SwiGLU outputs and UD down passes
// (64 / LPRI rows each) per wave, 8 waves per workgroup, E <= 64 experts,
// top-8; ADT the row scales' dtype; NX: the instance launched with a next
// projection (nx_w set).
template <int KWH, int US, int KWI, int LPRI, int UD, int ADT, bool NX>
//
// The arguments the first loads need come first (the first 14 dwords arrive
// preloaded in SGPRs); mode = the norm weights' dtype | kXHasO with the O
// projection in front.
__global__ __launch_bounds__(512) void k_moe_xcd(
    const uint16_t* __restrict__ xa, uint32_t* __restrict__ ws, const uint16_t* __restrict__ gate_w,
    const uint16_t* __restrict__ residual, const uint16_t* __restrict__ xb, const void* __restrict__ norm_w,
    int n_exp, int mode, float eps, const float* __restrict__ bias,
    const uint32_t* __restrict__ ug, const void* __restrict__ ug_alpha,
    const uint32_t* __restrict__ dn, const void* __restrict__ dn_alpha,
    uint16_t* __restrict__ y, int32_t* __restrict__ ids_out, float* __restrict__ wts_out,
    const uint32_t* __restrict__ nx_w, const void* __restrict__ nx_alpha,
    const float* __restrict__ nx_rms, float nx_eps, int nx_rows,
    uint16_t* __restrict__ nx_out, const uint16_t* __restrict__ attn, const uint32_t* __restrict__ o_w,
    const void* __restrict__ o_alpha, const uint4* __restrict__ pf, int pf_units, uint64_t wait_bound) {
  constexpr int TK = kXcds;  // one slot per XCD
  constexpr int W = 8;
  constexpr int LPRH = 32;
  constexpr int NWH = KWH * LPRH, H = 16 * NWH;
  constexpr int NWI = KWI * LPRI, I = 16 * NWI;
  constexpr int XPL = NWH / 64;       // words of x per lane of a router wave
  constexpr int RPID = 64 / LPRI;     // down rows per wave pass
  constexpr int RPW = RPID * UD;      // down rows per wave
  constexpr int FR = H / (kXcds * kXcdWgs);  // y rows finished per workgroup
  constexpr int RPIH = 64 / LPRH;
  static_assert(NWH % 64 == 0, "x layout");
  static_assert(W * US * kXcdWgs == I, "h outputs per XCD");
  static_assert(W * RPW * kXcdWgs == H, "down rows per XCD");
  static_assert(FR * TK == 64, "combine: one slot value per lane");
  static_assert(NWI <= 64 && 4 * I + 512 <= static_cast<int>(kXRegion), "h region");

  __shared__ __align__(16) uint32_t xs[NWH][8];
  __shared__ float cw[NWH];
  __shared__ __align__(16) uint32_t hs[NWI][8];
  __shared__ float hc[NWI];
  __shared__ uint64_t s_key[64];
  __shared__ uint32_t s_cnt[W][64];
  __shared__ __align__(16) uint32_t xbf[NWH][8];  // x in bf16 pairs, for the router waves
  __shared__ float s_red[W];
  __shared__ float s_w;
  __shared__ float s_pv[TK][64];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = gridDim.x, wg = blockIdx.x;
  const int xcd = xcc_id();
  const int lw = wg >> 3;  // this workgroup's number among its XCD's
  char* const wsb = reinterpret_cast<char*>(ws);
  uint32_t* const calls = reinterpret_cast<uint32_t*>(wsb + kXEpochOff) + 32 * wg;
  uint64_t* const xlog = reinterpret_cast<uint64_t*>(wsb + kXRegionOff + xcd * kXRegion);
  uint32_t* const xh = reinterpret_cast<uint32_t*>(wsb + kXRegionOff + xcd * kXRegion + 512);
  uint64_t* const part = reinterpret_cast<uint64_t*>(wsb + kXPartOff);
  uint64_t* const yx = reinterpret_cast<uint64_t*>(wsb + kXYOff + xcd * kXYRegion);
  uint64_t* const ox = reinterpret_cast<uint64_t*>(wsb + kXOOff + xcd * kXYRegion);
  // This call's tag is the count + 1, formed where it is first needed (after
  // x is staged): formed here, it made every wave wait for this load before
  // requesting x.
  uint32_t tag_raw = ld_coh32(calls);
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  bool timed_out = false;
  // the layout check: this call's tag into the slot of (this XCD, this
  // workgroup's number on it), one device-coherent store, nothing waited for
  uint32_t* const present = reinterpret_cast<uint32_t*>(wsb + kXPresentOff);
#ifdef MA_PHASE_STAMPS
  uint32_t* const stamps = reinterpret_cast<uint32_t*>(wsb + kXStampOff) + kXStampWords * wg;
  if (wv == 0) {
    MA_XSTAMP(0);  // start
    if (lane == 0) stamps[15] = static_cast<uint32_t>(xcd);
  }
#endif

  // The residual of the y rows this workgroup finishes (wave 0): rows
  // 64 lw + lane with a next projection (every XCD combines all of y), else
  // rows wg * FR + lane, lanes < FR.
  const int ro = NX ? 64 * lw + lane : wg * FR + (lane < FR ? lane : 0);
  const int norm_dt = mode & 0xff;
  const bool has_o = (mode & kXHasO) != 0;
  const bool addp = xb || has_o;  // x + (add or the O projection), then RMSNorm
  const uint16_t* const res_a = addp ? xa : (residual ? residual : xa);
  const uint16_t* const res_b = xb ? xb : xa;
  const uint32_t ra = res_a[ro];
  uint32_t rb = has_o ? 0u : res_b[ro];  // with the O projection: from the XCD's copy of o, below

  // ---- 1. x (optionally add + RMSNorm) staged once per workgroup: thread
  // t < NWH takes word t, in bf16 (for the router waves) and as x' pairs (for
  // the SwiGLU rows); then wave w of workgroup j < 8 of an XCD takes router row
  // 8 j + w (loaded at the start) against x from LDS, lane l words l + 64 i
  const int re = 8 * lw + wv;
  const bool router_wave = lw < 8 && re < n_exp;  // wave-uniform
  uint4 gr[XPL][2];
  if (router_wave) {
#pragma unroll
    for (int i = 0; i < XPL; ++i) {
      const uint4* gp = reinterpret_cast<const uint4*>(gate_w + static_cast<int64_t>(re) * H + (lane + 64 * i) * 16);
      gr[i][0] = gp[0];
      gr[i][1] = gp[1];
    }
  }
  // x, its addend and the norm weights requested now, ahead of everything
  // that needs an argument read from memory (the word of x of thread t <
  // NWH; the addend and the weights only with an add in front, the weights
  // from an address that their dtype selects, not from a dtype branch)
  static_assert(NWH <= 512, "one word of x per thread");
  const int wc = tid < NWH ? tid : NWH - 1;
  const uint4 xa0 = reinterpret_cast<const uint4*>(xa + wc * 16)[0];
  const uint4 xa1 = reinterpret_cast<const uint4*>(xa + wc * 16)[1];
  uint4 xb0 = make_uint4(0u, 0u, 0u, 0u), xb1 = xb0, nw0 = xb0, nw1 = xb0, nw2 = xb0, nw3 = xb0;
  const bool nf32 = norm_dt == MA_F32;
  if (xb) {
    xb0 = reinterpret_cast<const uint4*>(xb + wc * 16)[0];
    xb1 = reinterpret_cast<const uint4*>(xb + wc * 16)[1];
  }
  if (addp) {  // f32: 4 x 16 bytes per word of x; bf16: 2 x 16 (loaded twice)
    const uint4* const np = reinterpret_cast<const uint4*>(static_cast<const char*>(norm_w) + wc * (nf32 ? 64 : 32));
    nw0 = np[0];
    nw1 = np[1];
    nw2 = np[nf32 ? 2 : 0];
    nw3 = np[nf32 ? 3 : 1];
  }
  // The other arguments the layer reads before its expert loads, read at
  // once with one wait (left to itself, the compiler read each where first
  // used, a wait each).
  asm volatile("" ::"s"(eps), "s"(bias), "s"(ug), "s"(ug_alpha), "s"(dn), "s"(dn_alpha), "s"(nx_w),
               "s"(pf), "s"(pf_units), "s"(wait_bound)
               : "memory");

  // ---- 0. the O projection (optional): o = ternary_gemv(attn, o_w, o_alpha)
  // with the standalone fast GEMV's per-lane arithmetic (so the same bits);
  // every XCD computes all of o (wave w of workgroup j: rows 64 j + 8 w ..
  // + 8, two per pass) and hands it to its workgroups through its L2, two
  // bf16 values per tagged word, as y below.
  __shared__ __align__(16) uint32_t os[NWH][8];
  __shared__ float oc[NWH];
  if (has_o) {
    const int okl = lane % LPRH, osub = lane / LPRH;
    constexpr int OP = 64 / (W * RPIH);  // passes of RPIH rows per wave
    uint32_t wo[OP][KWH];
    float ao[OP];
#pragma unroll
    for (int p = 0; p < OP; ++p) {
      const int r = 64 * lw + (64 / W) * wv + RPIH * p + osub;
      load_words_v<KWH>(o_w + static_cast<int64_t>(r) * NWH + okl * KWH, wo[p]);
      ao[p] = ld_t<ADT>(o_alpha, r);
    }
    stage_row(attn, NWH, os, oc);
    __syncthreads();
    XSlice<KWH> osl;
    slice_from_lds<KWH>(os, oc, okl, osl);
    const ExpandConsts kc;
#pragma unroll
    for (int p = 0; p < OP; ++p) {
      const float d = group_sum<LPRH>(slice_dot<KWH>(wo[p], osl, kc) * ao[p]);
      const uint32_t bits = f32_to_bf16(d);
      const uint32_t odd = __shfl(bits, LPRH, 64);  // row r + 1, held by lane LPRH
      const int r = 64 * lw + (64 / W) * wv + RPIH * p;
      if (lane == 0) st_l2_64(&ox[r >> 1], (static_cast<uint64_t>(tag_raw + 1u) << 32) | bits | (odd << 16));
    }
  }
  {
    float v[16];
    {
      const uint32_t u[8] = {xa0.x, xa0.y, xa0.z, xa0.w, xa1.x, xa1.y, xa1.z, xa1.w};
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        v[2 * q] = __uint_as_float(u[q] << 16);
        v[2 * q + 1] = __uint_as_float(u[q] & 0xffff0000u);
      }
    }
    if (addp) {
      float nw[16];
      uint32_t ub[8];
      if (has_o) {  // word wc of o: tagged words 8 wc .. + 8 of the XCD's copy
        const CoherentBuf oq(ox, NWH * 8 * 8);
        uint4 q[4];
        for (;;) {
          MA_POLL_RELOAD();
#pragma unroll
          for (int i = 0; i < 4; ++i) q[i] = oq.ld4u(static_cast<uint32_t>((8 * wc + 2 * i) * 8));
          uint32_t bad = 0;
#pragma unroll
          for (int i = 0; i < 4; ++i) bad |= (q[i].y ^ (tag_raw + 1u)) | (q[i].w ^ (tag_raw + 1u));
          if (__all(bad == 0) || timed_out) break;
          __builtin_amdgcn_s_sleep(1);
          timed_out = (__builtin_amdgcn_s_memrealtime() - t0) > wait_bound;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          ub[2 * i] = q[i].x;
          ub[2 * i + 1] = q[i].z;
        }
      } else {
        ub[0] = xb0.x, ub[1] = xb0.y, ub[2] = xb0.z, ub[3] = xb0.w;
        ub[4] = xb1.x, ub[5] = xb1.y, ub[6] = xb1.z, ub[7] = xb1.w;
      }
      {
        const uint32_t un[16] = {nw0.x, nw0.y, nw0.z, nw0.w, nw1.x, nw1.y, nw1.z, nw1.w,
                                 nw2.x, nw2.y, nw2.z, nw2.w, nw3.x, nw3.y, nw3.z, nw3.w};
#pragma unroll
        for (int q = 0; q < 16; ++q)
          nw[q] = nf32 ? __uint_as_float(un[q])
                       : (q & 1 ? __uint_as_float(un[q >> 1] & 0xffff0000u) : __uint_as_float(un[q >> 1] << 16));
      }
      float ss = 0.f;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        v[2 * q] += __uint_as_float(ub[q] << 16);
        v[2 * q + 1] += __uint_as_float(ub[q] & 0xffff0000u);
      }
      if (tid < NWH) {
#pragma unroll
        for (int q = 0; q < 16; ++q) ss += v[q] * v[q];
      }
      ss = group_sum<64>(ss);
      if (lane == 0) s_red[wv] = ss;
      __syncthreads();
      float ssum = s_red[0];
#pragma unroll
      for (int w = 1; w < W; ++w) ssum += s_red[w];
      const float rstd = rsqrtf(ssum / static_cast<float>(H) + eps);
#pragma unroll
      for (int q = 0; q < 16; ++q) v[q] = bf16_to_f32(f32_to_bf16(v[q] * rstd * nw[q]));
    }
    if (tid < NWH) {
      uint32_t pr[8];
      cw[tid] = prep_word_pairs(v, pr);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        xs[tid][j] = pr[j];
        xbf[tid][j] = pack_bf16x2(v[2 * j], v[2 * j + 1]);
      }
    }
  }
  __syncthreads();
  asm volatile("" : "+v"(tag_raw));  // (keeps the + 1 below from moving up)
  const uint32_t tag = tag_raw + 1u;
  const uint32_t tag16 = tag & 0xffffu;
  if (router_wave) {
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < XPL; ++i) {
      const uint4 x0 = *reinterpret_cast<const uint4*>(&xbf[lane + 64 * i][0]);
      const uint4 x1 = *reinterpret_cast<const uint4*>(&xbf[lane + 64 * i][4]);
      const uint32_t xw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      const uint32_t gw[8] = {gr[i][0].x, gr[i][0].y, gr[i][0].z, gr[i][0].w,
                              gr[i][1].x, gr[i][1].y, gr[i][1].z, gr[i][1].w};
#pragma unroll
      for (int j = 0; j < 8; ++j) dot = dot2(xw[j], gw[j], dot);
    }
    const float l = group_sum<64>(dot) + (bias ? bias[re] : 0.f);
    if (lane == 0) st_l2_64(&xlog[re], (static_cast<uint64_t>(tag) << 32) | __float_as_uint(l));
    if (wv == 0) MA_XSTAMP(1);  // router logit out (workgroups 0..7 of an XCD)
  }

  // ---- 2. ranks: wave 0 polls its XCD's copy of the logits (lane e, expert
  // e) and puts one 64-bit key per expert in LDS (the logit's order bits over
  // the complemented index: keys differ, ties go to the lower index); wave w
  // counts, for every expert, the keys [8 w, 8 w + 8) above its own; the
  // counts sum to the expert's rank, and slot s is the expert of rank s.
  float lg = -INFINITY;
  int key = INT_MIN + 1;  // experts past E rank below every logit
  if (wv == 0) {
    bool have = lane >= n_exp;
    for (;;) {
      if (!have) {
        const uint64_t q = ld_coh64(&xlog[lane]);
        have = static_cast<uint32_t>(q >> 32) == tag;
        lg = __uint_as_float(static_cast<uint32_t>(q));
      }
      if (__all(have) || timed_out) break;
      __builtin_amdgcn_s_sleep(1);
      timed_out = (__builtin_amdgcn_s_memrealtime() - t0) > wait_bound;
    }
    MA_XSTAMP(2);  // every logit of the XCD seen
    if (lane < n_exp) key = float_order_key(lg);
    s_key[lane] = (static_cast<uint64_t>(static_cast<uint32_t>(key) ^ 0x80000000u) << 32) |
                  static_cast<uint32_t>(~lane);
  }
  __syncthreads();
  uint32_t rank = 0;
  {
    const uint64_t mine = s_key[lane];
#pragma unroll
    for (int j = 0; j < 64 / W; ++j) rank += s_key[(64 / W) * wv + j] > mine ? 1u : 0u;
    s_cnt[wv][lane] = rank;
    __syncthreads();
    rank = 0;
#pragma unroll
    for (int w = 0; w < W; ++w) rank += s_cnt[w][lane];
  }
  // this XCD's expert (clamped: only a timed-out wait can leave an absent
  // expert among the first 8 ranks)
  const int64_t ex = clamp_id(__builtin_ctzll(__ballot(rank == static_cast<uint32_t>(xcd))), n_exp);
  if (wv == 0) MA_XSTAMP(3);  // ranked

  // ---- 3. weights of slot xcd: this wave's SwiGLU rows (outputs o0 .. o0 +
  // US, lanes 0..31 the up row and 32..63 the gate row, each lane 16 KWH
  // contiguous bytes), then its down rows (rows r0 .. r0 + RPW, LPRI lanes per
  // row), all issued before any arithmetic
  const int klh = lane % LPRH, half = lane / LPRH;
  const int o0 = (lw * W + wv) * US;
  uint32_t wu[US][KWH];
  float au[US];
#pragma unroll
  for (int u = 0; u < US; ++u) {
    const int64_t row = ex * (2 * I) + o0 + u + half * I;
    load_words_v<KWH>(ug + row * NWH + klh * KWH, wu[u]);
    au[u] = ld_t<ADT>(ug_alpha, row);
  }
  // Next projection (nx_w): this workgroup's rows, as in k_moe_fused.  In
  // the instance built for it (NX) the loads are not behind a branch: past a
  // branch holding loads, a wait for the loads issued before it also waits
  // for these (the counts of the two paths merge).  (The instance without
  // keeps the run-time branches: the same code without them measured 0.09 us
  // slower per layer.)
  constexpr int NXP = 1;
  const int nx_rq = nx_w ? (nx_rows + G - 1) / G : 0;
  uint32_t nxw[NXP][KWH];
  uint32_t nxa_raw[NXP] = {};  // converted where used (ld_raw)
  // and its RMS weights (NX), loaded now: loaded after y, they would hold up
  // the reads of y (memory counters complete in issue order)
  NxRms<(NWH * 2 + 64 * W - 1) / (64 * W)> nxr{};
  if constexpr (NX) nxr = load_nx_rms<NWH, 64 * W>(nx_rms, tid);
  if (NX || nx_w) {
    const int subh = lane / LPRH;
#pragma unroll
    for (int p = 0; p < NXP; ++p) {
      int r = wg * nx_rq + p * W * RPIH + wv * RPIH + subh;
      r = r < nx_rows ? r : nx_rows - 1;
      load_words_v<KWH>(nx_w + static_cast<int64_t>(r) * NWH + klh * KWH, nxw[p]);
      nxa_raw[p] = ld_raw<ADT>(nx_alpha, r);
    }
  }
  MA_ISSUE_FENCE();
  if (wv == 0) MA_XSTAMP(4);  // weight loads issued
  if (tid == 0) st_l2_32(present + xcd * kXcdWgs + (lw & (kXcdWgs - 1)), tag);

  // routing weights while the loads are in flight (wave 0): the softmax over
  // all E logits with the max-subtracted exp, then p / (sum of the selected p
  // in slot order + 1e-20)
  if (wv == 0) {
    const float m = float_from_order_key(wave_max_ui(key));
    const float e = lane < n_exp ? expf(lg - m) : 0.f;
    const float p = e * (1.0f / wave_sum_u(e));
    float sel = 0.f;
#pragma unroll
    for (int s = 0; s < TK; ++s) sel += lane_bcast(p, __builtin_ctzll(__ballot(rank == static_cast<uint32_t>(s))));
    const float w = p * (1.0f / (sel + 1e-20f));
    if (lane == ex) s_w = w;
    if (wg == 0 && rank < static_cast<uint32_t>(TK)) {
      ids_out[rank] = lane < n_exp ? lane : n_exp - 1;
      wts_out[rank] = w;
    }
  }

  // This wave's down rows, requested once its SwiGLU rows are in and before
  // their products (requested with them, they held up the SwiGLU rows;
  // after the outputs are published, they arrived ~0.5 us later).
  asm volatile("" ::"v"(au[US - 1]));  // (in-order counters: every SwiGLU row is in)
  const int kld = lane % LPRI, subd = lane / LPRI;
  const int r0 = (lw * W + wv) * RPW;
  uint32_t wd[UD][KWI];
  float ad[UD];
#pragma unroll
  for (int u = 0; u < UD; ++u) {
    const int64_t r = ex * H + r0 + u * RPID + subd;
    load_words_v<KWI>(dn + r * NWI + kld * KWI, wd[u]);
    ad[u] = ld_t<ADT>(dn_alpha, r);
  }

  // SwiGLU outputs o0 .. o0 + US of slot xcd, published in the XCD's region
  {
    XSlice<KWH> xsl;
    slice_from_lds<KWH>(xs, cw, klh, xsl);
    const ExpandConsts kc;
    float up_t = 0.f, gate_t = 0.f;
#pragma unroll
    for (int u = 0; u < US; ++u) {
      const float v = group_sum_last<LPRH>(slice_dot<KWH>(wu[u], xsl, kc) * au[u]);
      const float up = lane_bcast(v, LPRH - 1), gt = lane_bcast(v, 2 * LPRH - 1);
      if (lane == u) {
        up_t = up;
        gate_t = gt;
      }
    }
    if (lane < US) st_l2_32(&xh[o0 + lane], (tag16 << 16) | f32_to_bf16(swiglu_act(up_t, gate_t)));
  }
  if (wv == 0) MA_XSTAMP(5);  // this wave's h outputs published
  // Prefetch (optional): waves 1..7 pull pf_units 16-byte units (the next
  // layer's router rows, say) into this XCD's L2 and the Infinity Cache
  // while they would otherwise wait for h; every XCD reads all of it (each
  // has its own L2).  The values are only held (consumed at the end), so
  // the loads are off every wait of the layer's own data except the last.
  uint4 pfv[kPfPerLane];
  constexpr int kPfLanes = kXcdWgs * (W - 1) * 64;  // lanes of an XCD that prefetch
  const int pfl = (lw * (W - 1) + wv - 1) * 64 + lane;
#pragma unroll
  for (int k = 0; k < kPfPerLane; ++k) {
    const int u = pfl + k * kPfLanes;
    pfv[k] = make_uint4(0u, 0u, 0u, 0u);
    if (pf && wv > 0 && u < pf_units) pfv[k] = pf[u];
  }
  MA_ISSUE_FENCE();

  // ---- 4. h of slot xcd from the XCD's region: thread t < NWI polls the 16
  // values of h word t until all carry this call's tag, then builds its x'
  // pairs
  if (tid < NWI) {
    const CoherentBuf hb(xh, 4 * I);
    uint4 q[4];
    for (;;) {
      MA_POLL_RELOAD();
#pragma unroll
      for (int k = 0; k < 4; ++k) q[k] = hb.ld4u(static_cast<uint32_t>((16 * tid + 4 * k) * 4));
      uint32_t bad = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        bad |= ((q[k].x >> 16) ^ tag16) | ((q[k].y >> 16) ^ tag16) | ((q[k].z >> 16) ^ tag16) |
               ((q[k].w >> 16) ^ tag16);
      if (__all(bad == 0) || timed_out) break;
      __builtin_amdgcn_s_sleep(1);
      timed_out = (__builtin_amdgcn_s_memrealtime() - t0) > wait_bound;
    }
    if (wv == 0) MA_XSTAMP(6);  // h word 0 .. 15 seen (thread 0)
    float hv[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      hv[4 * k] = __uint_as_float(q[k].x << 16);
      hv[4 * k + 1] = __uint_as_float(q[k].y << 16);
      hv[4 * k + 2] = __uint_as_float(q[k].z << 16);
      hv[4 * k + 3] = __uint_as_float(q[k].w << 16);
    }
    uint32_t pr[8];
    hc[tid] = prep_word_pairs(hv, pr);
#pragma unroll
    for (int j = 0; j < 8; ++j) hs[tid][j] = pr[j];
  }
  __syncthreads();
  if (wv == 0) MA_XSTAMP(7);  // all of h staged in LDS

  // ---- 5. slot xcd's down rows r0 .. r0 + RPW, each rounded to bf16 (as the
  // reference's ternary_expert_gemv stores it) and scaled by the slot's
  // routing weight, published for the combining workgroups
  {
    XSlice<KWI> hsl;
    slice_from_lds<KWI>(hs, hc, kld, hsl);
    const ExpandConsts kc;
    const float wx = s_w;
#pragma unroll
    for (int u = 0; u < UD; ++u) {
      const float eo = group_sum<LPRI>(slice_dot<KWI>(wd[u], hsl, kc) * ad[u]);
      const float pv = wx * bf16_to_f32(f32_to_bf16(eo));
      if (kld == 0)
        st_coh64(&part[xcd * H + r0 + u * RPID + subd], (static_cast<uint64_t>(tag) << 32) | __float_as_uint(pv));
    }
  }
  if (wv == 0) MA_XSTAMP(8);  // this wave's weighted down values published

  // The O values of this workgroup's combine rows (wave 0), from the XCD's copy.
  if (o_w && wv == 0) {
    for (;;) {
      const uint64_t q = ld_coh64(&ox[ro >> 1]);
      const bool ok = static_cast<uint32_t>(q >> 32) == tag;
      rb = (ro & 1) ? (static_cast<uint32_t>(q) >> 16) : (static_cast<uint32_t>(q) & 0xffffu);
      if (__all(ok) || timed_out) break;
      __builtin_amdgcn_s_sleep(1);
      timed_out = (__builtin_amdgcn_s_memrealtime() - t0) > wait_bound;
    }
  }

  // ---- 6. y = residual + the slots' values in slot order.  With a next
  // projection every XCD combines all of y for its own workgroups (wave w of
  // workgroup lw polls slot w's values of rows 64 lw .. + 64) and hands it
  // over through its L2, two values per tagged word; each XCD stores an
  // eighth of y.  Otherwise workgroup wg finishes rows wg * FR .. + FR:
  // lane l of wave 0 polls slot l / FR's value of row wg * FR + l % FR.
  if (NX || nx_w) {
    static_assert(H == 64 * kXcdWgs, "64 rows of y per workgroup of an XCD");
    const int row = 64 * lw + lane;
    float pv = 0.f;
    for (;;) {
      const uint64_t q = ld_coh64(&part[wv * H + row]);
      const bool ok = static_cast<uint32_t>(q >> 32) == tag;
      pv = __uint_as_float(static_cast<uint32_t>(q));
      if (__all(ok) || timed_out) break;
      __builtin_amdgcn_s_sleep(1);
      timed_out = (__builtin_amdgcn_s_memrealtime() - t0) > wait_bound;
    }
    if (wv == 0) MA_XSTAMP(9);  // the slots' values of this workgroup's rows seen
    s_pv[wv][lane] = pv;
    __syncthreads();
    if (wv == 0) {
      float v = addp ? bf16_to_f32(f32_to_bf16(__uint_as_float(ra << 16) + __uint_as_float(rb << 16)))
                   : residual ? __uint_as_float(ra << 16) : 0.f;
#pragma unroll
      for (int k = 0; k < TK; ++k) v += s_pv[k][lane];
      const uint32_t bits = f32_to_bf16(v);
      if ((lane >> 3) == xcd) y[row] = static_cast<uint16_t>(bits);
      const uint32_t odd = __shfl_xor(bits, 1, 64);
      if (!(lane & 1)) st_l2_64(&yx[row >> 1], (static_cast<uint64_t>(tag) << 32) | bits | (odd << 16));
      MA_XSTAMP(10);  // y out
    }
  } else if (wv == 0) {
    const int s = lane / FR, r = lane % FR;
    float pv = 0.f;
    for (;;) {
      const uint64_t q = ld_coh64(&part[s * H + wg * FR + r]);
      const bool ok = static_cast<uint32_t>(q >> 32) == tag;
      pv = __uint_as_float(static_cast<uint32_t>(q));
      if (__all(ok) || timed_out) break;
      __builtin_amdgcn_s_sleep(1);
      timed_out = (__builtin_amdgcn_s_memrealtime() - t0) > wait_bound;
    }
    MA_XSTAMP(9);
    float v = addp ? bf16_to_f32(f32_to_bf16(__uint_as_float(ra << 16) + __uint_as_float(rb << 16)))
                 : residual ? __uint_as_float(ra << 16) : 0.f;
#pragma unroll
    for (int k = 0; k < TK; ++k) v += __shfl(pv, k * FR + r, 64);
    if (lane < FR) y[wg * FR + lane] = f32_to_bf16(v);
    MA_XSTAMP(10);
  }

  // ---- 7. next projection (optional), from the XCD's copy of y
  if (NX || nx_w) {
    float nxa[NXP];
#pragma unroll
    for (int p = 0; p < NXP; ++p) nxa[p] = from_raw<ADT>(nxa_raw[p]);
    timed_out = next_projection<KWH, LPRH, W, NXP, true>(y, nx_rms, nx_eps, nx_rows, nx_rq, nx_out, nxw, nxa, ws,
                                                         0u, G, wg, tid, lane, wv, t0, yx, tag, wait_bound,
#ifdef MA_PHASE_STAMPS
                                                         stamps,
#else
                                                         nullptr,
#endif
                                                         NX ? &nxr : nullptr) ||
                timed_out;
  }
  if (pf && wv > 0) {  // hold the prefetched lines until they have arrived
#pragma unroll
    for (int k = 0; k < kPfPerLane; ++k) asm volatile("" ::"v"(pfv[k].x));
  }
  if (wv == 0) MA_XSTAMP(11);  // end
  if (__ballot(timed_out)) {
    if (lane == 0) st_coh32(&ws[2], 1u);
    // the layout check: a slot of this XCD still without this call's tag
    // after 10 us more means no workgroup with that number ran here
    // (another XCD ran two of one)
    if (wv == 0) {
      const uint32_t* const slot = present + xcd * kXcdWgs + (lane & (kXcdWgs - 1));
      bool empty = __any(ld_coh32(slot) != tag);
      const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
      while (empty && __builtin_amdgcn_s_memrealtime() - t1 < 1000) {
        __builtin_amdgcn_s_sleep(8);
        empty = __any(ld_coh32(slot) != tag);
      }
      if (empty && lane == 0) st_coh32(&ws[kXLayoutWord], 1u);
    }
  }
  if (tid == 0) st_coh32(calls, tag);
}

// The instances in a fixed order in the code object: the forms without the
// next projection first (the kernel's timing moved by ~0.7 % with its
// position in the code object alone).
#define MA_XCD_INST(US, KWI, ADT, NX)                                                                      \
  template __global__ void k_moe_xcd<4, US, KWI, 16, 2, ADT, NX>(                                         \
      const uint16_t*, uint32_t*, const uint16_t*, const uint16_t*, const uint16_t*, const void*, int, int, \
      float, const float*, const uint32_t*, const void*, const uint32_t*, const void*, uint16_t*, int32_t*, \
      float*, const uint32_t*, const void*, const float*, float, int, uint16_t*,                         \
      const uint16_t*, const uint32_t*, const void*, const uint4*, int, uint64_t);
MA_XCD_INST(3, 3, MA_F32, false)
MA_XCD_INST(2, 2, MA_F32, false)
MA_XCD_INST(3, 3, MA_BF16, false)
MA_XCD_INST(2, 2, MA_BF16, false)
MA_XCD_INST(3, 3, MA_F32, true)
MA_XCD_INST(2, 2, MA_F32, true)
MA_XCD_INST(3, 3, MA_BF16, true)
MA_XCD_INST(2, 2, MA_BF16, true)
#undef MA_XCD_INST

namespace {

template <int ADT, bool NX>
const void* xcd_kernel_t(int64_t inter) {
  return inter == 768 ? reinterpret_cast<const void*>(&k_moe_xcd<4, 3, 3, 16, 2, ADT, NX>)
                      : reinterpret_cast<const void*>(&k_moe_xcd<4, 2, 2, 16, 2, ADT, NX>);
}

}  // namespace

}  // namespace ma

// Where the XCD kernel's phase stamps sit in the workspace (MA_OK only in the
// library's stamped variant, built with -DMA_PHASE_STAMPS).
extern "C" int ma_moe_phase_stamps(size_t* offset, int* words_per_workgroup, int* workgroups) {
  using namespace ma;
  if (!offset || !words_per_workgroup || !workgroups) return fail(MA_EVALUE, "moe_phase_stamps: null output");
#ifdef MA_PHASE_STAMPS
  *offset = kXStampOff;
  *words_per_workgroup = kXStampWords;
  *workgroups = kXcds * kXcdWgs;
  return MA_OK;
#else
  *offset = 0;
  *words_per_workgroup = 0;
  *workgroups = 0;
  return fail(MA_EVALUE, "moe_phase_stamps: this library was built without phase stamps "
                         "(libmaple_amd_stamps.so has them)");
#endif
}

namespace ma {

bool moe_xcd_supported(int64_t n_experts, int64_t hidden, int64_t inter, int64_t top_k, hipStream_t st) {
  if (!(hidden == 2048 && (inter == 768 || inter == 512) && top_k == kXcds && n_experts >= top_k &&
        n_experts <= 64))
    return false;
  const char* force = getenv("MAPLE_AMD_MOE_FUSED");  // "grid": the one-barrier form (A/B timing)
  if (force && strcmp(force, "grid") == 0) return false;
  int cus = 0, dev = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus != kXcds * kXcdWgs)
    return false;
  int64_t capacity = 0;  // every workgroup resident (the grid form is used otherwise)
  for (const void* k : {xcd_kernel_t<MA_BF16, false>(inter), xcd_kernel_t<MA_BF16, true>(inter)})
    if (resident_capacity(k, 512, &capacity) != MA_OK || capacity < kXcds * kXcdWgs) return false;
  bool ok = false;
  return xcd_round_robin(st, &ok) == MA_OK && ok;
}

int moe_xcd_launch(const void* x, const void* x_add, const void* norm_weight, int norm_dtype, float eps,
                   const void* residual, const void* gate_weight, const float* router_bias, int64_t n_experts,
                   int64_t hidden, int64_t inter, const uint32_t* up_gate, const void* up_gate_alpha,
                   const uint32_t* down, const void* down_alpha, int alpha_dtype, void* y, int32_t* topk_ids,
                   float* topk_weight, void* workspace, const uint32_t* next_w, const void* next_alpha,
                   const float* next_rms, float next_eps, int64_t next_rows, void* next_out, const void* attn,
                   const uint32_t* o_w, const void* o_alpha, const void* prefetch, int64_t prefetch_bytes,
                   hipStream_t st) {
  (void)hidden;
  const bool nx = next_w != nullptr;
  const void* kern = alpha_dtype == MA_F32 ? (nx ? xcd_kernel_t<MA_F32, true>(inter) : xcd_kernel_t<MA_F32, false>(inter))
                                           : (nx ? xcd_kernel_t<MA_BF16, true>(inter) : xcd_kernel_t<MA_BF16, false>(inter));
  int64_t capacity = 0;
  if (int rc = resident_capacity(kern, 512, &capacity)) return rc;
  if (capacity < kXcds * kXcdWgs)
    return fail(MA_ERUNTIME, "moe_fused: its %d workgroups wait on each other but the device holds %lld at once",
                kXcds * kXcdWgs, static_cast<long long>(capacity));
#define MA_XCD_ARGS                                                                                      \
  static_cast<const uint16_t*>(x), static_cast<uint32_t*>(workspace),                                 \
      static_cast<const uint16_t*>(gate_weight), static_cast<const uint16_t*>(residual),               \
      static_cast<const uint16_t*>(x_add), norm_weight, static_cast<int>(n_experts),                   \
      (norm_dtype & 0xff) | (o_w ? kXHasO : 0), eps, router_bias, up_gate, up_gate_alpha, down,        \
      down_alpha, static_cast<uint16_t*>(y), topk_ids, topk_weight, next_w, next_alpha, next_rms, next_eps, \
      static_cast<int>(next_rows), static_cast<uint16_t*>(next_out), static_cast<const uint16_t*>(attn), o_w, \
      o_alpha, static_cast<const uint4*>(prefetch), pf_units, wait_bound
  // the prefetch is a hint: whole 16-byte units, at most what the lanes cover
  const int64_t pf_max = static_cast<int64_t>(kPfPerLane) * kXcdWgs * 7 * 64;
  const int pf_units = prefetch ? static_cast<int>(std::min<int64_t>(prefetch_bytes / 16, pf_max)) : 0;
  if (prefetch && (reinterpret_cast<uintptr_t>(prefetch) & 15))
    return fail(MA_EVALUE, "moe_fused: the prefetch range must be 16-byte aligned");
  // the waits' bound (MAPLE_AMD_WAIT_BOUND_US, for tests)
  uint64_t wait_bound = kXWaitTicks;
  if (const char* e = getenv("MAPLE_AMD_WAIT_BOUND_US")) wait_bound = static_cast<uint64_t>(atoll(e)) * 100;
  const dim3 grid(kXcds * kXcdWgs), block(512);
#define MA_XCD_LAUNCH(ADT, NX)                                                                 \
  do {                                                                                        \
    if (inter == 768)                                                                         \
      hipLaunchKernelGGL((k_moe_xcd<4, 3, 3, 16, 2, ADT, NX>), grid, block, 0, st, MA_XCD_ARGS); \
    else                                                                                      \
      hipLaunchKernelGGL((k_moe_xcd<4, 2, 2, 16, 2, ADT, NX>), grid, block, 0, st, MA_XCD_ARGS); \
  } while (0)
  if (alpha_dtype == MA_F32) {
    if (nx)
      MA_XCD_LAUNCH(MA_F32, true);
    else
      MA_XCD_LAUNCH(MA_F32, false);
  } else {
    if (nx)
      MA_XCD_LAUNCH(MA_BF16, true);
    else
      MA_XCD_LAUNCH(MA_BF16, false);
  }
#undef MA_XCD_LAUNCH
#undef MA_XCD_ARGS
  return check_launch("moe_fused");
}

}  // namespace ma
