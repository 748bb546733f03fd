/*
 * maple_amd -- C ABI of the MI355X (gfx950) packed-ternary MoE decode kernels.
 *
 * Every entry point takes raw device pointers, int64 sizes/leading dimensions,
 * dtype enums and a hipStream_t passed as void*.  Nothing here allocates,
 * synchronises the device or the host, or keeps state between calls, so all
 * calls are capturable in a HIP graph.  Outputs are written in the dtype the
 * reference uses for them; inputs are never modified.
 *
 * Return value: MA_OK (0) or an MA_E* status; ma_last_error() then holds a
 * message for the calling thread.  The Python host maps MA_EVALUE to
 * ValueError, MA_ETYPE to TypeError and MA_ERUNTIME to RuntimeError, the
 * exception types the reference raises for the same conditions.
 *
 * Layouts (reference src/maple_run/pack.py:17-20):
 *   ternary   uint32 [N, K/16] (or [K/16, N] with packed_kn), 16 two-bit
 *             codes per word, LSB first, value = code - 1.
 *   rtn4      uint32 [N, K/8] (or [K/8, N] with packed_kn), 8 four-bit codes
 *             per word, LSB first, value = q * scale[g] + bias[g].
 * Rows of x / y are contiguous along K / N with leading dimension ld*.
 */
#ifndef MAPLE_AMD_H
#define MAPLE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of float tensors. */
enum { MA_F32 = 0, MA_BF16 = 1, MA_F16 = 2 };
/* Status codes. */
enum { MA_OK = 0, MA_EVALUE = 1, MA_ETYPE = 2, MA_ERUNTIME = 3 };

/* Library version (major * 10000 + minor * 100 + patch). */
int ma_version(void);

/* Message of the last failing call on this host thread ("" if none). */
const char* ma_last_error(void);

/*
 * y[b, n] = alpha[n] * sum_k (code[n, k] - 1) * x_hat[b, k]
 * with x_hat = x, or with rms_weight != NULL, x_hat = x * w_rms and the row
 * scaled by rsqrt(mean(x^2) + rms_eps): the fused input RMSNorm.
 * y has x's dtype.  Replaces ternary_gemv, src/maple_run/kernels/ternary_gemv.py:261-388.
 */
int ma_ternary_gemv(const void* x, int x_dtype, int64_t batch, int64_t ldx,
                    const uint32_t* packed, int64_t n_out, int64_t nwords, int packed_kn,
                    const void* row_alpha, int alpha_dtype,
                    const void* rms_weight, int rms_dtype, float rms_eps,
                    void* y, int64_t ldy, void* stream);

/*
 * ma_ternary_gemv with a caller-supplied workspace.  With the fused RMSNorm
 * (rms_weight != NULL) and 17 tokens or more, every token's GEMM operands
 * (the x' pairs of the hi and lo halves of x * w_rms, the correction and the
 * RMS scale) are built once into the workspace by a first launch and the MFMA
 * GEMM reads them from there.  workspace: 256-byte aligned, at least
 * ma_ternary_gemv_workspace_bytes(batch, nwords, rms_weight != NULL) bytes;
 * that query returns 0 where no workspace is used (no RMSNorm, batch < 17,
 * nwords % 16 != 0), and then -- as for any input the GEMM does not take --
 * the call is ma_ternary_gemv's and workspace may be NULL.  Same values as
 * ma_ternary_gemv up to float32 summation order.  Replaces ternary_gemv,
 * src/maple_run/kernels/ternary_gemv.py:261-388 (its batched path :156-258).
 */
size_t ma_ternary_gemv_workspace_bytes(int64_t batch, int64_t nwords, int rms);
int ma_ternary_gemv_ws(const void* x, int x_dtype, int64_t batch, int64_t ldx,
                       const uint32_t* packed, int64_t n_out, int64_t nwords, int packed_kn,
                       const void* row_alpha, int alpha_dtype,
                       const void* rms_weight, int rms_dtype, float rms_eps,
                       void* y, int64_t ldy, void* workspace, size_t workspace_bytes,
                       void* stream);

/*
 * The grouped MoE's combine and the next RMS-folded ternary GEMM in the same
 * two launches as ma_ternary_gemv_ws: x[t] = sum_j topk_weight[t, j] *
 * slot_out[inverse[t, j]] (+ residual[t]) in float32, slot order, rounded to
 * bf16 -- the values ma_moe_grouped's combine stores -- is written to x_out
 * (bf16 [batch, nwords * 16]) and is the GEMM's x; y as ma_ternary_gemv_ws
 * with that x.  slot_out is the per-pair down output ma_moe_grouped leaves at
 * byte offset n_pairs * inter * 2 (rounded up to a multiple of 256) of its
 * workspace (bf16 [n_pairs, hidden]);
 * call ma_moe_grouped with y = NULL to skip its own combine.  Needs
 * rms_weight, batch >= 17, nwords % 16 == 0, top_k <= 8, bf16 rows and
 * 16-byte aligned buffers (returns MA_EVALUE otherwise); workspace as for
 * ma_ternary_gemv_ws.  Reference counterpart: moe_reduce_add
 * (src/maple_run/kernels/fused_norm.py:59-96) at the end of one decoder
 * layer, then the next layer's input RMSNorm + QKV ternary_gemv
 * (src/maple_run/kernels/ternary_gemv.py:261-388) -- one boundary crossing
 * fewer per layer.
 */
int ma_ternary_gemv_combine_ws(const void* slot_out, const int32_t* inverse,
                               const float* topk_weight, int64_t top_k, const void* residual,
                               void* x_out, int64_t batch, const uint32_t* packed, int64_t n_out,
                               int64_t nwords, const void* row_alpha, int alpha_dtype,
                               const void* rms_weight, int rms_dtype, float rms_eps, void* y,
                               int64_t ldy, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Router: logits = x @ W^T (+ bias), softmax over the experts, the top_k
 * largest probabilities in descending order (ties: lowest expert index) and
 * their renormalised weights p / (sum p_top + 1e-20).
 * ids int32 [tokens, top_k], weights float32 [tokens, top_k].
 * workspace: at least ma_router_workspace_bytes(tokens, n_experts) bytes.
 * Replaces router_topk, src/maple_run/kernels/router.py:141-217 (the bias is
 * an optional addition; NULL is the reference behaviour).
 */
size_t ma_router_workspace_bytes(int64_t tokens, int64_t n_experts);
int ma_router_topk(const void* x, int x_dtype, int64_t tokens, int64_t ldx,
                   const void* gate_weight, int w_dtype, int64_t n_experts, int64_t k_in,
                   const float* bias, int top_k,
                   int32_t* ids, float* weights,
                   void* workspace, size_t workspace_bytes, void* stream);
/*
 * ma_router_topk that also writes x in the form the grouped expert GEMMs
 * read (x_pairs uint32 [tokens, k_in / 2], 16-byte aligned; x_corr float32
 * [tokens]: each token's correction sum), from the same per-token launch as
 * the top-k; ma_moe_grouped given them skips its own x' launch and returns
 * the same bits.  x bfloat16, k_in a multiple of 16, rows 16-byte aligned.
 * No reference counterpart: a fused form of router_topk and the first step
 * of the grouped experts, for prefill-sized batches.
 */
int ma_router_topk_pairs(const void* x, int x_dtype, int64_t tokens, int64_t ldx,
                         const void* gate_weight, int w_dtype, int64_t n_experts, int64_t k_in,
                         const float* bias, int top_k,
                         int32_t* ids, float* weights, uint32_t* x_pairs, float* x_corr,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * Dispatch of (token, slot) pairs p = token * top_k + slot to experts:
 * counts[e], offsets[e] (exclusive scan, n_experts + 1 entries), pair_ids
 * (pairs stably sorted by expert id, so every expert's list is ascending in
 * token) and inverse[p] (position of pair p in pair_ids).  ids may be int32
 * or int64 (ids_is_int64).  No reference counterpart: the reference grids over
 * pairs directly (src/maple_run/kernels/ternary_expert.py:210,443).
 */
int ma_moe_dispatch(const void* ids, int ids_is_int64, int64_t n_pairs, int n_experts,
                    int32_t* counts, int32_t* offsets, int32_t* pair_ids, int32_t* inverse,
                    void* stream);

/*
 * y[s, n] = alpha[e, n] * sum_k (code[e, n, k] - 1) * x[s / x_div, k], e = ids[s].
 * x_div = 1 for one x row per slot, top_k for one x row per token.
 * packed: [E, N, K/16] (or [E, K/16, N] with packed_kn); alpha [E, N].
 * Replaces ternary_expert_gemv, src/maple_run/kernels/ternary_expert.py:125-234.
 */
int ma_ternary_expert_gemv(const void* x, int x_dtype, int64_t ldx, int64_t x_div,
                           const uint32_t* packed, int64_t n_experts, int64_t n_out,
                           int64_t nwords, int packed_kn,
                           const void* row_alpha, int alpha_dtype,
                           const void* ids, int ids_is_int64, int64_t n_slots,
                           void* y, int64_t ldy, void* stream);

/*
 * h[t, j, i] = clamp(up, -7, 7) * g * sigmoid(g), g = min(gate, 7), with
 * up = alpha[e, i] * (T_e[i] . x[t]) and gate the same on row N + i
 * (rows are [up; gate]), e = ids[t, j].  h has x's dtype, [tokens*top_k, N].
 * Replaces ternary_expert_swiglu, src/maple_run/kernels/ternary_expert.py:403-468.
 */
int ma_ternary_expert_swiglu(const void* x, int x_dtype, int64_t ldx, int64_t tokens,
                             int64_t top_k, const uint32_t* packed, int64_t n_experts,
                             int64_t n_rows, int64_t nwords, int packed_kn,
                             const void* row_alpha, int alpha_dtype,
                             const void* ids, int ids_is_int64,
                             void* h, int64_t ldh, void* stream);

/*
 * y[t, n] = sum_j w[t, j] * alpha[e, n] * (T_e[n] . x[t, j]) (+ residual[t, n])
 * in float32 with a single rounding on store; x is [tokens, top_k, K]
 * (row stride ldx per slot), y has x's dtype.
 * Replaces ternary_expert_down_sum, src/maple_run/kernels/ternary_expert.py:471-556.
 */
int ma_ternary_expert_down_sum(const void* x, int x_dtype, int64_t ldx,
                               const uint32_t* packed, int64_t n_experts, int64_t n_out,
                               int64_t nwords, int packed_kn,
                               const void* row_alpha, int alpha_dtype,
                               const void* ids, int ids_is_int64, const float* topk_weight,
                               const void* residual, int residual_dtype,
                               int64_t tokens, int64_t top_k,
                               void* y, int64_t ldy, void* stream);

/*
 * The MoE block's down projection and top-k combine in one launch, with the
 * block's rounding: out_j = alpha_e (.) (T_e h[t, j]) rounded to x_dtype per
 * slot (what ternary_expert_gemv stores), then y[t] = sum_j w[t, j] * out_j
 * in float32 in slot order, + residual[t] last, stored in x_dtype (what
 * moe_reduce_add computes).  Same arguments as ma_ternary_expert_down_sum.
 * Replaces the pair ternary_expert_gemv + moe_reduce_add of
 * MapleSparseMoeBlock.__call__ (src/maple_run/model.py:470-473;
 * kernels/ternary_expert.py:125-234, kernels/fused_norm.py:164-202), two
 * launches there.
 */
int ma_ternary_expert_down_combine(const void* x, int x_dtype, int64_t ldx,
                                   const uint32_t* packed, int64_t n_experts, int64_t n_out,
                                   int64_t nwords, int packed_kn,
                                   const void* row_alpha, int alpha_dtype,
                                   const void* ids, int ids_is_int64, const float* topk_weight,
                                   const void* residual, int residual_dtype,
                                   int64_t tokens, int64_t top_k,
                                   void* y, int64_t ldy, void* stream);

/*
 * y[t, n] = sum_j w[t, j] * expert_out[t, j, n] (+ residual[t, n]), float32
 * accumulate, stored in expert_out's dtype.
 * Replaces moe_reduce_add, src/maple_run/kernels/fused_norm.py:164-202.
 */
int ma_moe_reduce_add(const void* expert_out, int eo_dtype, int64_t tokens, int64_t top_k,
                      int64_t n, const float* topk_weight,
                      const void* residual, int residual_dtype,
                      void* y, void* stream);

/*
 * RMSNorm over rows of n: y = x * rsqrt(mean(x^2) + eps) * w, y in x's dtype.
 * Replaces rms_norm, src/maple_run/kernels/fused_norm.py:105-125.
 */
int ma_rms_norm(const void* x, int x_dtype, int64_t rows, int64_t n,
                const void* weight, int w_dtype, float eps, void* y, void* stream);

/*
 * residual = x + y; normed = rms_norm(residual) (computed from the float32
 * sum); both in x's dtype.  Replaces add_rms_norm, fused_norm.py:128-161.
 */
int ma_add_rms_norm(const void* x, const void* y, int dtype, int64_t rows, int64_t n,
                    const void* weight, int w_dtype, float eps,
                    void* residual, void* normed, void* stream);

/*
 * y[b, n] = sum_g sum_{k in g} (q[n, k] * scale[n, g] + bias[n, g]) * x[b, k],
 * float32 accumulate, y in x's dtype.  scales/biases are [N, K/group]
 * (or [K/group, N] with packed_kn).
 * Replaces rtn4_gemv, src/maple_run/kernels/rtn4.py:285-415.
 */
int ma_rtn4_gemv(const void* x, int x_dtype, int64_t batch, int64_t ldx,
                 const uint32_t* packed, int64_t n_out, int64_t nwords, int packed_kn,
                 const void* scales, int scales_dtype, const void* biases, int biases_dtype,
                 int64_t group_size, void* y, int64_t ldy, void* stream);

/*
 * ma_rtn4_gemv with a workspace: from batch 5 in groups of 128 (N a multiple
 * of 32, bf16 x, [N, K/8] codes, 16-byte aligned) the x' operands and group
 * sums are built once into the workspace and copied into LDS by the LDS DMA
 * while the weights stream (the same bits as ma_rtn4_gemv); any other call
 * is ma_rtn4_gemv's.  workspace: ma_rtn4_gemv_workspace_bytes(batch, nwords,
 * group_size) bytes (0: none needed), 256-byte aligned; calls sharing one
 * must not overlap.  Replaces rtn4_gemv, src/maple_run/kernels/rtn4.py:285-415.
 */
size_t ma_rtn4_gemv_workspace_bytes(int64_t batch, int64_t nwords, int64_t group_size);
int ma_rtn4_gemv_ws(const void* x, int x_dtype, int64_t batch, int64_t ldx,
                    const uint32_t* packed, int64_t n_out, int64_t nwords, int packed_kn,
                    const void* scales, int scales_dtype, const void* biases, int biases_dtype,
                    int64_t group_size, void* y, int64_t ldy, void* workspace, size_t workspace_bytes,
                    void* stream);

/*
 * out[i, k] = q[ids[i], k] * scale[ids[i], g] + bias[ids[i], g] in float32.
 * Replaces rtn4_embedding, src/maple_run/kernels/rtn4.py:27-47.
 */
int ma_rtn4_embedding(const void* ids, int ids_is_int64, int64_t n_ids,
                      const uint32_t* packed, int64_t vocab, int64_t nwords,
                      const void* scales, int scales_dtype, const void* biases, int biases_dtype,
                      int64_t group_size, float* out, void* stream);

/*
 * Batched MoE routing in ONE launch: h = x + x_add (bf16; skipped when x_add
 * is NULL, then h is x), xn = RMSNorm(h) * norm_weight (bf16) -- with xn_pairs
 * / xn_corr (optional, both or neither; hidden % 16 == 0) also xn in the x'
 * pair form ma_moe_grouped reads and each token's correction -- the router
 * (logits = xn @ gate_weight^T + router_bias, softmax, top_k ids / weights)
 * and the dispatch lists (counts, offsets, pair_ids, inverse as
 * ma_moe_dispatch gives them).  Same values, bit for bit, as ma_add_rms_norm
 * (or ma_rms_norm), ma_router_topk and ma_moe_dispatch run one after another
 * at these sizes.  tokens <= 1024, hidden % 8 == 0 and <= 4096, n_experts <=
 * 256, top_k <= 64; bf16 rows, 16-byte aligned.  workspace: 256-byte aligned, at least
 * ma_moe_route_workspace_bytes(tokens, n_experts) bytes, zero-filled once
 * when allocated (the kernel leaves it zero; word 64 becomes non-zero if a
 * wait ever timed out); calls sharing a workspace must not overlap.
 * Composes add_rms_norm (src/maple_run/kernels/fused_norm.py:31-56) and
 * router_topk (src/maple_run/kernels/router.py:141-217) with the dispatch.
 */
size_t ma_moe_route_workspace_bytes(int64_t tokens, int64_t n_experts);
int ma_moe_route(const void* x, const void* x_add, int64_t tokens, int64_t hidden,
                 const void* norm_weight, int norm_dtype, float eps,
                 const void* gate_weight, const float* router_bias,
                 int64_t n_experts, int top_k, void* h_out, void* xn_out,
                 uint32_t* xn_pairs, float* xn_corr,
                 int32_t* topk_ids, float* topk_weight, int32_t* counts,
                 int32_t* offsets, int32_t* pair_ids, int32_t* inverse,
                 void* workspace, size_t workspace_bytes, void* stream);

/*
 * Grouped MoE FFN after dispatch (batched decode and prefill), on MFMA:
 * per expert, h = SwiGLU(up/gate GEMM) over its pairs (rounded to bf16 as the
 * reference stores it), out = down GEMM per pair (rounded to bf16), then
 * y[t] = sum_j w[t, j] * out[pair(t, j)] (+ residual) in float32, stored bf16.
 * offsets / pair_ids / inverse are ma_moe_dispatch's outputs.  x is bf16
 * [tokens, hidden]; hidden and inter must be multiples of 256; row_alpha bf16
 * or float32.  h_out (optional, bf16 [tokens*top_k, inter], row stride ldh)
 * receives h in slot order; y (optional) is bf16 [tokens, hidden].
 * workspace: ma_grouped_workspace_bytes(tokens * top_k, inter, hidden).
 * x_pairs / x_corr (optional, both or neither): x as ma_moe_route writes it
 * in x' pair form (uint32 [tokens, hidden / 2]) with each token's correction
 * (float32 [tokens]); decode batches then read the operands from there
 * instead of building them from x (x is still passed).  The per-pair down
 * outputs stay in the workspace at byte offset tokens * top_k * inter * 2
 * rounded up to a multiple of 256 (bf16 [tokens * top_k, hidden]); with
 * y = NULL the combine is skipped
 * (ma_ternary_gemv_combine_ws can run it in front of the next GEMM).
 * Replaces MapleSparseMoeBlock's SwiGLU -> down -> moe_reduce_add chain
 * (src/maple_run/model.py:468-473) for token counts where experts see many
 * tokens; the reference instead runs one program per (token, slot).
 */
size_t ma_grouped_workspace_bytes(int64_t n_pairs, int64_t inter, int64_t hidden);
int ma_moe_grouped(const void* x, int64_t ldx, const uint32_t* x_pairs, const float* x_corr,
                   int64_t tokens, int64_t top_k,
                   const uint32_t* up_gate, const void* up_gate_alpha,
                   const uint32_t* down, const void* down_alpha, int alpha_dtype,
                   int64_t n_experts, int64_t hidden, int64_t inter,
                   const int32_t* offsets, const int32_t* pair_ids, const int32_t* inverse,
                   const float* topk_weight, const void* residual, int residual_dtype,
                   void* h_out, int64_t ldh, void* y,
                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * ma_moe_grouped with no workspace argument that allocates nothing: the same
 * kernels stage h and the per-pair down outputs in a device array built into
 * the library (one per GPU, held until the process ends), of
 * ma_moe_grouped_noalloc_max_bytes() bytes (16 MiB: up to 339 tokens at
 * top-8, 2712 (token, expert) pairs, at hidden 2048 / intermediate 768).
 * Larger calls return MA_EVALUE.  y is required (the per-pair outputs stay in
 * the internal array).  Every call on one GPU shares that array: calls that
 * overlap on one GPU (other streams, other threads) race; calls ordered on a
 * stream do not.  Nothing in the array needs clearing between calls.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation).
 */
size_t ma_moe_grouped_noalloc_max_bytes(void);
int ma_moe_grouped_noalloc(const void* x, int64_t ldx, const uint32_t* x_pairs,
                           const float* x_corr, int64_t tokens, int64_t top_k,
                           const uint32_t* up_gate, const void* up_gate_alpha,
                           const uint32_t* down, const void* down_alpha, int alpha_dtype,
                           int64_t n_experts, int64_t hidden, int64_t inter,
                           const int32_t* offsets, const int32_t* pair_ids, const int32_t* inverse,
                           const float* topk_weight, const void* residual, int residual_dtype,
                           void* h_out, int64_t ldh, void* y, void* stream);

/*
 * One token through the whole MoE layer in ONE launch (decode batch 1):
 * router (x @ gate_weight^T + bias, softmax, top-k, renormalise), expert
 * SwiGLU (h in bf16), down projections and the weighted combine, + residual;
 * y bf16 [hidden], topk_ids int32 [top_k], topk_weight float32 [top_k].
 * With x_add != NULL the block first computes s = x + x_add (float32) and runs
 * on bf16(rms_norm(s) * norm_weight) with residual bf16(s) (the decoder's
 * post-attention add + RMSNorm); otherwise residual may be NULL.  bf16 x and
 * gate weight; row scales (up_gate_alpha, down_alpha) float32 or bf16, both
 * of alpha_dtype.  Built shapes (hidden, inter, top_k): (2048,
 * 768, 8), (2048, 512, 8) and (256, 128, 2); experts <= 256; other shapes
 * return MA_EVALUE (use the per-kernel entry points).  Two forms of the
 * launch give the same results to float32 rounding: at top-8 with hidden
 * 2048 and at most 64 experts, on a GPU of 8 XCDs x 32 compute units that
 * hands a launch's workgroups to its XCDs in turn (checked once per device,
 * by a probe launch on the call's stream that synchronises it -- the first
 * call outside graph capture; a call captured before that runs the second
 * form),
 * XCD x computes slot x and its workgroups hand data to each other through
 * that XCD's L2; otherwise one grid barrier separates SwiGLU and down
 * (ma_moe_fused_form says which; the environment variable
 * MAPLE_AMD_MOE_FUSED=grid forces the second form).  workspace:
 * ma_moe_fused_workspace_bytes(...) bytes, zero-filled before its first use
 * and never cleared again (the kernel keeps a call counter there and tags
 * the data it hands between workgroups with it); calls sharing a workspace
 * must not overlap.
 * A cross-workgroup
 * wait that exceeds about 0.2 s sets the word read by ma_moe_fused_timed_out
 * instead of hanging.  Replaces MapleSparseMoeBlock.__call__ at T = 1,
 * src/maple_run/model.py:448-474 (router_topk, ternary_expert_swiglu,
 * ternary_expert_gemv, moe_reduce_add: four launches there), optionally with
 * add_rms_norm, src/maple_run/kernels/fused_norm.py:128-161.
 * With next_w != NULL the same launch also computes the next layer's input
 * projection from y: next_out bf16 [next_rows] = ternary_gemv(y, next_w
 * [next_rows, hidden/16], next_alpha (alpha_dtype), rms_weight = next_rms
 * float32 [hidden], next_eps) -- the bits ma_ternary_gemv gives (reference
 * src/maple_run/kernels/ternary_gemv.py:110-146, the QKV projection of
 * MapleAttention, model.py:368-414); y, next_w and next_rms 16-byte aligned,
 * next_rows <= 4096 at hidden 2048.
 * prefetch / prefetch_bytes (optional, 16-byte aligned; NULL / 0 for none):
 * memory the launch only reads ahead into the caches for a later kernel,
 * such as the next MoE layer's router rows (routing-independent bytes): in
 * the XCD-split form every XCD reads the first min(prefetch_bytes, 448 KB)
 * bytes while its workgroups wait for h, so the next layer's router loads
 * hit.  No effect on the results; the one-barrier form ignores it.  No
 * reference counterpart (a scheduling hint).
 */
size_t ma_moe_fused_workspace_bytes(int64_t n_experts, int64_t hidden, int64_t inter,
                                    int64_t top_k);
int ma_moe_fused(const void* x, const void* x_add, const void* norm_weight, int norm_dtype,
                 float eps, const void* residual, const void* gate_weight,
                 const float* router_bias, int64_t n_experts, int64_t hidden, int64_t inter,
                 int64_t top_k, const uint32_t* up_gate, const void* up_gate_alpha,
                 const uint32_t* down, const void* down_alpha, int alpha_dtype, void* y,
                 int32_t* topk_ids,
                 float* topk_weight, void* workspace, size_t workspace_bytes,
                 const uint32_t* next_w, const void* next_alpha, int next_alpha_dtype,
                 const float* next_rms, float next_eps, int64_t next_rows, void* next_out,
                 const void* prefetch, int64_t prefetch_bytes, void* stream);
/* The one-launch layer's workgroups wait on each other (a grid barrier), so
 * all of them must be resident at once: *needed = its grid for this shape,
 * *capacity = compute units x resident workgroups per unit on the current
 * device.  ma_moe_fused itself fails with MA_ERUNTIME where needed >
 * capacity (a partitioned GPU, say); callers then run the multi-launch
 * kernels.  MA_EVALUE if the shape is not built.  No reference counterpart
 * (the reference has no persistent kernel); a query for the choice above. */
int ma_moe_fused_resident(int64_t n_experts, int64_t hidden, int64_t inter, int64_t top_k,
                          int64_t* needed, int64_t* capacity);

/* The form ma_moe_fused runs for this shape on the current device: 1 the
 * XCD split, 0 the one-barrier grid, -1 not built (may run the one-time probe
 * above on the null stream).  No reference counterpart. */
int ma_moe_fused_form(int64_t n_experts, int64_t hidden, int64_t inter, int64_t top_k);

/*
 * ma_moe_fused with the attention's output projection in front, in place of
 * x_add: the launch computes x_add = ternary_gemv(attn, o_w, o_alpha) itself
 * (attn bf16 [hidden], o_w [hidden, hidden / 16] uint32 codes, o_alpha
 * [hidden] of alpha_dtype; the bits ma_ternary_gemv gives), then the add +
 * RMSNorm (norm_weight required) and the layer as ma_moe_fused, optionally
 * with the next projection; the residual added back is bf16(x + x_add).
 * Only in the XCD-split form (ma_moe_fused_form == 1; MA_EVALUE otherwise):
 * each XCD computes all of the projection and hands it to its own
 * workgroups through its L2.  Same workspace as ma_moe_fused.  Replaces the
 * o_proj of MapleAttention (src/maple_run/model.py:412-414, ternary_gemv)
 * and the add + RMSNorm + MapleSparseMoeBlock of the decoder layer
 * (model.py:448-474, fused_norm.py:128-161) at T = 1, two launches there.
 */
int ma_moe_fused_o(const void* x, const void* attn, const uint32_t* o_w, const void* o_alpha,
                   const void* norm_weight, int norm_dtype, float eps, const void* gate_weight,
                   const float* router_bias, int64_t n_experts, int64_t hidden, int64_t inter, int64_t top_k,
                   const uint32_t* up_gate, const void* up_gate_alpha, const uint32_t* down,
                   const void* down_alpha, int alpha_dtype, void* y, int32_t* topk_ids, float* topk_weight,
                   void* workspace, size_t workspace_bytes, const uint32_t* next_w, const void* next_alpha,
                   int next_alpha_dtype, const float* next_rms, float next_eps, int64_t next_rows,
                   void* next_out, const void* prefetch, int64_t prefetch_bytes, void* stream);

/* Phase stamps of the XCD-split form (diagnostics, no reference
 * counterpart).  In the library's stamped variant (libmaple_amd_stamps.so,
 * built from the same sources with -DMA_PHASE_STAMPS) every call writes, per
 * workgroup, words_per_workgroup uint32 words at byte `offset` of its
 * workspace (workgroup g's row at offset + 4 * words * g): word i is the
 * 100 MHz real-time counter when the workgroup reached phase i (0 start,
 * 1 router logit out (workgroups 0..7 of an XCD), 2 all logits seen,
 * 3 ranked, 4 weight loads issued, 5 h published, 6 h seen, 7 h staged,
 * 8 weighted down values published, 9 the slots' values seen, 10 y out,
 * 11 end), word 15 its XCD.  Returns MA_OK there and MA_EVALUE in the
 * normal library, which writes none. */
int ma_moe_phase_stamps(size_t* offset, int* words_per_workgroup, int* workgroups);

/* *out = 1 if any ma_moe_fused call on this workspace timed out waiting,
 * 2 if the XCD-split form found its workgroups not spread over the XCDs as
 * it assumes (every XCD running 32 of them with distinct numbers i / 8: the
 * call is aborted at once, its outputs invalid; turn the form off with
 * ma_xcd_forms_disable), 0 otherwise, since the workspace was zeroed
 * (synchronises the stream).  No reference counterpart: the reference has no
 * cross-workgroup wait. */
int ma_moe_fused_timed_out(const void* workspace, int* out, void* stream);

/* Turn the XCD-split forms (ma_moe_fused's XCD split, the XCD-local decode
 * attention) off (disable != 0) or on again for device `device`: later calls
 * run the one-barrier / cross-XCD forms (same results to float32 rounding).
 * No reference counterpart. */
int ma_xcd_forms_disable(int device, int disable);

/*
 * Decode (q_len = 1) QK RMSNorm + partial RoPE + KV write.  qkv bf16
 * [batch, (n_heads + 2 n_kv_heads) * head_dim] (row stride ldq); per head
 * x * rsqrt(mean(x^2) + eps) * w (q_norm_w / k_norm_w [head_dim] of w_dtype),
 * rotate-half RoPE on the first rotary_dim dims.  cos/sin (cs_dtype, row
 * stride ld_cs): n_pos == 0 -> row b holds batch row b's values (the
 * reference's gathered [B, rotary_dim] form); n_pos > 0 -> a table of n_pos
 * rows indexed by seqlen[b] (clamped).  Values are rounded to bf16 before use.
 * K/V are stored at position seqlen[b] (clamped to [0, max_len)) of cache row
 * row_map[b] (b when row_map is NULL; clamped to [0, cache_rows)) of the bf16
 * caches [cache_rows, n_kv_heads, max_len, head_dim]; q_out bf16
 * [batch, n_heads, head_dim].  head_dim must be 64.
 * Replaces apply_qkv_decode, src/maple_run/kernels/decode_attn.py:362-439.
 */
int ma_qk_norm_rope_store(const void* qkv, int64_t ldq, int64_t batch, int n_heads,
                          int n_kv_heads, int head_dim, const void* q_norm_w,
                          const void* k_norm_w, int w_dtype, const void* cos, const void* sin,
                          int cs_dtype, int64_t ld_cs, int64_t n_pos, int rotary_dim,
                          int use_rope, float eps, const int64_t* seqlen,
                          const int64_t* row_map, void* k_cache, void* v_cache,
                          int64_t cache_rows, int64_t max_len, void* q_out, void* stream);

/*
 * Decode GQA attention: out[b, h] = softmax(q[b, h] . K^T * scale) V over
 * positions [start, min(seqlen[b] + 1, max_len)) of cache row row_map[b] (b
 * when NULL), start = kv_len - window when window > 0.  q / out bf16
 * [batch, n_heads, head_dim], float32 accumulation, P rounded to bf16, split
 * over the sequence (128 positions per split) and merged in the same launch
 * (the splits of a (row, KV head) meet at a barrier, then each merges a slice).
 * workspace: ma_gqa_workspace_bytes(batch, n_kv_heads, max_len, head_dim) bytes,
 * 16-byte aligned, zero-filled before the first call: it starts with a sync
 * area of 256-byte lines (line 0, int32 word 2: set to 1 if a barrier wait
 * ever exceeded about 0.2 s; then per (row, KV head) an arrival-counter line,
 * which each call leaves at zero, and a generation line; then 33 lines of a
 * grid barrier for the fused entry point's O projection).  Calls that share
 * a workspace must not overlap.  head_dim must be 64 or 128.
 * Replaces decode_gqa_attn, src/maple_run/kernels/decode_attn.py:470-592
 * (which merges the splits in a second kernel, :317-359).
 */
size_t ma_gqa_workspace_bytes(int64_t batch, int n_kv_heads, int64_t max_len, int head_dim);
int ma_decode_gqa_attn(const void* q, int64_t batch, int n_heads, int n_kv_heads, int head_dim,
                       const void* k_cache, const void* v_cache, int64_t cache_rows,
                       int64_t max_len, const int64_t* seqlen, const int64_t* row_map,
                       int64_t window, float scale, void* out, void* workspace,
                       size_t workspace_bytes, void* stream);

/*
 * ma_qk_norm_rope_store followed by ma_decode_gqa_attn in one launch (same
 * arguments and results; q is not written out).  The decode step of the
 * reference's MapleAttention, src/maple_run/model.py:368-414, which runs the
 * RoPE gather, apply_qkv_decode and decode_gqa_attn as separate launches.
 * With o_w != NULL (batch 1, n_heads * head_dim = 2048) the same launch also
 * computes the output projection o_proj of that attention:
 * o_out bf16 [o_rows] = ternary_gemv(out, o_w [o_rows, 128], o_alpha
 * (f32/bf16)) -- the bits ma_ternary_gemv gives (reference
 * src/maple_run/kernels/ternary_gemv.py:261-388); o_w 16-byte aligned,
 * o_rows <= 16 x the launch's workgroups (2112 for a 4224-position cache).
 */
int ma_decode_attn_fused(const void* qkv, int64_t ldq, int64_t batch, int n_heads,
                         int n_kv_heads, int head_dim, const void* q_norm_w,
                         const void* k_norm_w, int w_dtype, const void* cos, const void* sin,
                         int cs_dtype, int64_t ld_cs, int64_t n_pos, int rotary_dim,
                         int use_rope, float eps, const int64_t* seqlen, const int64_t* row_map,
                         void* k_cache, void* v_cache, int64_t cache_rows, int64_t max_len,
                         int64_t window, float scale, void* out, void* workspace,
                         size_t workspace_bytes, const uint32_t* o_w, const void* o_alpha,
                         int o_alpha_dtype, int64_t o_rows, void* o_out, void* stream);
/* 1 if ma_decode_attn_fused can compute an O projection of o_rows rows in the
 * launch for these sizes, else 0.  No reference counterpart (a capability
 * query for the fused output projection above). */
int ma_decode_attn_o_supported(int64_t batch, int n_heads, int n_kv_heads, int head_dim,
                               int64_t max_len, int64_t window, int64_t o_rows);
/* Which form ma_decode_gqa_attn (fused = 0) / ma_decode_attn_fused (fused = 1,
 * with_o = 1 with the O projection) launches for these sizes: 1 the
 * XCD-local form (every split of a (row, KV head) on one XCD, partials and
 * flags handed over through that XCD's L2; used where the GPU hands
 * workgroup i to XCD (i + o) mod 8, checked once per device by a small probe
 * kernel that is skipped while the stream is being captured), 0 the
 * cross-XCD form (arrival counter and generation word), -1 bad sizes.  Both
 * give the same bits.  MAPLE_AMD_ATTN=grid forces the cross-XCD form.  No
 * reference counterpart. */
int ma_decode_attn_form(int64_t batch, int n_kv_heads, int head_dim, int64_t max_len, int64_t window,
                        int fused, int with_o);

/*
 * Row-wise ternarisation (the converter's step): for each of `rows` rows of
 * k_in values of `weight` (float32, bfloat16 or float16; k_in a multiple of
 * 128, at most 8192): thr = threshold_scale * mean|w|, mask = |w| > thr,
 * row_alpha = sum(|w| * mask) / max(sum(mask), 1) in the weight dtype, and
 * packed uint32 [rows, k_in / 16] = codes sign(w) * mask + 1, 16 per word,
 * least significant first.  The means and sums are taken in float32 in
 * NumPy's pairwise summation order, so codes and row_alpha are the bits the
 * reference's NumPy converter produces.  Replaces ternarize,
 * src/maple_run/pack.py:120-149.
 */
int ma_ternarize(const void* weight, int dtype, int64_t rows, int64_t k_in, float threshold_scale,
                 uint32_t* packed, void* row_alpha, void* stream);

/*
 * Greedy choice: out[r] = argmax over the n values of row r (bf16 or float32,
 * row stride ldx), the lowest index on ties; out int64
 * [rows].  Replaces torch.argmax(logits, dim=-1) of the greedy step,
 * src/maple_run/generate.py:146-148.
 */
int ma_argmax_rows(const void* x, int x_dtype, int64_t rows, int64_t n, int64_t ldx,
                   int64_t* out, void* stream);

/*
 * The same choice, each row read by many workgroups (chunks of 1280 16-byte
 * vectors; the last one to finish reduces the row's partials): for rows of
 * 16-byte aligned bf16 / float32 logits up to 64 chunks long; other rows take
 * ma_argmax_rows.  workspace: ma_argmax_workspace_bytes(rows) bytes, 256-byte
 * aligned, zero-filled once (every call leaves it zero); calls sharing one
 * must not overlap.  Same replaced call as ma_argmax_rows.
 */
size_t ma_argmax_workspace_bytes(int64_t rows);
int ma_argmax_rows_ws(const void* x, int x_dtype, int64_t rows, int64_t n, int64_t ldx,
                      int64_t* out, void* workspace, size_t workspace_bytes, void* stream);

/*
 * GEMV over the rows of selected clusters: packed [n_clusters, cluster_size,
 * nwords] (the head's rows grouped by cluster), scales / biases [n_clusters,
 * cluster_size, groups] (bf16 or float32, one dtype), cluster_ids int32
 * [n_probes]; y[b, p * cluster_size + m] = row m of cluster cluster_ids[p]
 * dotted with x[b] -- the value ma_rtn4_gemv gives for that row, bit for bit.
 * x bf16 with 16-byte aligned rows; ids outside [0, n_clusters) are clamped.
 * Replaces rtn4_indexed_gemv, src/maple_run/kernels/rtn4.py:418-611.
 */
int ma_rtn4_indexed_gemv(const void* x, int x_dtype, int64_t batch, int64_t ldx,
                         const uint32_t* packed, int64_t n_clusters, int64_t cluster_size,
                         int64_t nwords, const void* scales, int scales_dtype, const void* biases,
                         int biases_dtype, int64_t group_size, const int32_t* cluster_ids,
                         int64_t n_probes, void* y, int64_t ldy, void* stream);

/* Workspace bytes of ma_flash_head (256-byte aligned): the centroid scores
 * and, when cluster_ids is NULL, the selected ids. */
size_t ma_flash_head_workspace_bytes(int64_t n_clusters, int64_t n_probes);

/*
 * FlashHead for one token x (bf16 [nwords * 8]): scores = the RTN4 GEMV of
 * the n_clusters centroid rows (bf16, as ma_rtn4_gemv stores them); the
 * n_probes highest-scoring clusters (equal scores: the lower cluster index;
 * written to cluster_ids in ascending order when it is not NULL); logits
 * (bf16 [vocab]) = -inf, then for every token of a probed cluster its exact
 * head logit at token_map[c * cluster_size + m] (head = the lm_head rows
 * permuted by token_map, [n_clusters, cluster_size, nwords]), and the n_force
 * forced tokens' exact logits (their own rows, force_ids int32).  The exact
 * logits are ma_rtn4_gemv's values bit for bit.  Four launches, no
 * allocation; n_clusters <= 8192.  Replaces FlashHead.__call__,
 * src/maple_run/flash_head.py:334-370 (centroid rtn4_gemv, torch.topk,
 * rtn4_indexed_gemv, the force rows, fill + index_put).
 */
int ma_flash_head(const void* x, const uint32_t* centroids, const void* c_scales,
                  const void* c_biases, int c_dtype, int64_t n_clusters, int64_t c_group,
                  const uint32_t* head, const void* h_scales, const void* h_biases, int h_dtype,
                  int64_t cluster_size, int64_t h_group, const int32_t* token_map,
                  int64_t n_probes, const uint32_t* force_w, const void* force_scales,
                  const void* force_biases, const int32_t* force_ids, int64_t n_force,
                  int64_t nwords, int64_t vocab, void* logits, int32_t* cluster_ids,
                  void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes ma_fused_sample needs for rows x vocab at top_k (0 for bad
 * sizes).  Replaces sampler_workspace / batched_sampler_workspace,
 * src/maple_run/kernels/sampler.py:202-232. */
size_t ma_sampler_workspace_bytes(int64_t rows, int64_t vocab, int top_k);

/*
 * Fused top-k / temperature / nucleus draw, one token per row: the top_k
 * largest logits of row r (bf16, fp16 or float32, row stride ld; descending,
 * ties at the lower index), p = exp((v - v_max) * inv_temperature) normalised
 * over them, tokens dropped once the mass before them exceeds top_p, then the
 * first token whose inclusive prefix of the kept p exceeds
 * uniform[r] * (kept mass); out int64 [rows].  Two launches; every row draws
 * exactly what it draws alone.  1 <= top_k <= min(64, vocab),
 * inv_temperature finite > 0, 0 < top_p <= 1, ceil(vocab / 4096) * top_k <=
 * 4096.  Replaces fused_sample / fused_sample_batched
 * (src/maple_run/kernels/sampler.py:106-199: _topk_partial_kernel :24-53,
 * _sample_final_kernel :56-103).
 */
int ma_fused_sample(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                    const float* uniform, int top_k, float inv_temperature, float top_p,
                    void* workspace, size_t ws_bytes, int64_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MAPLE_AMD_H */
