"""MoE FFN layer on the HIP kernels vs the CPU oracle (needs the GPU).

Shapes are the synthetic workloads: hidden 2048, 64 experts, intermediate
768, top-8; decode batch 1 (per-slot kernels) and 32 / 128 tokens with
Zipf(1.1)-skewed routing plus a 2048-token prefill chunk (dispatch + grouped
MFMA kernels).  Routing is checked against the oracle's (ids exact on rows
without float near-ties); the expert outputs against the oracle evaluated on
the kernel's own routing, with the reference's bf16 rounding points; the
dispatch lists exactly.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import assert_bf16_close, load_tv_distance, np_f, np_u32, tie_safe_rows, zipf_bias
from maple_amd import synthetic
from maple_amd.kernels import moe_dispatch, router_topk
from maple_amd.moe import GROUPED_MIN_TOKENS, moe_block, moe_grouped
from oracle import kernels as ok

pytestmark = pytest.mark.gpu

H, E, I, K = 2048, 64, 768, 8


@pytest.fixture(scope="module")
def layer(dev):
    return synthetic.make_moe_layer(H, E, I, seed=7, device=dev)


def _oracle_inputs(L):
    return (np_u32(L.up_gate_packed), np_f(L.up_gate_alpha), np_u32(L.down_packed), np_f(L.down_alpha))


def _check_routing(x, L, ids, wts, k=K):
    rid, rw, probs = ok.router_topk(np_f(x), np_f(L.gate_weight), k,
                                    bias=None if L.router_bias is None else np_f(L.router_bias))
    safe = tie_safe_rows(probs, k)
    assert safe.sum() >= len(safe) - max(1, len(safe) // 50), "too many near-tie rows for the check to mean much"
    np.testing.assert_array_equal(ids.cpu().numpy()[safe], rid[safe])
    np.testing.assert_allclose(wts.cpu().numpy()[safe], rw[safe], rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("tokens", [1, 2])
def test_moe_block_decode_vs_oracle(dev, layer, tokens):
    x = synthetic.randn_bf16((tokens, H), 100 + tokens, dev)
    res = synthetic.randn_bf16((tokens, H), 200 + tokens, dev)
    y, ids, wts = moe_block(x, layer, K, residual=res)
    torch.cuda.synchronize()
    _check_routing(x, layer, ids, wts)
    ref, _ = ok.moe_experts(np_f(x), ids.cpu().numpy(), wts.cpu().numpy(), *_oracle_inputs(layer),
                            residual=np_f(res))
    # two bf16 rounding points (h; each slot's down output in the oracle and
    # the one-launch kernel): the grouped path's 2^-7 absolute tolerance
    assert_bf16_close(np_f(y), ref, atol_frac=2.0 ** -7, what=f"moe bs{tokens}")


@pytest.mark.parametrize("tokens", [32, 128, 2048])
def test_moe_grouped_zipf_vs_oracle(dev, layer, tokens):
    assert tokens >= GROUPED_MIN_TOKENS
    L = synthetic.MoELayer(layer.gate_weight, layer.up_gate_packed, layer.up_gate_alpha,
                           layer.down_packed, layer.down_alpha, zipf_bias(dev))
    x = synthetic.randn_bf16((tokens, H), 300 + tokens, dev)
    ids, wts = router_topk(x, L.gate_weight, K, bias=L.router_bias)
    y, h = moe_grouped(x, L, ids, wts, return_h=True)
    torch.cuda.synchronize()
    _check_routing(x, L, ids, wts)
    idn, wn = ids.cpu().numpy(), wts.cpu().numpy()
    # the expert load follows the capped Zipf(1.1) target: total-variation
    # distance within what sampling leaves at this many pairs (a numpy
    # simulation of this router over random layers gives 99th percentiles
    # 0.18 / 0.09 / 0.024 at 32 / 128 / 2048 tokens), far from uniform routing
    tv = load_tv_distance(idn, E)
    assert tv <= {32: 0.25, 128: 0.13, 2048: 0.04}[tokens], f"load TV distance {tv:.3f}"
    assert load_tv_distance(np.arange(E).repeat(tokens * K // E), E) > 0.3
    if tokens == 2048:
        top2 = np.sort(np.bincount(idn.reshape(-1), minlength=E))[-2:] / idn.size
        assert (top2 >= 0.11).all() and (top2 <= 0.125).all(), top2  # the two capped ranks
    d = moe_dispatch(ids, E)
    c, o, p, inv = ok.dispatch(idn, E)
    np.testing.assert_array_equal(d.pair_ids.cpu().numpy(), p)
    np.testing.assert_array_equal(d.offsets.cpu().numpy(), o)
    np.testing.assert_array_equal(d.inverse.cpu().numpy(), inv)
    ref, href = ok.moe_experts(np_f(x), idn, wn, *_oracle_inputs(L))
    assert_bf16_close(np_f(h), href, what=f"h T={tokens}")
    for _ in range(2):  # every sum has a fixed order: the same bits on every run
        y2, h2 = moe_grouped(x, L, ids, wts, return_h=True)
        assert torch.equal(y2, y) and torch.equal(h2, h), f"T={tokens}: a second run differs"
    # y passes two bf16 rounding points (h and each slot's down output, as in
    # the reference), so an element may differ by sum_j w_j * ulp(out_j):
    # about one bf16 ulp of the output scale, whatever |y| itself is.
    assert_bf16_close(np_f(y), ref, atol_frac=2.0 ** -7, what=f"y T={tokens}")


@pytest.mark.parametrize("tokens", [256, 2048])
def test_router_pairs_equal_grouped_own_prep(dev, layer, tokens):
    """router_topk(pairs=True) writes x' from its top-k launch; moe_block's
    prefill path hands them to the grouped kernels: the same ids, weights, x'
    and y bits as router_topk + moe_grouped building x' itself."""
    L = synthetic.MoELayer(layer.gate_weight, layer.up_gate_packed, layer.up_gate_alpha,
                           layer.down_packed, layer.down_alpha, zipf_bias(dev))
    x = synthetic.randn_bf16((tokens, H), 700 + tokens, dev)
    ids, wts = router_topk(x, L.gate_weight, K, bias=L.router_bias)
    ids2, wts2, (xp, xc) = router_topk(x, L.gate_weight, K, bias=L.router_bias, pairs=True)
    assert torch.equal(ids, ids2) and torch.equal(wts, wts2)
    y_ref = moe_grouped(x, L, ids, wts)
    y_pairs = moe_grouped(x, L, ids2, wts2, x_pairs=(xp, xc))
    y_block, ids3, _ = moe_block(x, L, K, plan="grouped")
    torch.cuda.synchronize()
    assert torch.equal(y_pairs, y_ref) and torch.equal(y_block, y_ref) and torch.equal(ids3, ids)
    # x' against the oracle's pair form (word w, pair j: (f_j x[16w+j], f_j x[16w+j+8]))
    xf = np_f(x)[:4].reshape(4, -1, 2, 8)
    f = np.where(np.arange(8) % 2 == 1, 4.0, 16.0).astype(np.float32)
    lo, hi = (xf[:, :, 0, :] * f), (xf[:, :, 1, :] * f)
    got = xp[:4].cpu().numpy().reshape(4, -1, 8)
    np.testing.assert_array_equal(got & 0xFFFF, lo.astype(np.float32).view(np.uint32) >> 16)
    np.testing.assert_array_equal(got >> 16, hi.astype(np.float32).view(np.uint32) >> 16)


@pytest.mark.parametrize("hidden,n_exp,inter,k,tokens", [(3072, 8, 1024, 4, 96), (1024, 16, 512, 2, 200)])
def test_moe_grouped_prefill_form_other_shapes(dev, hidden, n_exp, inter, k, tokens):
    """The prefill-form grouped kernels (more than 16 pairs per expert: x'
    copied into LDS a K step ahead, 128-pair x 256-row tiles) at hidden sizes
    and expert widths other than the synthetic layer's (K loops of 24 / 8 /
    64 / 4 steps): h and y against the oracle on the kernel's own routing, and
    the same bits on a second run."""
    L = synthetic.make_moe_layer(hidden, n_exp, inter, seed=11, device=dev)
    assert tokens * k > 16 * n_exp  # the prefill form
    x = synthetic.randn_bf16((tokens, hidden), 500 + hidden, dev)
    ids, wts = router_topk(x, L.gate_weight, k)
    y, h = moe_grouped(x, L, ids, wts, return_h=True)
    torch.cuda.synchronize()
    idn, wn = ids.cpu().numpy(), wts.cpu().numpy()
    ref, href = ok.moe_experts(np_f(x), idn, wn, *_oracle_inputs(L))
    assert_bf16_close(np_f(h), href, what=f"h H={hidden} I={inter}")
    assert_bf16_close(np_f(y), ref, atol_frac=2.0 ** -7, what=f"y H={hidden} I={inter}")
    y2, h2 = moe_grouped(x, L, ids, wts, return_h=True)
    assert torch.equal(y2, y) and torch.equal(h2, h)


@pytest.mark.parametrize("tokens", [8, 32, 128])
def test_moe_layer_routed_pairs_vs_oracle(dev, layer, tokens):
    """The decoder's batched MoE half: one routing launch that also writes xn
    as x' pairs, then the tile-resident expert kernels reading those pairs
    (hidden 2048, intermediate 768), against the oracle on the same routing."""
    from maple_amd.moe import moe_layer
    L = synthetic.MoELayer(layer.gate_weight, layer.up_gate_packed, layer.up_gate_alpha,
                           layer.down_packed, layer.down_alpha, zipf_bias(dev))
    x = synthetic.randn_bf16((tokens, H), 600 + tokens, dev)
    add = synthetic.randn_bf16((tokens, H), 700 + tokens, dev)
    nw = synthetic.uniform_bf16((H,), 0.5, 1.5, 800, dev)
    y, ids = moe_layer(x, L, K, nw, 1e-6, add=add)
    from maple_amd.kernels import add_rms_norm
    h, xn = add_rms_norm(x, add, nw, 1e-6)
    ids2, wts = router_topk(xn, L.gate_weight, K, bias=L.router_bias)
    torch.cuda.synchronize()
    assert torch.equal(ids, ids2)
    idn, wn = ids.cpu().numpy(), wts.cpu().numpy()
    ref, _ = ok.moe_experts(np_f(xn), idn, wn, *_oracle_inputs(L), residual=np_f(h))
    assert_bf16_close(np_f(y), ref, atol_frac=2.0 ** -7, what=f"routed y T={tokens}")
    y2, _ = moe_layer(x, L, K, nw, 1e-6, add=add)
    assert torch.equal(y, y2)  # deterministic


def test_moe_block_grouped_matches_per_slot(dev, layer):
    """The two plans agree on the same routing (bf16 tolerance)."""
    x = synthetic.randn_bf16((16, H), 400, dev)
    res = synthetic.randn_bf16((16, H), 401, dev)
    ids, wts = router_topk(x, layer.gate_weight, K)
    yg = moe_grouped(x, layer, ids, wts, res)
    from maple_amd.kernels import ternary_expert_down_sum, ternary_expert_swiglu

    hs = ternary_expert_swiglu(x, layer.up_gate_packed, layer.up_gate_alpha, ids)
    ys = ternary_expert_down_sum(hs, layer.down_packed, layer.down_alpha, ids, wts, residual=res)
    assert_bf16_close(np_f(yg), np_f(ys), rtol=2 ** -7, atol_frac=2e-3, what="grouped vs per-slot")


def test_moe_block_graph_replays_match_eager(dev, layer):
    """Captured once, replayed three times with eager work in between."""
    x = synthetic.randn_bf16((1, H), 500, dev)
    y_eager, _, _ = moe_block(x, layer, K)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        moe_block(x, layer, K)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y_g, _, _ = moe_block(x, layer, K)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(y_g, y_eager, rtol=0, atol=0)
        moe_block(x, layer, K)  # eager work between replays
        torch.cuda.synchronize()
    from maple_amd.kernels.router import router_wait_timed_out

    assert not router_wait_timed_out(dev)


# ---------------------------------------------------------------- one-launch routing
@pytest.mark.parametrize("tokens,n_exp,hidden,with_add,nw_dtype,with_bias", [
    (4, 64, 2048, True, torch.float32, False),
    (32, 64, 2048, True, torch.bfloat16, True),
    (33, 64, 2048, False, torch.float32, False),
    (128, 256, 2048, True, torch.float32, True),
    (5, 20, 4096, True, torch.bfloat16, False),
    (1024, 64, 2048, True, torch.float32, False),
])
def test_moe_route_equals_separate_launches(dev, tokens, n_exp, hidden, with_add, nw_dtype, with_bias):
    """ma_moe_route gives, bit for bit, add_rms_norm (or rms_norm) +
    router_topk + moe_dispatch (router weights to float32 rounding where
    router_topk's one-launch form or its MFMA logits GEMM runs); its routing
    matches the oracle's; the
    workspace is left all-zero; called twice in a row (the ticket counter and
    the tagged logits are reused)."""
    from maple_amd.kernels import add_rms_norm, rms_norm
    from maple_amd import workspace
    from maple_amd.moe import moe_route, route_timed_out
    L = synthetic.make_moe_layer(hidden, n_exp, 256, seed=9, device=dev)
    if with_bias:
        L.router_bias = synthetic.zipf_router_bias(n_exp).to(dev)
    k = min(K, n_exp)
    x = synthetic.randn_bf16((tokens, hidden), 300 + tokens, dev)
    add = synthetic.randn_bf16((tokens, hidden), 400 + tokens, dev) if with_add else None
    g = torch.Generator(device=dev).manual_seed(500 + tokens)
    nw = (torch.rand(hidden, device=dev, generator=g) + 0.5).to(nw_dtype)
    for call in range(2):
        h, xn, ids, wts, d = moe_route(x, L, k, nw, 1e-6, add=add)
        if with_add:
            h_ref, xn_ref = add_rms_norm(x, add, nw, 1e-6)
        else:
            h_ref, xn_ref = x, rms_norm(x, nw, 1e-6)
        ids_ref, wts_ref = router_topk(xn_ref, L.gate_weight, k, bias=L.router_bias)
        d_ref = moe_dispatch(ids_ref, n_exp)
        torch.cuda.synchronize()
        assert torch.equal(h, h_ref) and torch.equal(xn, xn_ref), f"norm (call {call})"
        if tokens < 256:
            assert torch.equal(ids, ids_ref), f"router ids (call {call})"
        else:  # router_topk's MFMA logits GEMM sums in another order: equal ids
            # on the rows without a near-tie at the cut, and the same dispatch of
            # moe_route's own ids
            lg = np_f(xn_ref) @ np_f(L.gate_weight).T + (0 if L.router_bias is None else np_f(L.router_bias))
            pr = np.exp(lg - lg.max(-1, keepdims=True))
            safe = tie_safe_rows(pr / pr.sum(-1, keepdims=True), k)
            assert safe.mean() > 0.98
            np.testing.assert_array_equal(ids.cpu().numpy()[safe], ids_ref.cpu().numpy()[safe])
            d_ref = moe_dispatch(ids, n_exp)
        if 16 < tokens < 256:  # router_topk's two-launch form: the same float32 sums
            assert torch.equal(wts, wts_ref), f"router weights (call {call})"
        else:  # its one-launch form, and from 256 tokens its MFMA logits GEMM,
            # add each logit's products in another order
            sel = slice(None) if tokens < 256 else torch.from_numpy(safe).to(dev)
            torch.testing.assert_close(wts[sel], wts_ref[sel], rtol=1e-5, atol=1e-7)
        for a, b in zip(d, d_ref):
            assert torch.equal(a, b), f"dispatch (call {call})"
    assert not route_timed_out(dev)
    assert all(int(ws.count_nonzero()) == 0 for k, ws in workspace._POOL.items() if k[0] == "moe_route")
    if tokens <= 128:
        _check_routing(xn, L, ids, wts, k)


@pytest.mark.parametrize("tokens", [17, 32, 128])
def test_combine_in_front_of_next_gemv_equals_separate(dev, layer, tokens):
    """ma_ternary_gemv_combine_ws: the grouped MoE's combine run in the next
    RMS-folded GEMM's operand launch gives, bit for bit, the combined rows
    moe_grouped returns and the GEMM of those rows; twice in a row."""
    from maple_amd.kernels import ternary_gemv
    from maple_amd.kernels.ternary_gemv import combine_gemv_supported, ternary_gemv_combine
    from maple_amd.moe import PendingCombine, moe_layer
    x = synthetic.randn_bf16((tokens, H), 900 + tokens, dev)
    add = synthetic.randn_bf16((tokens, H), 950 + tokens, dev)
    nw = synthetic.uniform_bf16((H,), 0.5, 1.5, 960, dev)
    qkv_w, qkv_a = synthetic.ternary_linear(3072, H, 970, dev)
    rms = synthetic.uniform_bf16((H,), 0.5, 1.5, 980, dev)
    assert combine_gemv_supported(tokens, K, qkv_w)
    y_ref, ids_ref = moe_layer(x, layer, K, nw, 1e-6, add=add)
    q_ref = ternary_gemv(y_ref, qkv_w, qkv_a, rms_weight=rms, rms_eps=1e-6)
    for call in range(2):
        pend, ids = moe_layer(x, layer, K, nw, 1e-6, add=add, defer_combine=True)
        assert isinstance(pend, PendingCombine)
        y, q = ternary_gemv_combine(pend, qkv_w, qkv_a, rms_weight=rms, rms_eps=1e-6)
        torch.cuda.synchronize()
        assert torch.equal(ids, ids_ref)
        assert torch.equal(y, y_ref), f"combined rows (call {call})"
        assert torch.equal(q, q_ref), f"GEMM (call {call})"
