"""One-launch MoE layer (``ma_moe_fused``) vs the CPU oracle (needs the GPU).

Decode batch 1 at the synthetic shapes: hidden 2048, 64 experts,
intermediate 768, top-8 (plain, with residual, with a Zipf router bias, and
with the decoder's add + RMSNorm in front), and the small smoke shape (hidden
256, 8 experts, intermediate 128, top-2).  Routing is checked against the
oracle's own top-k (ids exact where the k-th and (k+1)-th probabilities are
separated), y against the oracle on the kernel's routing.  y passes two bf16
rounding points (h, and each slot's down output, as the reference stores
them), so an input near a rounding boundary can land one bf16 ulp of that
intermediate away: y's absolute tolerance is 2^-7 of its scale (as for the
grouped path), the relative bound 1e-2 as everywhere.  Many consecutive
calls on one workspace (each call tags its data with a new generation), graph
replays equal to eager calls, and no cross-workgroup wait ever timing out.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import assert_bf16_close, np_f, np_u32, tie_safe_rows, zipf_bias
from maple_amd import synthetic
from maple_amd.kernels import ternary_gemv
from maple_amd.moe import moe_block, moe_fused, moe_fused_timed_out
from oracle import kernels as ok

pytestmark = pytest.mark.gpu


Y_ATOL = 2.0 ** -7


def _oracle(x, L, ids, wts, k, residual=None):
    rid, rw, probs = ok.router_topk(x, np_f(L.gate_weight), k,
                                    bias=None if L.router_bias is None else np_f(L.router_bias))
    safe = tie_safe_rows(probs, k)
    idn, wn = ids.cpu().numpy(), wts.cpu().numpy()
    np.testing.assert_array_equal(idn[safe], rid[safe])
    np.testing.assert_allclose(wn[safe], rw[safe], rtol=1e-4, atol=1e-6)
    y, _ = ok.moe_experts(x, idn, wn, np_u32(L.up_gate_packed), np_f(L.up_gate_alpha),
                          np_u32(L.down_packed), np_f(L.down_alpha), residual=residual)
    return y


@pytest.fixture(scope="module")
def layers(dev):
    return [synthetic.make_moe_layer(2048, 64, 768, seed=40 + i, device=dev) for i in range(3)]


@pytest.mark.parametrize("with_res", [False, True])
def test_fused_plain_vs_oracle(dev, layers, with_res):
    for step in range(4):  # consecutive calls over different layers
        L = layers[step % len(layers)]
        x = synthetic.randn_bf16((1, 2048), 500 + step, dev)
        res = synthetic.randn_bf16((1, 2048), 600 + step, dev) if with_res else None
        y, ids, wts = moe_fused(x, L, 8, res)
        torch.cuda.synchronize()
        ref = _oracle(np_f(x), L, ids, wts, 8, None if res is None else np_f(res))
        assert_bf16_close(np_f(y), ref, atol_frac=Y_ATOL, what=f"fused step {step}")
    assert not moe_fused_timed_out(dev)


def test_fused_float32_alphas_vs_oracle(dev, layers):
    """Row scales in float32 (as a converted checkpoint holds them) with
    values bf16 cannot represent: read unrounded, against the oracle."""
    L0 = layers[2]
    g = torch.Generator(device=dev).manual_seed(3)
    ua = torch.rand(L0.up_gate_alpha.shape, device=dev, generator=g) * 0.04 + 0.01
    da = torch.rand(L0.down_alpha.shape, device=dev, generator=g) * 0.04 + 0.01
    L = synthetic.MoELayer(L0.gate_weight, L0.up_gate_packed, ua, L0.down_packed, da)
    assert not torch.equal(ua, ua.bfloat16().float())
    from maple_amd.moe import fused_supported
    for step in range(2):
        x = synthetic.randn_bf16((1, 2048), 750 + step, dev)
        assert fused_supported(L, 8, x)
        y, ids, wts = moe_block(x, L, 8, plan="fused")
        torch.cuda.synchronize()
        assert_bf16_close(np_f(y), _oracle(np_f(x), L, ids, wts, 8), atol_frac=Y_ATOL, what=f"f32 alphas {step}")
        y_bf, _, _ = moe_block(x, synthetic.MoELayer(L0.gate_weight, L0.up_gate_packed, ua.bfloat16(),
                                                     L0.down_packed, da.bfloat16()), 8, plan="fused")
        assert not torch.equal(y, y_bf)  # the float32 values were used, not rounded ones
    assert not moe_fused_timed_out(dev)


def test_fused_zipf_bias_vs_oracle(dev, layers):
    L0 = layers[0]
    L = synthetic.MoELayer(L0.gate_weight, L0.up_gate_packed, L0.up_gate_alpha, L0.down_packed,
                           L0.down_alpha, zipf_bias(dev))
    for step in range(3):
        x = synthetic.randn_bf16((1, 2048), 700 + step, dev)
        y, ids, wts = moe_block(x, L, 8, plan="fused")
        torch.cuda.synchronize()
        assert_bf16_close(np_f(y), _oracle(np_f(x), L, ids, wts, 8), atol_frac=Y_ATOL, what=f"zipf step {step}")


def test_fused_add_norm_vs_oracle(dev, layers):
    L = layers[1]
    a = synthetic.randn_bf16((1, 2048), 801, dev)
    b = synthetic.randn_bf16((1, 2048), 802, dev, std=0.5)
    w = torch.rand(2048, device=dev) + 0.5
    y, ids, wts = moe_fused(a, L, 8, add=b, norm_weight=w, eps=1e-6)
    torch.cuda.synchronize()
    s = np_f(a) + np_f(b)
    res = ok.bf16_round(s).astype(np.float64)
    x = ok.bf16_round(ok.rms_norm(s, np_f(w), 1e-6)).astype(np.float64)
    assert_bf16_close(np_f(y), _oracle(x, L, ids, wts, 8, res), atol_frac=Y_ATOL, what="add+norm")


def test_fused_small_shape_vs_oracle(dev):
    L = synthetic.make_moe_layer(256, 8, 128, seed=9, device=dev)
    for step in range(3):
        x = synthetic.randn_bf16((1, 256), 900 + step, dev)
        y, ids, wts = moe_fused(x, L, 2)
        torch.cuda.synchronize()
        assert_bf16_close(np_f(y), _oracle(np_f(x), L, ids, wts, 2), atol_frac=Y_ATOL, what=f"small {step}")


def test_fused_agrees_with_per_slot_plan(dev, layers):
    L = layers[2]
    x = synthetic.randn_bf16((1, 2048), 1001, dev)
    y1, i1, w1 = moe_block(x, L, 8, plan="fused")
    y2, i2, w2 = moe_block(x, L, 8, plan="per_slot")
    torch.cuda.synchronize()
    assert torch.equal(i1, i2)
    torch.testing.assert_close(w1, w2, rtol=1e-6, atol=1e-7)
    assert_bf16_close(np_f(y1), np_f(y2), atol_frac=Y_ATOL, what="fused vs per-slot")


def test_fused_graph_replays_match_eager(dev, layers):
    xs = [synthetic.randn_bf16((1, 2048), 1100 + i, dev) for i in range(6)]
    eager = [moe_fused(xs[i], layers[i % 3], 8)[0].clone() for i in range(6)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        [moe_fused(xs[i], layers[i % 3], 8) for i in range(6)]
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = [moe_fused(xs[i], layers[i % 3], 8)[0] for i in range(6)]
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        for i in range(6):
            assert torch.equal(outs[i], eager[i]), f"replay {rep} layer {i}"
        torch.zeros(1, device=dev).add_(1)  # eager work between replays
    assert not moe_fused_timed_out(dev)


def _next_linear(n_out, hidden, seed, dev):
    packed, alpha = synthetic.ternary_linear(n_out, hidden, seed, dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    rms = torch.rand(hidden, device=dev, generator=g) + 0.5
    return packed, alpha, rms, 1e-6


@pytest.mark.parametrize("with_add", [False, True])
def test_fused_next_projection_equals_gemv(dev, layers, with_add):
    """The next layer's RMS-folded projection computed in the same launch
    gives the bits of ternary_gemv on the launch's own y (2560 rows, the
    synthetic decoder's QKV), over consecutive calls."""
    nl = _next_linear(2560, 2048, 77, dev)
    for step in range(3):
        L = layers[step % len(layers)]
        x = synthetic.randn_bf16((1, 2048), 1200 + step, dev)
        kw = {}
        if with_add:
            kw = dict(add=synthetic.randn_bf16((1, 2048), 1300 + step, dev, std=0.5),
                      norm_weight=torch.rand(2048, device=dev) + 0.5)
        y, ids, wts, q = moe_fused(x, L, 8, next_linear=nl, **kw)
        y0, _, _ = moe_fused(x, L, 8, **kw)
        ref = ternary_gemv(y, nl[0], nl[1], rms_weight=nl[2], rms_eps=nl[3])
        torch.cuda.synchronize()
        assert torch.equal(y, y0), f"y changed by the tail, step {step}"
        assert torch.equal(q, ref), f"next projection, step {step}"
    assert not moe_fused_timed_out(dev)


def test_fused_next_projection_small_shape(dev):
    L = synthetic.make_moe_layer(256, 8, 128, seed=19, device=dev)
    nl = _next_linear(512, 256, 78, dev)
    for step in range(2):
        x = synthetic.randn_bf16((1, 256), 1400 + step, dev)
        y, _, _, q = moe_fused(x, L, 2, next_linear=nl)
        ref = ternary_gemv(y, nl[0], nl[1], rms_weight=nl[2], rms_eps=nl[3])
        torch.cuda.synchronize()
        assert torch.equal(q, ref), f"small next projection, step {step}"


def test_fused_next_projection_graph_replays(dev, layers):
    nl = _next_linear(2560, 2048, 79, dev)
    xs = [synthetic.randn_bf16((1, 2048), 1500 + i, dev) for i in range(3)]
    eager = [moe_fused(xs[i], layers[i], 8, next_linear=nl)[3].clone() for i in range(3)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        [moe_fused(xs[i], layers[i], 8, next_linear=nl) for i in range(3)]
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = [moe_fused(xs[i], layers[i], 8, next_linear=nl)[3] for i in range(3)]
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        for i in range(3):
            assert torch.equal(outs[i], eager[i]), f"replay {rep} layer {i}"
        torch.zeros(1, device=dev).add_(1)  # eager work between replays
    assert not moe_fused_timed_out(dev)


def test_fused_rejects_unbuilt_shape(dev):
    L = synthetic.make_moe_layer(512, 8, 256, seed=1, device=dev)
    with pytest.raises(ValueError):
        moe_fused(synthetic.randn_bf16((1, 512), 1, dev), L, 2)


@pytest.mark.parametrize("inter", [768, 512])
def test_fused_forms_vs_oracle_on_one_workspace(dev, monkeypatch, inter):
    """Both forms of the one-launch layer (the XCD split and the one-barrier
    grid, forced by MAPLE_AMD_MOE_FUSED=grid) against the oracle, alternating
    on one workspace (each form's tags must survive the other's calls), and
    against each other: the same ids on tie-safe rows, y within the bar."""
    from maple_amd.moe import fused_form

    Ls = [synthetic.make_moe_layer(2048, 64, inter, seed=70 + i, device=dev) for i in range(2)]
    assert fused_form(Ls[0], 8) == 1, "the XCD split is expected on an 8-XCD MI355X"
    outs = {}
    for step in range(6):
        form = "grid" if step % 2 else "xcd"
        if form == "grid":
            monkeypatch.setenv("MAPLE_AMD_MOE_FUSED", "grid")
            assert fused_form(Ls[0], 8) == 0
        else:
            monkeypatch.delenv("MAPLE_AMD_MOE_FUSED", raising=False)
        L = Ls[(step // 2) % 2]
        x = synthetic.randn_bf16((1, 2048), 800 + step // 2, dev)
        res = synthetic.randn_bf16((1, 2048), 900 + step // 2, dev)
        y, ids, wts = moe_fused(x, L, 8, res)
        torch.cuda.synchronize()
        ref = _oracle(np_f(x), L, ids, wts, 8, np_f(res))
        assert_bf16_close(np_f(y), ref, atol_frac=Y_ATOL, what=f"{form} I{inter} step {step}")
        outs.setdefault(step // 2, {})[form] = (y, ids, wts)
    monkeypatch.delenv("MAPLE_AMD_MOE_FUSED", raising=False)
    for k, pair in outs.items():
        (y1, i1, w1), (y2, i2, w2) = pair["xcd"], pair["grid"]
        x = synthetic.randn_bf16((1, 2048), 800 + k, dev)
        _, _, probs = ok.router_topk(np_f(x), np_f(Ls[k % 2].gate_weight), 8)
        if not tie_safe_rows(probs, 8).all():
            continue  # a near-tie may order the two forms' experts differently
        assert torch.equal(i1, i2), f"pair {k}: ids"
        torch.testing.assert_close(w1, w2, rtol=1e-5, atol=1e-7)
        assert_bf16_close(np_f(y1), np_f(y2), atol_frac=Y_ATOL, what=f"xcd vs grid {k}")
    assert not moe_fused_timed_out(dev)


def test_fused_forms_next_projection_on_one_workspace(dev, monkeypatch, layers):
    """The next projection in the launch gives ternary_gemv's bits on the
    launch's y in both forms (the XCD form hands y to each XCD's workgroups
    through that XCD's L2, the one-barrier form through memory after a grid
    barrier), with calls of either form, with and without the projection,
    interleaved on one workspace (the XCD form's copies of y are written only
    by calls with a projection, so a later one must not take an older copy)."""
    from maple_amd.moe import fused_form

    nl = _next_linear(2560, 2048, 81, dev)
    seq = [("xcd", True), ("xcd", False), ("grid", True), ("xcd", True), ("xcd", False), ("xcd", True),
           ("grid", False), ("xcd", True)]
    for step, (form, proj) in enumerate(seq):
        if form == "grid":
            monkeypatch.setenv("MAPLE_AMD_MOE_FUSED", "grid")
        else:
            monkeypatch.delenv("MAPLE_AMD_MOE_FUSED", raising=False)
        assert fused_form(layers[0], 8) == (1 if form == "xcd" else 0)
        L = layers[step % len(layers)]
        x = synthetic.randn_bf16((1, 2048), 1600 + step, dev)
        res = synthetic.randn_bf16((1, 2048), 1700 + step, dev)
        if proj:
            y, ids, wts, q = moe_fused(x, L, 8, res, next_linear=nl)
            ref = ternary_gemv(y, nl[0], nl[1], rms_weight=nl[2], rms_eps=nl[3])
        else:
            y, ids, wts = moe_fused(x, L, 8, res)
        torch.cuda.synchronize()
        assert_bf16_close(np_f(y), _oracle(np_f(x), L, ids, wts, 8, np_f(res)), atol_frac=Y_ATOL,
                          what=f"{form} step {step}")
        if proj:
            assert torch.equal(q, ref), f"{form} next projection, step {step}"
    monkeypatch.delenv("MAPLE_AMD_MOE_FUSED", raising=False)
    assert not moe_fused_timed_out(dev)


@pytest.mark.parametrize("alpha_dtype", [torch.bfloat16, torch.float32])
def test_fused_o_projection_equals_two_launches(dev, alpha_dtype):
    """moe_fused(..., o_linear=(attn, W_o, alpha_o)) -- the attention's output
    projection computed by every XCD in the MoE launch -- gives the bits of
    ternary_gemv followed by moe_fused(..., add=o): y, ids, weights and the
    next projection, over consecutive calls interleaved with plain calls on
    one workspace."""
    from maple_amd.moe import fused_form

    Ls = [synthetic.make_moe_layer(2048, 64, 768, seed=120 + i, device=dev) for i in range(2)]
    if alpha_dtype == torch.float32:
        for L in Ls:
            L.up_gate_alpha = L.up_gate_alpha.float()
            L.down_alpha = L.down_alpha.float()
    assert fused_form(Ls[0], 8) == 1, "the XCD split is expected on an 8-XCD MI355X"
    wo, ao = synthetic.ternary_linear(2048, 2048, 131, dev)
    ao = ao.to(alpha_dtype)
    nl = _next_linear(2560, 2048, 132, dev)
    nl = (nl[0], nl[1].to(alpha_dtype), nl[2], nl[3])
    w = torch.rand(2048, device=dev) + 0.5
    for step in range(6):
        L = Ls[step % 2]
        x = synthetic.randn_bf16((1, 2048), 1800 + step, dev)
        attn = synthetic.randn_bf16((1, 2048), 1900 + step, dev)
        proj = step % 3 != 2
        o = ternary_gemv(attn, wo, ao)
        ref = moe_fused(x, L, 8, add=o, norm_weight=w, eps=1e-6, next_linear=nl if proj else None)
        got = moe_fused(x, L, 8, norm_weight=w, eps=1e-6, next_linear=nl if proj else None,
                        o_linear=(attn, wo, ao))
        moe_fused(x, L, 8)  # a plain call between
        torch.cuda.synchronize()
        assert len(got) == len(ref)
        for k, (a, b) in enumerate(zip(got, ref)):
            assert torch.equal(a, b), f"step {step} output {k}"
    assert not moe_fused_timed_out(dev)


_FIRST_CALL_CAPTURED = r"""
import os, sys, torch
sys.path.insert(0, sys.argv[1])
import __graft_entry__ as ge
ge.load_package()
from maple_amd import synthetic
from maple_amd.moe import moe_fused, fused_form, moe_fused_timed_out
dev = torch.device("cuda:0")
L = synthetic.make_moe_layer(2048, 64, 768, seed=91, device=dev)
x = synthetic.randn_bf16((1, 2048), 92, dev)
torch.cuda.synchronize()
s = torch.cuda.Stream()
with torch.cuda.stream(s):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):          # the process's first ma_moe_fused call
        y, ids, wts = moe_fused(x, L, 8)
    outs = []
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        outs.append(y.clone())
form = fused_form(L, 8)                          # the probe runs now, outside capture
os.environ["MAPLE_AMD_MOE_FUSED"] = "grid"
y_grid, ids_grid, _ = moe_fused(x, L, 8)
torch.cuda.synchronize()
assert all(torch.equal(o, y_grid) for o in outs), "captured call != eager one-barrier form"
assert torch.equal(ids, ids_grid)
assert not moe_fused_timed_out(dev)
print("FORM", form)
"""


def test_first_call_inside_graph_capture(dev):
    """The XCD form's one-time probe synchronises, so it cannot run under graph
    capture: a process whose first one-launch call is captured gets the
    one-barrier form in the graph (the same bits as that form eagerly), and
    the probe runs at the first call outside capture."""
    import subprocess
    import sys
    from pathlib import Path

    root = str(Path(__file__).resolve().parents[1])
    res = subprocess.run([sys.executable, "-c", _FIRST_CALL_CAPTURED, root], capture_output=True, text=True,
                         timeout=300)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-3000:]
    assert "FORM 1" in res.stdout, res.stdout[-2000:]


def test_prefetch_is_only_a_hint(dev, layers):
    """Reading the next layer's router ahead (prefetch) leaves every output
    bit unchanged, in both forms' launcher; a misaligned range is refused."""
    for step in range(3):
        L, nxt = layers[step % 3], layers[(step + 1) % 3]
        x = synthetic.randn_bf16((1, 2048), 800 + step, dev)
        a = moe_fused(x, L, 8)
        b = moe_fused(x, L, 8, prefetch=nxt.gate_weight)
        c = moe_fused(x, L, 8, prefetch=nxt.up_gate_packed.view(torch.int32)[0, :4096])  # a partial range
        torch.cuda.synchronize()
        for u, v, w in zip(a, b, c):
            assert torch.equal(u, v) and torch.equal(u, w)
    with pytest.raises(ValueError, match="aligned"):
        moe_fused(x, layers[0], 8, prefetch=layers[1].gate_weight.reshape(-1)[1:])
    assert not moe_fused_timed_out(dev)


def test_bounded_waits_end_the_call_and_spare_the_layout_word(dev, layers, monkeypatch):
    """The XCD form's waits end at their bound (200 us after the launch's
    start; here 0, MAPLE_AMD_WAIT_BOUND_US, so that every wait that has to
    wait at all runs out): the call returns at once with its error word set,
    and, every workgroup having taken its slot, without the layout word; the
    timeout check zeroes the workspace again, keeps the XCD forms on, and the
    next call is right."""
    import time

    from maple_amd import workspace
    from maple_amd.moe import LAYOUT_WORD, fused_form

    L = layers[0]
    if fused_form(L, 8) != 1:
        pytest.skip("the XCD-split form does not run on this device")
    x = synthetic.randn_bf16((1, 2048), 900, dev)
    y0 = moe_fused(x, L, 8)
    torch.cuda.synchronize()
    key = ("moe_fused", dev.index or 0, torch.cuda.current_stream(dev).cuda_stream, 2048, L.inter, 8)
    ws = workspace._POOL[key].view(torch.int32)
    monkeypatch.setenv("MAPLE_AMD_WAIT_BOUND_US", "0")
    t0 = time.perf_counter()
    moe_fused(x, L, 8)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    monkeypatch.delenv("MAPLE_AMD_WAIT_BOUND_US")
    assert elapsed < 0.05
    assert int(ws[workspace.TIMEOUT_WORD["moe_fused"]].item()) == 1 and int(ws[LAYOUT_WORD].item()) == 0
    with pytest.raises(RuntimeError, match="moe_fused") as ei:
        workspace.check_timeouts(dev)
    assert "XCD-split forms are now off" not in str(ei.value)
    assert fused_form(L, 8) == 1
    y1 = moe_fused(x, L, 8)
    torch.cuda.synchronize()
    for a, b in zip(y0, y1):
        assert torch.equal(a, b)
    assert not moe_fused_timed_out(dev)
