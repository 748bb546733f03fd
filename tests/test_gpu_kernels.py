"""HIP kernels vs the CPU oracle on seeded inputs (needs the GPU).

Tolerances: bf16 outputs within one bf16 ulp (2^-8 relative) plus 1e-3 of the
output scale of the float64 oracle evaluated on the same bf16 inputs, and max
relative error <= 1e-2; float32 outputs rtol/atol 1e-4 (the reference's own
float32 tolerance, tests/test_ternary_gemv.py:91).  Integer outputs (unpacked
values, top-k ids away from float ties, dispatch lists) are compared exactly.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import assert_bf16_close, assert_f32_close, np_f, np_u32, tie_safe_rows
from maple_amd import synthetic
from maple_amd.kernels import (
    add_rms_norm,
    moe_dispatch,
    moe_reduce_add,
    rms_norm,
    router_topk,
    rtn4_embedding,
    rtn4_gemv,
    ternary_expert_down_sum,
    ternary_expert_gemv,
    ternary_expert_swiglu,
    ternary_gemv,
)
from oracle import kernels as ok
from oracle import pack

pytestmark = pytest.mark.gpu


def _u32(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(dev).view(torch.uint32)


# ---------------------------------------------------------------- ternary GEMV
def test_gemv_reference_kat(dev):
    """tests/test_ternary_gemv.py:114-132: LSB-first codes, code 2 -> +a, code 0 -> -a."""
    codes = np.ones((2, 128), np.uint32)
    codes[0, 0] = 2
    codes[1, 1] = 0
    w = _u32(pack.pack_2bit(codes), dev)
    alpha = torch.tensor([0.5, 1.25], device=dev)
    x = torch.arange(128, device=dev, dtype=torch.float32)
    y = ternary_gemv(x, w, alpha)
    assert_f32_close(np_f(y), [0.0, -1.25], rtol=0, atol=1e-6)
    yb = ternary_gemv(x.bfloat16(), w, alpha)  # bf16 fast path: same answer
    assert_f32_close(np_f(yb), [0.0, -1.25], rtol=0, atol=1e-6)


@pytest.mark.parametrize("n_out,k_in", [(1536, 2048), (2560, 2048), (2048, 768), (96, 128), (64, 256),
                                        (33, 512), (40, 4096), (17, 2560)])
def test_gemv_bf16_batch1_vs_oracle(dev, n_out, k_in):
    w = synthetic.ternary_packed((n_out, k_in), 11, dev)
    alpha = synthetic.uniform_bf16((n_out,), 0.01, 0.05, 12, dev)
    x = synthetic.randn_bf16((1, k_in), 13, dev)
    y = ternary_gemv(x, w, alpha)
    assert y.shape == (1, n_out) and y.dtype == torch.bfloat16
    ref = ok.ternary_gemv(np_f(x), np_u32(w), np_f(alpha))
    assert_bf16_close(np_f(y), ref, what=f"gemv {n_out}x{k_in}")


def test_gemv_code3_is_plus_two(dev):
    """Code 3 (never produced by ternarize) reads as +2 (ternary_gemv.py:126-128)."""
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 4, (64, 2048), dtype=np.uint32)
    w = _u32(pack.pack_2bit(codes), dev)
    alpha = torch.rand(64, device=dev) + 0.5
    x = synthetic.randn_bf16((1, 2048), 3, dev)
    ref = ok.ternary_gemv(np_f(x), pack.pack_2bit(codes), np_f(alpha))
    assert_bf16_close(np_f(ternary_gemv(x, w, alpha)), ref, what="code3 bf16")
    assert_f32_close(np_f(ternary_gemv(x.float(), w, alpha)), ref, rtol=1e-4, atol=1e-3, what="code3 f32")


@pytest.mark.parametrize("batch", [2, 3, 4, 8, 17, 32])
def test_gemv_bf16_batched_vs_oracle(dev, batch):
    w = synthetic.ternary_packed((512, 2048), 21, dev)
    alpha = synthetic.uniform_bf16((512,), 0.01, 0.05, 22, dev)
    x = synthetic.randn_bf16((batch, 2048), 23, dev)
    y = ternary_gemv(x, w, alpha)
    assert_bf16_close(np_f(y), ok.ternary_gemv(np_f(x), np_u32(w), np_f(alpha)), what=f"B={batch}")
    rows = torch.cat([ternary_gemv(x[i:i + 1], w, alpha) for i in range(batch)])
    torch.testing.assert_close(y, rows, rtol=8e-3, atol=8e-3)


@pytest.mark.parametrize("batch", [1, 2, 8, 32])
def test_gemv_fused_rms_vs_oracle(dev, batch):
    w = synthetic.ternary_packed((2560, 2048), 31, dev)
    alpha = synthetic.uniform_bf16((2560,), 0.01, 0.05, 32, dev)
    x = synthetic.randn_bf16((batch, 2048), 33, dev)
    rms_w = torch.rand(2048, device=dev) + 0.5
    y = ternary_gemv(x, w, alpha, rms_weight=rms_w, rms_eps=1e-6)
    ref = ok.ternary_gemv(np_f(x), np_u32(w), np_f(alpha), rms_weight=np_f(rms_w), rms_eps=1e-6)
    assert_bf16_close(np_f(y), ref, what=f"rms B={batch}")


@pytest.mark.parametrize("batch", [1, 4])
def test_gemv_fp32_activations_and_packed_kn(dev, batch):
    rng = np.random.default_rng(7)
    wf = rng.standard_normal((96, 256)).astype(np.float32)
    packed, alpha = pack.ternarize(wf)
    w = _u32(packed, dev)
    a = torch.from_numpy(alpha).to(dev)
    x = torch.from_numpy(rng.standard_normal((batch, 256)).astype(np.float32)).to(dev)
    ref = ok.ternary_gemv(np_f(x), packed, alpha)
    assert_f32_close(np_f(ternary_gemv(x, w, a)), ref, what="fp32 nk")
    w_kn = _u32(np.ascontiguousarray(packed.T), dev)
    assert_f32_close(np_f(ternary_gemv(x, w_kn, a, packed_kn=True)), ref, what="fp32 kn")
    xb = x.bfloat16()
    refb = ok.ternary_gemv(np_f(xb), packed, alpha)
    assert_bf16_close(np_f(ternary_gemv(xb, w_kn, a, packed_kn=True)), refb, what="bf16 kn")


def test_gemv_1d_x_and_empty_batch(dev):
    w = synthetic.ternary_packed((48, 128), 41, dev)
    alpha = torch.rand(48, device=dev)
    x = synthetic.randn_bf16((128,), 42, dev)
    y = ternary_gemv(x, w, alpha)
    assert y.shape == (48,)
    assert_bf16_close(np_f(y), ok.ternary_gemv(np_f(x), np_u32(w), np_f(alpha)), what="1d")
    assert ternary_gemv(x[None][:0], w, alpha).shape == (0, 48)


def test_gemv_rejects_non_uint32(dev):
    with pytest.raises(TypeError, match="uint32"):
        ternary_gemv(torch.randn(128, device=dev), torch.randn(16, 8, device=dev).bfloat16(),
                     torch.ones(16, device=dev))


# ---------------------------------------------------------------- router
@pytest.mark.parametrize("tokens,n_exp,top_k", [(1, 64, 8), (32, 64, 8), (128, 64, 8), (2048, 64, 8),
                                                (3, 4, 2), (5, 256, 8)])
def test_router_vs_oracle(dev, tokens, n_exp, top_k):
    gw = synthetic.randn_bf16((n_exp, 2048), 51, dev, std=0.02)
    x = synthetic.randn_bf16((tokens, 2048), 52, dev)
    ids, wts = router_topk(x, gw, top_k)
    assert ids.dtype == torch.int32 and wts.dtype == torch.float32
    rid, rw, probs = ok.router_topk(np_f(x), np_f(gw), top_k)
    safe = tie_safe_rows(probs, top_k)
    assert safe.mean() > 0.98, f"too many near-ties ({(~safe).sum()})"
    np.testing.assert_array_equal(ids.cpu().numpy()[safe], rid[safe])
    np.testing.assert_allclose(wts.cpu().numpy()[safe], rw[safe], rtol=1e-4, atol=1e-6)


def test_router_ties_and_bias(dev):
    gw = torch.zeros(6, 64, device=dev, dtype=torch.bfloat16)
    gw[4, 0] = gw[2, 0] = 1.0
    x = torch.zeros(1, 64, device=dev, dtype=torch.bfloat16)
    x[0, 0] = 1.0
    ids, wts = router_topk(x, gw, 4)
    assert ids[0].tolist() == [2, 4, 0, 1]
    bias = torch.tensor([0, 0, 0, 0, 0, 5.0], device=dev)
    ids, _ = router_topk(x, gw, 2, bias=bias)
    assert ids[0].tolist() == [5, 2]


# ---------------------------------------------------------------- dispatch
# Beyond 4096 pairs (up to 256 experts) the lists are placed by several
# workgroups, 2048 pairs each: ragged last chunks and 512 experts (one
# workgroup) are covered too.
@pytest.mark.parametrize("tokens,top_k,n_exp", [(1, 8, 64), (32, 8, 64), (128, 8, 64), (2048, 8, 64),
                                                (7, 3, 5), (0, 8, 64), (1000, 8, 256), (700, 7, 64),
                                                (2500, 8, 200), (4096, 8, 512), (512, 8, 64), (513, 8, 64)])
def test_dispatch_bit_exact(dev, tokens, top_k, n_exp):
    g = torch.Generator(device=dev).manual_seed(tokens * 7 + n_exp)
    ids = torch.randint(0, n_exp, (tokens, top_k), generator=g, device=dev, dtype=torch.int32)
    d = moe_dispatch(ids, n_exp)
    c, o, p, inv = ok.dispatch(ids.cpu().numpy(), n_exp)
    np.testing.assert_array_equal(d.counts.cpu().numpy(), c)
    np.testing.assert_array_equal(d.offsets.cpu().numpy(), o)
    np.testing.assert_array_equal(d.pair_ids.cpu().numpy(), p)
    np.testing.assert_array_equal(d.inverse.cpu().numpy(), inv)


@pytest.mark.parametrize("tokens", [300, 1200])
def test_dispatch_skewed_int64(dev, tokens):
    """All pairs on one expert plus a few singletons, int64 ids (one
    workgroup, and several)."""
    ids = torch.full((tokens, 8), 17, device=dev, dtype=torch.int64)
    ids[5, 3] = 0
    ids[tokens - 1, 7] = 63
    d = moe_dispatch(ids, 64)
    c, o, p, inv = ok.dispatch(ids.cpu().numpy(), 64)
    np.testing.assert_array_equal(d.pair_ids.cpu().numpy(), p)
    np.testing.assert_array_equal(d.offsets.cpu().numpy(), o)
    np.testing.assert_array_equal(d.counts.cpu().numpy(), c)
    np.testing.assert_array_equal(d.inverse.cpu().numpy(), inv)


# ---------------------------------------------------------------- experts
def _experts(dev, n_exp=8, hidden=2048, inter=768, seed=0):
    return synthetic.make_moe_layer(hidden=hidden, n_experts=n_exp, inter=inter, seed=seed, device=dev)


@pytest.mark.parametrize("tokens,top_k", [(1, 8), (3, 2), (32, 8)])
def test_expert_swiglu_vs_oracle(dev, tokens, top_k):
    L = _experts(dev)
    x = synthetic.randn_bf16((tokens, 2048), 61, dev)
    g = torch.Generator(device=dev).manual_seed(62)
    ids = torch.stack([torch.randperm(8, generator=g, device=dev)[:top_k] for _ in range(tokens)]).int()
    h = ternary_expert_swiglu(x, L.up_gate_packed, L.up_gate_alpha, ids)
    assert h.shape == (tokens, top_k, 768) and h.dtype == torch.bfloat16
    ref = ok.ternary_expert_swiglu(np_f(x), np_u32(L.up_gate_packed), np_f(L.up_gate_alpha), ids.cpu().numpy())
    assert_bf16_close(np_f(h), ref, what="swiglu")


@pytest.mark.parametrize("per_slot", [True, False])
def test_expert_gemv_vs_oracle(dev, per_slot):
    L = _experts(dev)
    ids = torch.tensor([[0, 3], [5, 5], [7, 1]], device=dev, dtype=torch.int32)
    k = 768
    x = synthetic.randn_bf16((3, 2, k) if per_slot else (3, k), 71, dev)
    y = ternary_expert_gemv(x, L.down_packed, L.down_alpha, ids)
    ref = ok.ternary_expert_gemv(np_f(x), np_u32(L.down_packed), np_f(L.down_alpha), ids.cpu().numpy())
    assert_bf16_close(np_f(y), ref, what="expert gemv")


def test_expert_kernels_fp32_generic_path(dev):
    """fp32 activations take the generic kernels; reference tolerance 1e-4."""
    rng = np.random.default_rng(3)
    n_exp, hidden, inter = 4, 128, 128
    up, up_a = pack.ternarize(rng.standard_normal((n_exp, inter, hidden)).astype(np.float32))
    gt, gt_a = pack.ternarize(rng.standard_normal((n_exp, inter, hidden)).astype(np.float32))
    dn, dn_a = pack.ternarize(rng.standard_normal((n_exp, hidden, inter)).astype(np.float32))
    ug = np.concatenate([up, gt], axis=1)
    ug_a = np.concatenate([up_a, gt_a], axis=1)
    x = rng.standard_normal((3, hidden)).astype(np.float32)
    ids = np.array([[0, 3], [1, 1], [2, 0]], np.int32)
    w = np.array([[0.6, 0.4], [0.5, 0.5], [0.2, 0.8]], np.float32)
    res = rng.standard_normal((3, hidden)).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(dev)
    h = ternary_expert_swiglu(t(x), _u32(ug, dev), t(ug_a), t(ids))
    href = ok.ternary_expert_swiglu(x, ug, ug_a, ids)
    assert_f32_close(np_f(h), href, what="swiglu fp32")
    y = ternary_expert_down_sum(h, _u32(dn, dev), t(dn_a), t(ids), t(w), residual=t(res))
    assert_f32_close(np_f(y), ok.ternary_expert_down_sum(np_f(h), dn, dn_a, ids, w, residual=res),
                     what="down_sum fp32")
    eo = ternary_expert_gemv(h, _u32(dn, dev), t(dn_a), t(ids))
    assert_f32_close(np_f(moe_reduce_add(eo, t(w), t(res))), ok.moe_reduce_add(np_f(eo), w, res),
                     what="reduce fp32")


@pytest.mark.parametrize("tokens", [1, 4])
def test_expert_down_sum_vs_oracle(dev, tokens):
    L = _experts(dev)
    top_k = 8
    g = torch.Generator(device=dev).manual_seed(81)
    ids = torch.stack([torch.randperm(8, generator=g, device=dev) for _ in range(tokens)]).int()
    w = torch.softmax(torch.randn(tokens, top_k, device=dev, generator=g), -1)
    h = synthetic.randn_bf16((tokens, top_k, 768), 82, dev)
    res = synthetic.randn_bf16((tokens, 2048), 83, dev)
    y = ternary_expert_down_sum(h, L.down_packed, L.down_alpha, ids, w, residual=res)
    ref = ok.ternary_expert_down_sum(np_f(h), np_u32(L.down_packed), np_f(L.down_alpha), ids.cpu().numpy(),
                                     np_f(w), residual=np_f(res))
    assert_bf16_close(np_f(y), ref, what="down_sum")


def test_expert_ids_out_of_range_are_clamped_not_faulting(dev):
    L = _experts(dev, n_exp=4, hidden=256, inter=128)
    x = synthetic.randn_bf16((1, 256), 5, dev)
    bad = torch.tensor([[9, -1]], device=dev, dtype=torch.int32)
    good = torch.tensor([[3, 0]], device=dev, dtype=torch.int32)
    torch.testing.assert_close(ternary_expert_swiglu(x, L.up_gate_packed, L.up_gate_alpha, bad),
                               ternary_expert_swiglu(x, L.up_gate_packed, L.up_gate_alpha, good))


@pytest.mark.parametrize("batch,n_out,k_in", [(5, 2560, 2048), (16, 200, 256), (33, 2048, 2048),
                                                (64, 130, 512)])
def test_gemv_mfma_batched_vs_oracle(dev, batch, n_out, k_in):
    """Batch >= 5 runs the MFMA GEMM: partial row tiles, more than one token
    tile, and batched == per-row (reference tests/test_ternary_gemv.py:227-247)."""
    w = synthetic.ternary_packed((n_out, k_in), 41 + batch, dev)
    alpha = synthetic.uniform_bf16((n_out,), 0.01, 0.05, 42, dev)
    x = synthetic.randn_bf16((batch, k_in), 43, dev)
    y = ternary_gemv(x, w, alpha)
    assert_bf16_close(np_f(y), ok.ternary_gemv(np_f(x), np_u32(w), np_f(alpha)), what=f"mfma B={batch}")
    rows = torch.cat([ternary_gemv(x[i:i + 1], w, alpha) for i in range(batch)])
    torch.testing.assert_close(y, rows, rtol=8e-3, atol=8e-3)


@pytest.mark.parametrize("batch", [6, 48])
def test_gemv_mfma_fused_rms_vs_oracle(dev, batch):
    w = synthetic.ternary_packed((2560, 2048), 51, dev)
    alpha = synthetic.uniform_bf16((2560,), 0.01, 0.05, 52, dev).float()
    x = synthetic.randn_bf16((batch, 2048), 53, dev)
    rms_w = (torch.rand(2048, device=dev) + 0.5).to(torch.bfloat16)
    y = ternary_gemv(x, w, alpha, rms_weight=rms_w, rms_eps=1e-6)
    ref = ok.ternary_gemv(np_f(x), np_u32(w), np_f(alpha), rms_weight=np_f(rms_w), rms_eps=1e-6)
    assert_bf16_close(np_f(y), ref, what=f"mfma rms B={batch}")


def _gemv_c(entry, x, w, alpha, rms_w=None, ws=None):
    """Call ma_ternary_gemv / ma_ternary_gemv_ws directly on [B, K] x."""
    from maple_amd import _lib
    batch, k_in = x.shape
    n_out, nwords = w.shape
    y = torch.empty(batch, n_out, device=x.device, dtype=torch.bfloat16)
    args = [_lib.ptr(x), _lib.BF16, batch, k_in, _lib.ptr(w), n_out, nwords, 0,
            _lib.ptr(alpha), _lib.dtype_code(alpha, "alpha"), _lib.ptr(rms_w),
            _lib.dtype_code(rms_w, "rms") if rms_w is not None else 0, 1e-6, _lib.ptr(y), n_out]
    if entry == "ma_ternary_gemv_ws":
        args += [_lib.ptr(ws), ws.numel() if ws is not None else 0]
    _lib.call(entry, *args, _lib.stream_of(x))
    return y


@pytest.mark.parametrize("rms", [None, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("batch,n_out", [(5, 2560), (16, 130), (17, 2048), (32, 2560), (48, 700)])
def test_gemv_mfma_one_and_two_launch_vs_oracle(dev, batch, n_out, rms):
    """The one-launch K-split GEMM against the oracle, and the workspace entry
    point (the two-launch form with the RMSNorm from 17 tokens, else the same
    one launch) against it: same per-word arithmetic, only the float32 sums of
    the per-token correction and squares add up in another order."""
    from maple_amd import _lib
    w = synthetic.ternary_packed((n_out, 2048), 61 + batch, dev)
    alpha = synthetic.uniform_bf16((n_out,), 0.01, 0.05, 62, dev)
    x = synthetic.randn_bf16((batch, 2048), 63, dev)
    rms_w = None if rms is None else (torch.rand(2048, device=dev) + 0.5).to(rms)
    nbytes = _lib.load().ma_ternary_gemv_workspace_bytes(batch, 128, int(rms is not None))
    assert (nbytes > 0) == (rms is not None and batch >= 17)
    ws = torch.full((max(nbytes, 256),), 0xAB, device=dev, dtype=torch.uint8)  # stale bytes
    y1 = _gemv_c("ma_ternary_gemv", x, w, alpha, rms_w)
    ref = ok.ternary_gemv(np_f(x), np_u32(w), np_f(alpha),
                          rms_weight=None if rms_w is None else np_f(rms_w), rms_eps=1e-6)
    assert_bf16_close(np_f(y1), ref, what=f"one-launch B={batch} rms={rms}")
    y2 = _gemv_c("ma_ternary_gemv_ws", x, w, alpha, rms_w, ws)
    torch.testing.assert_close(y2.float(), y1.float(), rtol=8e-3, atol=8e-3)
    assert_bf16_close(np_f(y2), ref, what=f"workspace entry B={batch} rms={rms}")
    assert torch.equal(y1, _gemv_c("ma_ternary_gemv", x, w, alpha, rms_w))  # deterministic
    assert torch.equal(y2, _gemv_c("ma_ternary_gemv_ws", x, w, alpha, rms_w, ws))


@pytest.mark.parametrize("batch", [8, 24])
def test_gemv_mfma_rms_large_k(dev, batch):
    """K = 12288 with the fused RMSNorm (no K limit on either form)."""
    w = synthetic.ternary_packed((384, 12288), 71, dev)
    alpha = synthetic.uniform_bf16((384,), 0.01, 0.05, 72, dev)
    x = synthetic.randn_bf16((batch, 12288), 73, dev)
    rms_w = (torch.rand(12288, device=dev) + 0.5).to(torch.bfloat16)
    y = ternary_gemv(x, w, alpha, rms_weight=rms_w, rms_eps=1e-6)
    ref = ok.ternary_gemv(np_f(x), np_u32(w), np_f(alpha), rms_weight=np_f(rms_w), rms_eps=1e-6)
    assert_bf16_close(np_f(y), ref, what=f"rms K=12288 B={batch}")


def test_gemv_two_launch_small_workspace_raises(dev):
    from maple_amd import _lib
    w = synthetic.ternary_packed((256, 2048), 81, dev)
    alpha = synthetic.uniform_bf16((256,), 0.01, 0.05, 82, dev)
    x = synthetic.randn_bf16((20, 2048), 83, dev)
    rms_w = torch.rand(2048, device=dev) + 0.5
    nbytes = _lib.load().ma_ternary_gemv_workspace_bytes(20, 128, 1)
    ws = torch.empty(nbytes - 256, device=dev, dtype=torch.uint8)
    with pytest.raises(ValueError, match="workspace"):
        _gemv_c("ma_ternary_gemv_ws", x, w, alpha, rms_w, ws)
    with pytest.raises(ValueError, match="workspace"):
        _gemv_c("ma_ternary_gemv_ws", x, w, alpha, rms_w, None)


# ---------------------------------------------------------------- RTN4 / norms
@pytest.mark.parametrize("batch,group", [(1, 128), (1, 64), (2, 128), (4, 64), (32, 128)])
def test_rtn4_gemv_vs_oracle(dev, batch, group):
    w, sc, bs = synthetic.rtn4_table(4096, 2048, group, 91, dev)
    x = synthetic.randn_bf16((batch, 2048), 92, dev)
    y = rtn4_gemv(x, w, sc, bs, group_size=group)
    ref = ok.rtn4_gemv(np_f(x), np_u32(w), np_f(sc), np_f(bs), group_size=group)
    assert_bf16_close(np_f(y), ref, what=f"rtn4 B={batch} g={group}")


@pytest.mark.parametrize("batch,group,n_out", [(5, 64, 4000), (16, 128, 4096), (32, 64, 1000),
                                               (40, 128, 4096)])
def test_rtn4_mfma_batched_vs_oracle(dev, batch, group, n_out):
    """Batch >= 5 runs the MFMA RTN4 GEMM (both group sizes, partial row
    tiles, several token tiles); batched == per-row within 8e-3
    (reference tests/test_rtn4.py:151-169)."""
    w, sc, bs = synthetic.rtn4_table(n_out, 2048, group, 93 + batch, dev)
    x = synthetic.randn_bf16((batch, 2048), 94, dev)
    y = rtn4_gemv(x, w, sc, bs, group_size=group)
    ref = ok.rtn4_gemv(np_f(x), np_u32(w), np_f(sc), np_f(bs), group_size=group)
    assert_bf16_close(np_f(y), ref, what=f"rtn4 mfma B={batch} g={group}")
    rows = torch.cat([rtn4_gemv(x[i:i + 1], w, sc, bs, group_size=group) for i in range(batch)])
    torch.testing.assert_close(y, rows, rtol=8e-3, atol=8e-3)
    # every sum has a fixed order: the same bits on every run
    for _ in range(3):
        assert torch.equal(rtn4_gemv(x, w, sc, bs, group_size=group), y)


@pytest.mark.parametrize("batch,n_out", [(5, 4096), (17, 4096), (32, 8192), (64, 4064)])
def test_rtn4_workspace_form_equals_one_launch(dev, batch, n_out):
    """ma_rtn4_gemv_ws (groups of 128: x' and group sums built once, copied
    into LDS by the LDS DMA) gives the bits of the one-launch ma_rtn4_gemv,
    on two calls in a row; a workspace one byte short is refused."""
    from maple_amd import _lib
    group = 128
    w, sc, bs = synthetic.rtn4_table(n_out, 2048, group, 95 + batch, dev)
    x = synthetic.randn_bf16((batch, 2048), 96 + batch, dev)
    nwords = 2048 // 8
    nbytes = int(_lib.load().ma_rtn4_gemv_workspace_bytes(batch, nwords, group))
    assert nbytes > 0
    ws = torch.zeros(nbytes, device=dev, dtype=torch.uint8)
    args = lambda y: (_lib.ptr(x), _lib.dtype_code(x, "x"), batch, x.stride(0), _lib.ptr(w), n_out, nwords, 0,
                      _lib.ptr(sc), _lib.dtype_code(sc, "s"), _lib.ptr(bs), _lib.dtype_code(bs, "b"), group,
                      _lib.ptr(y), n_out)
    y1 = torch.empty(batch, n_out, device=dev, dtype=torch.bfloat16)
    _lib.call("ma_rtn4_gemv", *args(y1), _lib.stream_of(x))
    for _ in range(2):
        y2 = torch.full((batch, n_out), 7.0, device=dev, dtype=torch.bfloat16)
        _lib.call("ma_rtn4_gemv_ws", *args(y2), _lib.ptr(ws), ws.numel(), _lib.stream_of(x))
        torch.cuda.synchronize()
        assert torch.equal(y1, y2)
    with pytest.raises(ValueError):
        _lib.call("ma_rtn4_gemv_ws", *args(y2), _lib.ptr(ws), nbytes - 1, _lib.stream_of(x))
    # n_out not a whole number of 32-row blocks: the one-launch kernel (no workspace needed)
    y3 = torch.empty(batch, n_out - 16, device=dev, dtype=torch.bfloat16)
    _lib.call("ma_rtn4_gemv_ws", _lib.ptr(x), _lib.dtype_code(x, "x"), batch, x.stride(0), _lib.ptr(w),
              n_out - 16, nwords, 0, _lib.ptr(sc), _lib.dtype_code(sc, "s"), _lib.ptr(bs), _lib.dtype_code(bs, "b"),
              group, _lib.ptr(y3), n_out - 16, None, 0, _lib.stream_of(x))
    torch.cuda.synchronize()
    assert torch.equal(y3, y1[:, : n_out - 16])


def test_rtn4_reference_fixture_fp32_and_kn(dev):
    rng = np.random.default_rng(1)
    wf = rng.standard_normal((64, 256)).astype(np.float32)
    packed, scales, biases = pack.quantize_rtn(wf)
    x = rng.standard_normal((2, 256)).astype(np.float32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    ref = ok.rtn4_gemv(x, packed, scales, biases)
    assert_f32_close(np_f(rtn4_gemv(t(x), _u32(packed, dev), t(scales), t(biases))), ref, what="rtn4 fp32")
    y_kn = rtn4_gemv(t(x), _u32(np.ascontiguousarray(packed.T), dev), t(scales.T), t(biases.T), packed_kn=True)
    assert_f32_close(np_f(y_kn), ref, what="rtn4 kn")
    ids = torch.tensor([[3, 7, 0], [1, 1, 63]], device=dev)
    emb = rtn4_embedding(ids, _u32(packed, dev), t(scales), t(biases))
    assert_f32_close(np_f(emb), ok.rtn4_embedding(ids.cpu().numpy(), packed, scales, biases),
                     rtol=1e-6, atol=1e-6, what="embedding")


def test_norms_vs_oracle(dev):
    x = synthetic.randn_bf16((3, 2048), 101, dev)
    y = synthetic.randn_bf16((3, 2048), 102, dev)
    w = torch.rand(2048, device=dev) + 0.5
    assert_bf16_close(np_f(rms_norm(x, w)), ok.rms_norm(np_f(x), np_f(w)), what="rms_norm")
    res, nrm = add_rms_norm(x, y, w)
    s, n = ok.add_rms_norm(np_f(x), np_f(y), np_f(w))
    assert_bf16_close(np_f(res), s, what="residual")
    assert_bf16_close(np_f(nrm), n, what="normed")


# ---------------------------------------------------------------- greedy argmax
@pytest.mark.parametrize("rows,n,dtype", [(1, 151936, torch.bfloat16), (32, 151936, torch.bfloat16),
                                          (3, 1001, torch.float32), (5, 7, torch.bfloat16)])
def test_greedy_argmax_matches_torch(dev, rows, n, dtype):
    from maple_amd.kernels import greedy_argmax

    g = torch.Generator(device=dev).manual_seed(rows * 7 + n)
    x = torch.randn(rows, n, generator=g, device=dev).to(dtype)
    # plant ties: the row maximum also at a later and at an earlier position
    m = x.float().amax(dim=1)
    x[0, n - 1] = m[0].to(dtype)
    if n > 2:
        x[rows - 1, 1] = (m[rows - 1] + 1).to(dtype)
        x[rows - 1, n - 2] = (m[rows - 1] + 1).to(dtype)
    got = greedy_argmax(x)
    torch.testing.assert_close(got, torch.argmax(x.float(), dim=-1), rtol=0, atol=0)
    out = torch.empty(rows, dtype=torch.int64, device=dev)
    assert greedy_argmax(x, out=out) is out and torch.equal(out, got)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_greedy_argmax_ties_within_and_across_vectors(dev, dtype):
    """The kernel compares whole 16-byte vectors by their maxima and rescans
    the winning one: the lowest index still wins for ties inside one vector,
    across vectors of one thread (vectors v and v + 1024), across threads,
    and a row of -inf gives 0 (torch.argmax's answer)."""
    from maple_amd.kernels import greedy_argmax

    n = 151936
    per = 8 if dtype == torch.bfloat16 else 4
    x = torch.full((5, n), -3.0, device=dev).to(dtype)
    x[0, 8 * per + 3] = 5.0
    x[0, 8 * per + 1] = 5.0  # same vector, lower index
    x[1, (7 + 1024) * per] = 2.0
    x[1, 7 * per + per - 1] = 2.0  # same thread, earlier vector
    x[2, 4000 * per + 2] = 1.0
    x[2, 17 * per + 2] = 1.0  # another thread, lower index
    x[2, 90000] = 1.0
    x[3] = -float("inf")
    x[4, n - 1] = 7.0  # the last element
    got = greedy_argmax(x)
    torch.testing.assert_close(got, torch.argmax(x.float(), dim=-1), rtol=0, atol=0)
    assert got.tolist()[:3] == [8 * per + 1, 7 * per + per - 1, 17 * per + 2]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_greedy_argmax_split_rows_equal_one_workgroup_form(dev, dtype):
    """greedy_argmax reads each row in chunks of 1280 vectors, one
    workgroup each, the last to finish reducing the partials: ties across
    chunks go to the lower index, the maximum may sit on a chunk's last
    element or in the elements past the last whole vector (a row of 151939
    values at stride 151944), and three calls in a row on one workspace give
    the one-workgroup ma_argmax_rows's ids and torch.argmax's."""
    from maple_amd import _lib
    from maple_amd.kernels import greedy_argmax

    per = 8 if dtype == torch.bfloat16 else 4
    chunk = 1280 * per
    n, ld = 151939, 151944
    g = torch.Generator(device=dev).manual_seed(5)
    base = torch.randn(6, ld, generator=g, device=dev).to(dtype)
    x = base[:, :n]
    x[0, 5 * chunk + 7] = 9.0
    x[0, 2 * chunk + 100] = 9.0  # an earlier chunk, same value
    x[1, 3 * chunk - 1] = 9.0  # the last element of chunk 2
    x[2, n - 2] = 9.0  # past the last whole vector
    x[3] = -float("inf")
    x[4, 0] = 9.0
    x[4, n - 1] = 9.0
    want = torch.argmax(x.float(), dim=-1)
    one = torch.empty(6, dtype=torch.int64, device=dev)
    _lib.call("ma_argmax_rows", _lib.ptr(x), _lib.dtype_code(x, "logits"), 6, n, x.stride(0), _lib.ptr(one),
              _lib.stream_of(x))
    for _ in range(3):
        got = greedy_argmax(x)
        torch.cuda.synchronize()
        assert torch.equal(got, want) and torch.equal(got, one)
    assert got.tolist()[:5] == [2 * chunk + 100, 3 * chunk - 1, n - 2, 0, 0]
    # a row stride that is not a whole number of vectors takes the one-workgroup form
    y = torch.randn(2, 1001 * per + 1, generator=g, device=dev).to(dtype)[:, :1001 * per - 3]
    assert torch.equal(greedy_argmax(y), torch.argmax(y.float(), dim=-1))


@pytest.mark.parametrize("n", [1024, 4096, 20000])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_greedy_argmax_all_negative_short_rows(dev, n, dtype):
    """Rows whose every value is negative, short enough that most threads of
    the workgroup have no vector of the row at all: the vectors past the row
    (filled with -inf, never re-read) must not win."""
    from maple_amd.kernels import greedy_argmax

    g = torch.Generator(device=dev).manual_seed(n)
    x = (-1.0 - torch.rand(4, n, generator=g, device=dev)).to(dtype)
    got = greedy_argmax(x)
    torch.testing.assert_close(got, torch.argmax(x.float(), dim=-1), rtol=0, atol=0)


@pytest.mark.parametrize("tokens,top_k,dtype", [(1, 8, torch.bfloat16), (2, 8, torch.bfloat16),
                                                (3, 8, torch.bfloat16), (5, 4, torch.bfloat16),
                                                (3, 2, torch.float32)])
def test_down_combine_is_the_blocks_two_launches(dev, tokens, top_k, dtype):
    """ternary_expert_down_sum(..., round_slots=True) (ma_ternary_expert_down_combine,
    what the per-slot MoE plan runs) gives the bits of the reference block's
    two launches, ternary_expert_gemv then moe_reduce_add (model.py:470-473):
    each slot's output rounded to x's dtype, the float32 combine in slot
    order, the residual last; the plain down_sum keeps its float32 sum (and
    differs); float32 x takes the generic kernel."""
    from maple_amd.kernels import moe_reduce_add, ternary_expert_down_sum, ternary_expert_gemv

    e, n_out, inter = 16, 2048, 768
    w = synthetic.ternary_packed((e, n_out, inter), 31, dev)
    alpha = synthetic.uniform_bf16((e, n_out), 0.01, 0.05, 32, dev)
    h = synthetic.randn_bf16((tokens, top_k, inter), 33, dev).to(dtype)
    g = torch.Generator(device=dev).manual_seed(34)
    ids = torch.stack([torch.randperm(e, generator=g, device=dev)[:top_k] for _ in range(tokens)]).to(torch.int32)
    wts = torch.rand(tokens, top_k, device=dev, generator=g)
    wts = wts / wts.sum(-1, keepdim=True)
    res = synthetic.randn_bf16((tokens, n_out), 35, dev).to(dtype)
    y = ternary_expert_down_sum(h, w, alpha, ids, wts, residual=res, round_slots=True)
    ref = moe_reduce_add(ternary_expert_gemv(h, w, alpha, ids), wts, residual=res)
    plain = ternary_expert_down_sum(h, w, alpha, ids, wts, residual=res)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)
    assert_bf16_close(np_f(plain), np_f(ref), rtol=2 ** -7, atol_frac=2e-3, what="plain vs rounded")
