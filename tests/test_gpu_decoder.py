"""Decode attention and the synthetic decoder vs the CPU oracle (needs the GPU).

Attention: QK-norm + RoPE + KV write and split GQA at ragged lengths up to
4096 (the reference's ragged set, tests/test_fused_decode.py:245, plus 4096).
Decoder: a reduced model over several teacher-forced steps at batch 1 and 3,
graph replays equal to eager, and one step of the full 24-layer synthetic
decoder (hidden 2048, 32/4 heads, 64 experts, vocab 151936) at batch 1.
Logits: cosine >= 0.9999 and max error <= 1e-2 of the logit scale; greedy ids
equal where the top-2 logits of the oracle are separated.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import assert_bf16_close, np_f, np_u32
from maple_amd import synthetic
from maple_amd.kernels import apply_qkv_decode, decode_attention, decode_gqa_attn, gqa_workspace, ternary_gemv
from maple_amd.kernels.decode_attn import attention_form, o_projection_supported
from maple_amd.model import DecoderConfig, SyntheticDecoder
from oracle import decoder as od

pytestmark = pytest.mark.gpu


# (query heads, KV heads, head_dim, rotary_dim): the synthetic decoder's, the
# Maple-Preview shape (16 / 4 heads of 128, partial rotary 0.5) and a full
# rotary over 128 (rotate-half pairs dims 64 apart, across a lane's two dims).
HEADS = [(32, 4, 64, 32), (16, 4, 128, 64), (16, 4, 128, 128)]
# Attention outputs against the oracle: elementwise |y - ref| <= 2^-8 |ref| +
# ATTN_ATOL * max|ref|.  Both sides round P to bf16 before P V, at different
# maxima: the oracle at the max over all positions (the reference's rounding
# when the positions fit one tile), the kernel at each wave's running max over
# its 32-position blocks, so each term's rounding differs by up to 2^-9
# relative; over ~4k positions the two P V sums differ by ~2e-3 of the output
# scale (a CPU simulation of both schemes on this distribution: 1.4e-4 at a
# scale of 0.07), on top of the output's own bf16 rounding.
ATTN_ATOL = 4e-3


def _rope_rows(table, seqlen, dev):
    """The reference's gather: float32 table rows at seqlen, cast to bf16."""
    return torch.from_numpy(table).to(dev)[seqlen.clamp(0, table.shape[0] - 1)].to(torch.bfloat16)


@pytest.mark.parametrize("heads", HEADS)
@pytest.mark.parametrize("mapped", [False, True])
def test_qk_norm_rope_store_vs_oracle(dev, mapped, heads):
    nq, nkv, d, rot = heads
    max_len = 4224
    seqlen = torch.tensor([0, 100, 4095], device=dev)
    rows = 5 if mapped else 3
    row_map = torch.tensor([4, 0, 2], device=dev) if mapped else None
    crow = row_map.tolist() if mapped else [0, 1, 2]
    qkv = synthetic.randn_bf16((3, (nq + 2 * nkv) * d), 1, dev)
    kc = synthetic.randn_bf16((rows, nkv, max_len, d), 2, dev)
    vc = synthetic.randn_bf16((rows, nkv, max_len, d), 3, dev)
    k0, v0 = kc.clone(), vc.clone()
    qw = torch.rand(d, device=dev) + 0.5
    kw = torch.rand(d, device=dev) + 0.5
    cos, sin = od.rope_tables(max_len, rot, 1e4)
    q = apply_qkv_decode(qkv, qw, kw, _rope_rows(cos, seqlen, dev), _rope_rows(sin, seqlen, dev),
                         kc, vc, seqlen, row_map=row_map, num_heads=nq, num_kv_heads=nkv,
                         head_dim=d, rotary_dim=rot, use_rope=True, use_qk_norm=True, eps=1e-6)
    x = np_f(qkv)
    touched = torch.zeros(rows, max_len, dtype=torch.bool, device=dev)
    for b, pos in enumerate(seqlen.tolist()):
        cs, sn = od.bf(cos[pos]), od.bf(sin[pos])
        ref_q = np.stack([od.head_norm_rope(x[b, h * d:(h + 1) * d], np_f(qw), cs, sn, rot, 1e-6)
                          for h in range(nq)])
        assert_bf16_close(np_f(q[b, :, 0]), ref_q, what=f"q row {b}")
        r = crow[b]
        for kh in range(nkv):
            o0, o1 = (nq + kh) * d, (nq + nkv + kh) * d
            ref_k = od.head_norm_rope(x[b, o0:o0 + d], np_f(kw), cs, sn, rot, 1e-6)
            assert_bf16_close(np_f(kc[r, kh, pos]), ref_k, what=f"k row {b}")
            np.testing.assert_array_equal(np_f(vc[r, kh, pos]), x[b, o1:o1 + d])
        touched[r, pos] = True
    untouched = ~touched
    for r in range(rows):
        assert torch.equal(kc[r][:, untouched[r]], k0[r][:, untouched[r]])
        assert torch.equal(vc[r][:, untouched[r]], v0[r][:, untouched[r]])


@pytest.mark.parametrize("heads", HEADS[:2])
@pytest.mark.parametrize("window", [None, 512])
def test_gqa_ragged_vs_oracle(dev, window, heads):
    nq, nkv, d, _ = heads
    max_len = 4096
    lens = [1, 63, 64, 65, 300, 511, 1000, 4096]
    seqlen = torch.tensor([n - 1 for n in lens], device=dev)
    q = synthetic.randn_bf16((len(lens), nq, 1, d), 11, dev)
    kc = synthetic.randn_bf16((len(lens), nkv, max_len, d), 12, dev)
    vc = synthetic.randn_bf16((len(lens), nkv, max_len, d), 13, dev)
    out = decode_gqa_attn(q, kc, vc, seqlen, scale=d ** -0.5, window=window)
    for b, n in enumerate(lens):
        ref = od.gqa(np_f(q[b, :, 0]), np_f(kc[b]), np_f(vc[b]), n, d ** -0.5, window)
        assert_bf16_close(np_f(out[b, :, 0]), ref, atol_frac=ATTN_ATOL, what=f"len {n}")
    # a row alone gives the same bits as in the batch
    solo = decode_gqa_attn(q[6:7], kc[6:7], vc[6:7], seqlen[6:7], scale=d ** -0.5, window=window)
    assert torch.equal(solo, out[6:7])


@pytest.mark.parametrize("heads", HEADS)
@pytest.mark.parametrize("window", [None, 300])
def test_fused_attention_equals_two_step(dev, window, heads):
    """decode_attention gives the bits of apply_qkv_decode + decode_gqa_attn
    (q, the written K/V and the output), for ragged rows through a row map,
    leaves the per-(row, KV head) arrival counters of the split barrier at zero
    and records no timed-out wait."""
    nq, nkv, d, rot = heads
    max_len = 1100
    seqlen = torch.tensor([0, 127, 128, 700, 1099], device=dev)
    row_map = torch.tensor([3, 5, 0, 1, 4], device=dev)
    qkv = synthetic.randn_bf16((5, (nq + 2 * nkv) * d), 21, dev)
    kc = synthetic.randn_bf16((6, nkv, max_len, d), 22, dev)
    vc = synthetic.randn_bf16((6, nkv, max_len, d), 23, dev)
    qw = (torch.rand(d, device=dev) + 0.5).to(torch.bfloat16)
    kw = (torch.rand(d, device=dev) + 0.5).to(torch.bfloat16)
    cos, sin = od.rope_tables(max_len, rot, 1e4)
    kc2, vc2 = kc.clone(), vc.clone()
    q = apply_qkv_decode(qkv, qw, kw, _rope_rows(cos, seqlen, dev), _rope_rows(sin, seqlen, dev),
                         kc, vc, seqlen, row_map=row_map, num_heads=nq, num_kv_heads=nkv,
                         head_dim=d, rotary_dim=rot, use_rope=True, use_qk_norm=True, eps=1e-6)
    ref = decode_gqa_attn(q, kc, vc, seqlen, row_map=row_map, scale=d ** -0.5, window=window)
    ws = gqa_workspace(5, nkv, max_len, dev, d)
    for _ in range(2):
        out = decode_attention(qkv, qw, kw, torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev),
                               kc2, vc2, seqlen, ws, row_map=row_map, num_heads=nq, num_kv_heads=nkv,
                               head_dim=d, rotary_dim=rot, eps=1e-6, scale=d ** -0.5, window=window)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        assert torch.equal(kc2, kc) and torch.equal(vc2, vc)
        sync = ws[:256 * (1 + 2 * 5 * nkv)].view(torch.int32)
        assert int(sync[2]) == 0, "a split barrier wait timed out"
        assert int(sync[64::128][:5 * nkv].count_nonzero()) == 0, "arrival counters not reset"
    # and the output matches the oracle on the written cache
    for b, n in enumerate((seqlen + 1).tolist()):
        r = int(row_map[b])
        o = od.gqa(np_f(q[b, :, 0]), np_f(kc[r]), np_f(vc[r]), n, d ** -0.5, window)
        assert_bf16_close(np_f(out[b, :, 0]), o, atol_frac=ATTN_ATOL, what=f"row {b}")


@pytest.mark.parametrize("heads", HEADS)
@pytest.mark.parametrize("wdt,tdt", [(torch.float16, torch.bfloat16), (torch.float32, torch.float16),
                                     (torch.bfloat16, torch.bfloat16)])
def test_fused_attention_weight_and_table_dtypes(dev, heads, wdt, tdt):
    """The fused launch reads its norm weights and RoPE rows as the aligned
    32-bit words that hold them, whatever their dtype: the same bits as the
    two-step path (which reads each element in its dtype) for f16, f32 and
    bf16 norm weights with bf16 and f16 tables, with RoPE and without."""
    nq, nkv, d, rot = heads
    max_len = 600
    seqlen = torch.tensor([5, 128, 433], device=dev)
    qkv = synthetic.randn_bf16((3, (nq + 2 * nkv) * d), 31, dev)
    kc = synthetic.randn_bf16((3, nkv, max_len, d), 32, dev)
    vc = synthetic.randn_bf16((3, nkv, max_len, d), 33, dev)
    qw = (torch.rand(d, device=dev) + 0.5).to(wdt)
    kw = (torch.rand(d, device=dev) + 0.5).to(wdt)
    cos, sin = od.rope_tables(max_len, rot, 1e4)
    cos_t, sin_t = torch.from_numpy(cos).to(dev).to(tdt), torch.from_numpy(sin).to(dev).to(tdt)
    for use_rope in (True, False):
        kc1, vc1, kc2, vc2 = kc.clone(), vc.clone(), kc.clone(), vc.clone()
        q = apply_qkv_decode(qkv, qw, kw, cos_t[seqlen], sin_t[seqlen],
                             kc1, vc1, seqlen, num_heads=nq, num_kv_heads=nkv, head_dim=d,
                             rotary_dim=rot, use_rope=use_rope, use_qk_norm=True, eps=1e-6)
        ref = decode_gqa_attn(q, kc1, vc1, seqlen, scale=d ** -0.5, window=None)
        ws = gqa_workspace(3, nkv, max_len, dev, d)
        out = decode_attention(qkv, qw, kw, cos_t, sin_t, kc2, vc2, seqlen, ws, num_heads=nq,
                               num_kv_heads=nkv, head_dim=d, rotary_dim=rot, use_rope=use_rope, eps=1e-6,
                               scale=d ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"use_rope={use_rope}"
        assert torch.equal(kc2, kc1) and torch.equal(vc2, vc1), f"use_rope={use_rope}"


@pytest.mark.parametrize("heads", HEADS[:2])
@pytest.mark.parametrize("seqlen", [0, 130, 2000, 4100])
def test_fused_attention_o_projection_equals_gemv(dev, seqlen, heads):
    """decode_attention(..., o_linear=...) at batch 1 returns the plain call's
    attention output and, from the same launch, the bits of ternary_gemv on
    it (the 2048 x 2048 o_proj), over consecutive calls on one workspace,
    with no timed-out wait recorded."""
    nq, nkv, d, rot = heads
    max_len = 4224
    qkv = synthetic.randn_bf16((1, (nq + 2 * nkv) * d), 31 + seqlen, dev)
    kc = synthetic.randn_bf16((1, nkv, max_len, d), 32, dev)
    vc = synthetic.randn_bf16((1, nkv, max_len, d), 33, dev)
    w = torch.ones(d, device=dev)
    cos, sin = (torch.from_numpy(t).to(dev) for t in od.rope_tables(max_len, rot, 1e4))
    sl = torch.tensor([seqlen], device=dev)
    wo, ao = synthetic.ternary_linear(2048, 2048, 34, dev)
    assert o_projection_supported(1, nq, nkv, d, max_len, None, 2048)
    kw = dict(num_heads=nq, num_kv_heads=nkv, head_dim=d, rotary_dim=rot, eps=1e-6, scale=d ** -0.5)
    kc2, vc2 = kc.clone(), vc.clone()
    ref = decode_attention(qkv, w, w, cos, sin, kc, vc, sl, gqa_workspace(1, nkv, max_len, dev, d), **kw)
    ws = gqa_workspace(1, nkv, max_len, dev, d)
    for _ in range(3):
        out, o = decode_attention(qkv, w, w, cos, sin, kc2, vc2, sl, ws, o_linear=(wo, ao), **kw)
        o_ref = ternary_gemv(out.reshape(1, -1), wo, ao)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        assert torch.equal(o, o_ref)
    assert int(ws[8:12].view(torch.int32).item()) == 0, "a barrier wait timed out"


@pytest.mark.parametrize("heads", HEADS[:2])
@pytest.mark.parametrize("batch,window", [(1, None), (4, None), (3, 300)])
def test_attention_ignores_cache_rows_past_the_sequence(dev, batch, window, heads):
    """Cache positions past a row's new one hold NaN in one call and zeros in
    the other: the outputs and the written K/V are the same bits (no load
    reaches past the sequence, or a value read there reaches the output)."""
    nq, nkv, d, rot = heads
    max_len = 1000
    seqlen = torch.tensor([999, 0, 130, 640][:batch], device=dev)
    qkv = synthetic.randn_bf16((batch, (nq + 2 * nkv) * d), 61, dev)
    kc = synthetic.randn_bf16((batch, nkv, max_len, d), 62, dev)
    vc = synthetic.randn_bf16((batch, nkv, max_len, d), 63, dev)
    past = torch.arange(max_len, device=dev)[None, :] > seqlen[:, None]  # [B, max_len]
    m = past[:, None, :, None].expand_as(kc)
    w = torch.ones(d, device=dev)
    cos, sin = (torch.from_numpy(t).to(dev) for t in od.rope_tables(max_len, rot, 1e4))
    kw = dict(num_heads=nq, num_kv_heads=nkv, head_dim=d, rotary_dim=rot, eps=1e-6, scale=d ** -0.5,
              window=window)
    outs, caches = [], []
    for fill in (float("nan"), 0.0):
        k2, v2 = kc.masked_fill(m, fill), vc.masked_fill(m, fill)
        outs.append(decode_attention(qkv, w, w, cos, sin, k2, v2, seqlen,
                                     gqa_workspace(batch, nkv, max_len, dev, d), **kw))
        caches.append((k2, v2))
    torch.cuda.synchronize()
    assert not torch.isnan(outs[0]).any()
    assert torch.equal(outs[0], outs[1])
    live = ~m
    for a, b in zip(caches[0], caches[1]):
        assert torch.equal(a[live], b[live])


@pytest.mark.parametrize("heads", HEADS[:2])
@pytest.mark.parametrize("batch,window", [(1, None), (3, 300), (9, None), (32, None)])
def test_attention_xcd_form_equals_grid_form(dev, monkeypatch, batch, window, heads):
    """The XCD-local attention form (every split of a (row, KV head) on one
    XCD: 1 row leaves 4 of 8 XCD slots idle, 9 rows a part-filled last block
    of 8 pairs) gives the cross-XCD form's bits, the forms alternating on one
    workspace (their arrival lines are shared), with no timed-out wait and the
    arrival counters at zero; and the output matches the oracle."""
    nq, nkv, d, rot = heads
    max_len = 4224
    g = torch.Generator().manual_seed(batch)
    seqlen = torch.randint(0, max_len, (batch,), generator=g).to(dev)
    seqlen[0] = 4100
    qkv = synthetic.randn_bf16((batch, (nq + 2 * nkv) * d), 41, dev)
    kc = synthetic.randn_bf16((batch, nkv, max_len, d), 42, dev)
    vc = synthetic.randn_bf16((batch, nkv, max_len, d), 43, dev)
    w = torch.ones(d, device=dev)
    cos, sin = (torch.from_numpy(t).to(dev) for t in od.rope_tables(max_len, rot, 1e4))
    kw = dict(num_heads=nq, num_kv_heads=nkv, head_dim=d, rotary_dim=rot, eps=1e-6, scale=d ** -0.5,
              window=window)
    assert attention_form(batch, nkv, d, max_len, window) == "xcd"
    ws = gqa_workspace(batch, nkv, max_len, dev, d)
    outs = []
    for form in ("xcd", "grid", "xcd", "grid", "xcd"):
        if form == "grid":
            monkeypatch.setenv("MAPLE_AMD_ATTN", "grid")
        else:
            monkeypatch.delenv("MAPLE_AMD_ATTN", raising=False)
        assert attention_form(batch, nkv, d, max_len, window) == form
        kc2, vc2 = kc.clone(), vc.clone()
        outs.append(decode_attention(qkv, w, w, cos, sin, kc2, vc2, seqlen, ws, **kw))
        torch.cuda.synchronize()
        sync = ws[:256 * (1 + 2 * batch * nkv)].view(torch.int32)
        assert int(sync[2]) == 0, f"{form}: a split barrier wait timed out"
        assert int(sync[64::128][:batch * nkv].count_nonzero()) == 0, "arrival counters not reset"
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    for b in range(0, batch, 8):  # the oracle over every row is slow; rows 0, 8, ... suffice
        n = int(seqlen[b]) + 1
        qn = apply_qkv_decode(qkv[b:b + 1], w, w, cos[seqlen[b:b + 1]].to(torch.bfloat16),
                              sin[seqlen[b:b + 1]].to(torch.bfloat16), kc[b:b + 1].clone(), vc[b:b + 1].clone(),
                              seqlen[b:b + 1], num_heads=nq, num_kv_heads=nkv, head_dim=d, rotary_dim=rot,
                              use_rope=True, use_qk_norm=True, eps=1e-6)
        ref = od.gqa(np_f(qn[0, :, 0]), np_f(kc2[b]), np_f(vc2[b]), n, d ** -0.5, window)
        assert_bf16_close(np_f(outs[0][b, :, 0]), ref, atol_frac=ATTN_ATOL, what=f"row {b}")


def test_attention_rejects_bad_shapes(dev):
    q = torch.zeros(2, 32, 1, 96, device=dev, dtype=torch.bfloat16)
    kc = torch.zeros(2, 4, 64, 96, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        decode_gqa_attn(q, kc, kc, torch.zeros(2, device=dev, dtype=torch.int64), scale=1.0, window=None)
    q = torch.zeros(2, 34, 1, 64, device=dev, dtype=torch.bfloat16)
    kc = torch.zeros(2, 4, 64, 64, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        decode_gqa_attn(q, kc, kc, torch.zeros(2, device=dev, dtype=torch.int64), scale=1.0, window=None)


def _to_np(model: SyntheticDecoder) -> dict:
    c = model.cfg
    layers = []
    for L in model.layers:
        layers.append(dict(
            qkv=np_u32(L.qkv), qkv_alpha=np_f(L.qkv_alpha), o=np_u32(L.o), o_alpha=np_f(L.o_alpha),
            input_ln=np_f(L.input_ln), post_ln=np_f(L.post_ln), q_norm=np_f(L.q_norm),
            k_norm=np_f(L.k_norm),
            moe=dict(gate_weight=np_f(L.moe.gate_weight), up_gate_packed=np_u32(L.moe.up_gate_packed),
                     up_gate_alpha=np_f(L.moe.up_gate_alpha), down_packed=np_u32(L.moe.down_packed),
                     down_alpha=np_f(L.moe.down_alpha))))
        layers[-1]["window"], layers[-1]["use_rope"] = c.layer_attention(len(layers) - 1)
    cfg = dict(hidden=c.hidden, heads=c.heads, kv_heads=c.kv_heads, head_dim=c.head_dim,
               rotary_dim=c.rotary_dim, eps=c.eps, rtn_group=c.rtn_group, top_k=c.top_k)
    w, s, b = model.embed
    lw, ls, lb = model.lm_head
    return dict(cfg=cfg, layers=layers, embed=(np_u32(w), np_f(s), np_f(b)),
                lm_head=(np_u32(lw), np_f(ls), np_f(lb)), final_norm=np_f(model.final_norm),
                cos=np_f(model.cos), sin=np_f(model.sin))


def _cache_np(cache) -> dict:
    return dict(k=[np_f(k) for k in cache.k], v=[np_f(v) for v in cache.v],
                seqlen=cache.seqlen.cpu().numpy().copy())


def _check_logits(logits, ref, what):
    y = np_f(logits)
    for b in range(y.shape[0]):
        cos = float(np.dot(y[b], ref[b]) / (np.linalg.norm(y[b]) * np.linalg.norm(ref[b])))
        assert cos >= 0.9999, f"{what} row {b}: cosine {cos:.6f}"
        err = np.abs(y[b] - ref[b]).max() / np.abs(ref[b]).max()
        assert err <= 1e-2, f"{what} row {b}: max rel err {err:.3g}"
        top2 = np.sort(ref[b])[-2:]
        if top2[1] - top2[0] > 4 * 2 ** -8 * abs(top2[1]):
            assert int(np.argmax(y[b])) == int(np.argmax(ref[b])), f"{what} row {b}: greedy id"


SMALL = DecoderConfig(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64, experts=8, inter=256,
                      top_k=2, vocab=1024, rtn_group=128, lm_scale=(0.01, 0.02))


@pytest.mark.parametrize("batch", [1, 3])
def test_small_decoder_steps_vs_oracle(dev, batch):
    model = SyntheticDecoder(SMALL, dev, seed=5, max_len=128)
    cache = model.make_cache(batch, prefill_len=37, seed=1)
    m = _to_np(model)
    cnp = _cache_np(cache)
    ids = torch.randint(0, SMALL.vocab, (batch,), device=dev, generator=torch.Generator(device=dev).manual_seed(3))
    for step in range(3):
        logits = model.forward(ids, cache)
        ref, _ = od.decoder_step(m, cnp, ids.cpu().numpy())
        _check_logits(logits, ref, f"step {step}")
        ids = torch.argmax(logits, dim=-1)  # teacher-forced: both continue from the device ids
    np.testing.assert_array_equal(cache.seqlen.cpu().numpy(), cnp["seqlen"])


@pytest.mark.parametrize("batch", [2, 20])
def test_decoder_graph_replays_match_eager(dev, batch):
    """Graph replays of the greedy step equal eager steps bit for bit, at a
    batch of 2 (per-slot MoE) and of 20 (routing launch + grouped MoE, the
    combine inside the next layer's QKV launch, the MFMA lm_head)."""
    model = SyntheticDecoder(SMALL, dev, seed=6, max_len=128)
    ids0 = torch.tensor([5, 900] * (batch // 2), device=dev)
    c_e = model.make_cache(batch, prefill_len=20, seed=2)
    ids_e = ids0.clone()
    eager = [model.greedy_step(ids_e, c_e).clone() for _ in range(4)]
    c_g = model.make_cache(batch, prefill_len=20, seed=2)
    ids_g = ids0.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # warm-up step, then rewind the cache position
        model.greedy_step(ids_g, c_g)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    c_g.seqlen.fill_(20)
    ids_g.copy_(ids0)
    c_g2 = model.make_cache(batch, prefill_len=20, seed=2)
    for i in range(SMALL.layers):
        c_g.k[i].copy_(c_g2.k[i])
        c_g.v[i].copy_(c_g2.v[i])
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        lg = model.greedy_step(ids_g, c_g)
    c_g.seqlen.fill_(20)
    ids_g.copy_(ids0)
    for i in range(SMALL.layers):
        c_g.k[i].copy_(c_g2.k[i])
        c_g.v[i].copy_(c_g2.v[i])
    for step in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(lg, eager[step]), f"replay {step}"
        torch.zeros(1, device=dev).add_(1)  # eager work between replays


def _cos(a, b):
    a, b = np.ravel(a), np.ravel(b)
    return float(np.dot(a, b) / (np.linalg.norm(a) * np.linalg.norm(b)))


def test_full_decoder_one_step_vs_oracle(dev):
    """Full 24-layer model, one step at batch 1 over a 4096-token cache.

    Layer by layer, each device layer's output is compared with the oracle's
    layer on the same (device) input: cosine >= 0.9999 and max error <= 1e-2;
    the expert ids equal the oracle's own top-k where the k-th and (k+1)-th
    probabilities differ by more than 1e-3 (the two layers see inputs that
    differ by rounding, about 2e-3 in a router logit).  The logits from the device's final hidden
    state meet the logits bar.  End to end, with no teacher forcing, the
    logits cosine is held to >= 0.99: this random 24-layer network amplifies
    rounding, and the oracle itself, given half-an-ulp relative noise at each
    RMSNorm output and the same routing, reaches only cosine 0.998.
    """
    model = SyntheticDecoder(DecoderConfig(), dev, seed=0, max_len=4096 + 64)
    c = model.cfg
    cache = model.make_cache(1, prefill_len=4096, seed=0)
    m = _to_np(model)
    cnp = _cache_np(cache)
    e2e = _cache_np(cache)
    oc = dict(m["cfg"], cos=m["cos"], sin=m["sin"])
    ids = torch.tensor([12345], device=dev)
    h = model.embed_tokens(ids)
    h_ref = od.bf(od.ok.rtn4_embedding(ids.cpu().numpy(), *m["embed"], group_size=c.rtn_group))
    np.testing.assert_array_equal(np_f(h), h_ref)
    h_e2e = h_ref
    dev_ids = []
    for i in range(c.layers):
        routing = []
        out = model.layer_step(i, h, cache, routing)
        rid = routing[0].cpu().numpy()
        dev_ids.append(rid)
        ref, (own, probs) = od.decoder_layer(m["layers"][i], oc, np_f(h), cnp, i, router_ids=rid)
        y = np_f(out)
        assert _cos(y, ref) >= 0.9999, f"layer {i}: cosine {_cos(y, ref):.6f}"
        assert np.abs(y - ref).max() <= 1e-2 * np.abs(ref).max(), f"layer {i}: max err"
        p = np.sort(probs.reshape(-1))[::-1]
        if p[c.top_k - 1] - p[c.top_k] > 1e-3:
            np.testing.assert_array_equal(np.sort(rid, -1), np.sort(own, -1), err_msg=f"layer {i} ids")
        h_e2e, _ = od.decoder_layer(m["layers"][i], oc, h_e2e, e2e, i, router_ids=rid)
        h = out
    cache.seqlen.add_(1)
    logits = model.head(h)
    torch.cuda.synchronize()
    _check_logits(logits, od.final_logits(m, np_f(h)), "full decoder head")
    ref_e2e = od.final_logits(m, h_e2e)
    cos = _cos(np_f(logits), ref_e2e)
    assert cos >= 0.99, f"end-to-end cosine {cos:.6f}"
    # forward() gives the same bits as the layer-by-layer calls
    cache2 = model.make_cache(1, prefill_len=4096, seed=0)
    assert torch.equal(model.forward(ids, cache2), logits)


def test_decoder_from_packed_checkpoint_equals_original(dev, tmp_path):
    """A packed-ternary-v1 directory written from a decoder and loaded back
    (maple_amd.checkpoint) decodes the same logits, bit for bit, over three
    greedy steps."""
    from maple_amd import checkpoint
    model = SyntheticDecoder(SMALL, dev, seed=8, max_len=128)
    checkpoint.save_decoder(model, tmp_path)
    back = checkpoint.load_decoder(tmp_path, dev, max_len=128)
    c1, c2 = model.make_cache(2, prefill_len=20, seed=2), back.make_cache(2, prefill_len=20, seed=2)
    ids = torch.tensor([11, 700], device=dev)
    for step in range(3):
        l1, l2 = model.forward(ids, c1), back.forward(ids, c2)
        torch.cuda.synchronize()
        assert torch.equal(l1, l2), f"step {step}"
        ids = torch.argmax(l1, dim=-1)


def test_sliding_and_nope_layers_vs_oracle(dev):
    """The reference's layer pattern (model.py:784-786): a sliding-window layer
    (the last 16 positions) and a full-attention layer without RoPE, three
    greedy steps at batch 2 against the oracle with the same per-layer
    attention."""
    import dataclasses
    cfg = dataclasses.replace(SMALL, layer_types=("sliding_attention", "full_attention"),
                              sliding_window=16, nope_on_global=True)
    model = SyntheticDecoder(cfg, dev, seed=9, max_len=128)
    cache = model.make_cache(2, prefill_len=41, seed=3)
    m = _to_np(model)
    assert m["layers"][0]["window"] == 16 and m["layers"][1]["use_rope"] is False
    cnp = _cache_np(cache)
    ids = torch.tensor([3, 517], device=dev)
    for step in range(3):
        logits = model.forward(ids, cache)
        ref, _ = od.decoder_step(m, cnp, ids.cpu().numpy())
        _check_logits(logits, ref, f"step {step}")
        ids = torch.argmax(logits, dim=-1)


def _step_with_device_routing(model, m, ids, cache, what, k):
    """One forward step checked against the oracle from the same state (the
    device's KV cache, so rounding differences do not carry over from earlier
    steps) and on the device's routing (top-k is discontinuous: two paths
    whose router inputs differ by bf16 rounding may pick different near-tied
    experts and then diverge); the device's ids equal the oracle's own where
    the k-th and (k+1)-th probabilities are more than 1e-3 apart."""
    cnp = _cache_np(cache)
    routing = []
    logits = model.forward(ids, cache, routing=routing)
    rids = [r.cpu().numpy() for r in routing]
    ref, own = od.decoder_step(m, cnp, ids.cpu().numpy(), router_ids=rids)
    _check_logits(logits, ref, what)
    for li, (oid, probs) in enumerate(own):
        p = np.sort(probs, axis=-1)[:, ::-1]
        clear = p[:, k - 1] - p[:, k] > 1e-3
        np.testing.assert_array_equal(np.sort(rids[li][clear], -1), np.sort(oid[clear], -1),
                                      err_msg=f"{what} layer {li} ids")
    return logits


@pytest.mark.parametrize("batch", [17, 32])
def test_small_decoder_batched_steps_vs_oracle(dev, batch):
    """Decode batches that take the batched forms: the routing launch and the
    grouped MoE (4+ tokens), the RTN4 MFMA lm_head (5+), the MoE combine in the
    next layer's QKV launch (17+), over a sliding-window layer and a NoPE
    full-attention layer, three steps against the oracle."""
    import dataclasses
    cfg = dataclasses.replace(SMALL, layer_types=("sliding_attention", "full_attention"),
                              sliding_window=16, nope_on_global=True)
    model = SyntheticDecoder(cfg, dev, seed=10, max_len=128)
    cache = model.make_cache(batch, prefill_len=33, seed=4)
    m = _to_np(model)
    gen = torch.Generator(device=dev).manual_seed(batch)
    ids = torch.randint(0, cfg.vocab, (batch,), device=dev, generator=gen)
    for step in range(3):
        logits = _step_with_device_routing(model, m, ids, cache, f"batch {batch} step {step}", cfg.top_k)
        ids = torch.argmax(logits, dim=-1)
    np.testing.assert_array_equal(cache.seqlen.cpu().numpy(), [33 + 3] * batch)


@pytest.mark.timeout(900)
def test_full_decoder_bs32_one_step_vs_oracle(dev, capsys):
    """Full 24-layer model, one step at batch 32 over a 4096-token cache
    (vocab 151936): the batched decode path (routing launch, grouped MFMA
    experts, batched QKV / O GEMMs, MFMA lm_head).

    Layer by layer, each device layer's output against the oracle's layer on
    the same device input with the device's routing: cosine >= 0.9999 per
    row and max error <= 1e-2 of the row's scale; the expert ids equal the
    oracle's own top-k on rows where the k-th and (k+1)-th probabilities are
    more than 1e-3 apart.  The logits of the device's final hidden state
    meet the logits bar on every row.  ``forward`` (which runs each layer's
    MoE combine inside the next layer's QKV launch) gives the same logits bit
    for bit.  End to end without teacher forcing, on two rows, cosine >= 0.99
    (as at batch 1: the random 24-layer network amplifies rounding)."""
    batch = 32
    model = SyntheticDecoder(DecoderConfig(), dev, seed=0, max_len=4096 + 64)
    c = model.cfg
    cache = model.make_cache(batch, prefill_len=4096, seed=0)
    m = _to_np(model)
    oc = dict(m["cfg"], cos=m["cos"], sin=m["sin"])
    ids = torch.randint(0, c.vocab, (batch,), device=dev, generator=torch.Generator(device=dev).manual_seed(32))
    e2e_rows = [0, batch - 1]
    h = model.embed_tokens(ids)
    h_ref = od.bf(od.ok.rtn4_embedding(ids.cpu().numpy(), *m["embed"], group_size=c.rtn_group))
    np.testing.assert_array_equal(np_f(h), h_ref)
    h_e2e = h_ref[e2e_rows]
    for i in range(c.layers):
        # the oracle cache of this layer only, taken before the device writes it
        ck = [None] * i + [np_f(cache.k[i]).astype(np.float32)]
        cv = [None] * i + [np_f(cache.v[i]).astype(np.float32)]
        cnp = dict(k=ck, v=cv, seqlen=cache.seqlen.cpu().numpy().copy())
        e2e = dict(k=[None] * i + [ck[i][e2e_rows].copy()], v=[None] * i + [cv[i][e2e_rows].copy()],
                   seqlen=cnp["seqlen"][e2e_rows].copy())
        routing = []
        out = model.layer_step(i, h, cache, routing)
        rid = routing[0].cpu().numpy()
        ref, (own, probs) = od.decoder_layer(m["layers"][i], oc, np_f(h), cnp, i, router_ids=rid)
        y = np_f(out)
        for b in range(batch):
            assert _cos(y[b], ref[b]) >= 0.9999, f"layer {i} row {b}: cosine {_cos(y[b], ref[b]):.6f}"
            assert np.abs(y[b] - ref[b]).max() <= 1e-2 * np.abs(ref[b]).max(), f"layer {i} row {b}: max err"
            p = np.sort(probs[b])[::-1]
            if p[c.top_k - 1] - p[c.top_k] > 1e-3:
                np.testing.assert_array_equal(np.sort(rid[b]), np.sort(own[b]), err_msg=f"layer {i} row {b} ids")
        h_e2e, _ = od.decoder_layer(m["layers"][i], oc, h_e2e, e2e, i, router_ids=rid[e2e_rows])
        h = out
        with capsys.disabled():  # the oracle takes seconds per layer at this size
            print(f"  bs32 layer {i} matches the oracle", flush=True)
    cache.seqlen.add_(1)
    logits = model.head(h)
    torch.cuda.synchronize()
    _check_logits(logits, od.final_logits(m, np_f(h)), "full decoder bs32 head")
    ref_e2e = od.final_logits(m, h_e2e)
    for j, b in enumerate(e2e_rows):
        cos = _cos(np_f(logits[b]), ref_e2e[j])
        assert cos >= 0.99, f"row {b}: end-to-end cosine {cos:.6f}"
    cache2 = model.make_cache(batch, prefill_len=4096, seed=0)
    assert torch.equal(model.forward(ids, cache2), logits)


def test_checkpoint_float32_alphas_decode_vs_oracle(dev, tmp_path):
    """A checkpoint whose row_alpha values bf16 cannot hold (float32, as the
    converter writes them) loads with float32 alphas and decodes against the
    oracle on those exact values, at batch 1 and 20."""
    from maple_amd import checkpoint
    model = SyntheticDecoder(SMALL, dev, seed=11, max_len=128)
    g = torch.Generator(device=dev).manual_seed(4)
    for L in model.layers:
        L.qkv_alpha = torch.rand(L.qkv_alpha.shape, device=dev, generator=g) * 0.04 + 0.01
        L.o_alpha = torch.rand(L.o_alpha.shape, device=dev, generator=g) * 0.04 + 0.01
        L.moe.up_gate_alpha = torch.rand(L.moe.up_gate_alpha.shape, device=dev, generator=g) * 0.04 + 0.01
        L.moe.down_alpha = torch.rand(L.moe.down_alpha.shape, device=dev, generator=g) * 0.04 + 0.01
    checkpoint.save_decoder(model, tmp_path)
    back = checkpoint.load_decoder(tmp_path, dev, max_len=128)
    assert back.layers[0].moe.down_alpha.dtype == torch.float32
    m = _to_np(back)
    for batch in (1, 20):
        cache = back.make_cache(batch, prefill_len=29, seed=5)
        ids = torch.arange(batch, device=dev) * 37 % SMALL.vocab
        for step in range(2):
            logits = _step_with_device_routing(back, m, ids, cache,
                                               f"float32 alphas batch {batch} step {step}", SMALL.top_k)
            ids = torch.argmax(logits, dim=-1)
