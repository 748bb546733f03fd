"""Pins for the oracle's composition functions (CPU only).

``moe_experts``, ``moe_block``, ``moe_layer_cpu_fp32``, ``decoder_layer``,
``decoder_step`` and ``final_logits`` are each checked against something a
plausible mistake would fail:

* the reference's own composition test (tests/test_model.py:194-242):
  separately packed up and gate matrices, one GEMV per selected expert in a
  Python loop, then concatenated -- a swapped ``[up; gate]`` order, a wrong
  expert index or a transposed weight fails it;
* brute-force scalar loops on tiny inputs (the bf16 rounding points of
  ``h`` and of each slot's down output are applied by hand where the
  reference stores ``x.dtype``, so a missing or extra rounding fails);
* closed forms that zero weights make exact: with every expert and O-projection
  alpha zero a decoder layer returns its input; with the q/k rows zero the
  attention weights are uniform and the output is the mean of V, so the
  q/k/v offsets, the K/V write and the GQA head mapping are all fixed.
"""

from __future__ import annotations

import math

import numpy as np

from oracle import decoder as od
from oracle import kernels as ok
from oracle import pack

bf = od.bf


def _ternarized_experts(rng, e_n, hid, inter):
    """Expert weights built as the reference's test builds them: ``ternarize``
    of normal matrices, up / gate / down packed separately."""
    up_p, up_a = pack.ternarize(rng.standard_normal((e_n, inter, hid)).astype(np.float32))
    gate_p, gate_a = pack.ternarize(rng.standard_normal((e_n, inter, hid)).astype(np.float32))
    down_p, down_a = pack.ternarize(rng.standard_normal((e_n, hid, inter)).astype(np.float32))
    up_a, gate_a, down_a = (np.asarray(a, np.float64).reshape(e_n, -1) for a in (up_a, gate_a, down_a))
    return up_p, up_a, gate_p, gate_a, down_p, down_a


def _scalar_gemv(codes, alpha, x):
    """``alpha[n] * sum_k (code[n, k] - 1) x[k]`` by loops over unpacked codes."""
    n, k = codes.shape
    return np.array([alpha[r] * math.fsum((int(codes[r, c]) - 1) * float(x[c]) for c in range(k))
                     for r in range(n)])


def _silu_clamped(up, gate):
    u = min(max(up, -7.0), 7.0)
    g = min(gate, 7.0)
    return u * g / (1.0 + math.exp(-g))


def test_moe_experts_matches_selected_expert_loop():
    """reference tests/test_model.py:194-242, float64, with and without the
    reference's bf16 stores of h and of each slot's down output."""
    rng = np.random.default_rng(3)
    n_tok, hid, e_n, topk, inter = 3, 128, 4, 2, 128
    up_p, up_a, gate_p, gate_a, down_p, down_a = _ternarized_experts(rng, e_n, hid, inter)
    ug_p = np.concatenate([up_p, gate_p], axis=1)
    ug_a = np.concatenate([up_a, gate_a], axis=1)
    x = bf(rng.standard_normal((n_tok, hid)))
    ids = np.array([[0, 3], [2, 1], [3, 0]])
    wts = np.array([[0.7, 0.3], [0.45, 0.55], [0.2, 0.8]], np.float32)
    res = bf(rng.standard_normal((n_tok, hid)))
    up_c = pack.unpack_2bit(up_p)
    gate_c = pack.unpack_2bit(gate_p)
    down_c = pack.unpack_2bit(down_p)
    for rounding in (False, True):
        y, h = ok.moe_experts(x, ids, wts, ug_p, ug_a, down_p, down_a, residual=res, round_bf16=rounding)
        rnd = bf if rounding else (lambda a: np.asarray(a, np.float64))
        for t in range(n_tok):
            acc = res[t].astype(np.float64).copy()
            for s in range(topk):
                e = int(ids[t, s])
                up = _scalar_gemv(up_c[e], up_a[e], x[t])
                gate = _scalar_gemv(gate_c[e], gate_a[e], x[t])
                hh = rnd(np.array([_silu_clamped(u, g) for u, g in zip(up, gate)]))
                np.testing.assert_allclose(h[t, s], hh, rtol=1e-12, atol=1e-300)
                acc += float(wts[t, s]) * rnd(_scalar_gemv(down_c[e], down_a[e], hh))
            np.testing.assert_allclose(y[t], acc, rtol=1e-12, atol=1e-12)
    # the roundings are really applied: the two results differ
    y0, _ = ok.moe_experts(x, ids, wts, ug_p, ug_a, down_p, down_a, round_bf16=False)
    y1, _ = ok.moe_experts(x, ids, wts, ug_p, ug_a, down_p, down_a, round_bf16=True)
    assert np.abs(y0 - y1).max() > 1e-6


def test_moe_experts_unrounded_equals_down_sum():
    rng = np.random.default_rng(11)
    e_n, hid, inter, t, k = 6, 64, 32, 4, 3
    ug = pack.pack_2bit(rng.integers(0, 3, (e_n, 2 * inter, hid), dtype=np.uint32))
    ug_a = rng.uniform(0.01, 0.05, (e_n, 2 * inter))
    dn = pack.pack_2bit(rng.integers(0, 3, (e_n, hid, inter), dtype=np.uint32))
    dn_a = rng.uniform(0.01, 0.05, (e_n, hid))
    x = rng.standard_normal((t, hid))
    ids = rng.integers(0, e_n, (t, k))
    w = rng.uniform(0.0, 1.0, (t, k))
    res = rng.standard_normal((t, hid))
    y, h = ok.moe_experts(x, ids, w, ug, ug_a, dn, dn_a, residual=res, round_bf16=False)
    want = ok.ternary_expert_down_sum(ok.ternary_expert_swiglu(x, ug, ug_a, ids), dn, dn_a, ids, w,
                                      residual=res)
    np.testing.assert_allclose(y, want, rtol=1e-12, atol=1e-12)


def test_moe_block_is_router_then_experts():
    rng = np.random.default_rng(12)
    e_n, hid, inter = 8, 64, 32
    gw = rng.standard_normal((e_n, hid)) * 0.3
    ug = pack.pack_2bit(rng.integers(0, 3, (e_n, 2 * inter, hid), dtype=np.uint32))
    ug_a = rng.uniform(0.01, 0.05, (e_n, 2 * inter))
    dn = pack.pack_2bit(rng.integers(0, 3, (e_n, hid, inter), dtype=np.uint32))
    dn_a = rng.uniform(0.01, 0.05, (e_n, hid))
    x = bf(rng.standard_normal((5, hid)))
    bias = rng.standard_normal(e_n)
    for rounding in (True, False):
        y, ids, wts, _ = ok.moe_block(x, gw, ug, ug_a, dn, dn_a, 3, residual=x, router_bias=bias,
                                      round_bf16=rounding)
        rid, rw, _ = ok.router_topk(x, gw, 3, bias=bias)
        np.testing.assert_array_equal(ids, rid)
        np.testing.assert_array_equal(wts, rw)
        ye, _ = ok.moe_experts(x, rid, rw, ug, ug_a, dn, dn_a, residual=x, round_bf16=rounding)
        np.testing.assert_array_equal(y, ye)


def test_cpu_fp32_layer_matches_float64_block():
    """The CPU baseline path (float32 NumPy) against the float64 block without
    intermediate rounding: the same function to float32 precision."""
    rng = np.random.default_rng(13)
    e_n, hid, inter, k = 8, 256, 128, 2
    gw = (rng.standard_normal((e_n, hid)) * 0.05).astype(np.float32)
    ug = pack.pack_2bit(rng.integers(0, 3, (e_n, 2 * inter, hid), dtype=np.uint32))
    ug_a = rng.uniform(0.01, 0.05, (e_n, 2 * inter)).astype(np.float32)
    dn = pack.pack_2bit(rng.integers(0, 3, (e_n, hid, inter), dtype=np.uint32))
    dn_a = rng.uniform(0.01, 0.05, (e_n, hid)).astype(np.float32)
    x = rng.standard_normal((3, hid)).astype(np.float32)
    y32 = ok.moe_layer_cpu_fp32(x, gw, ug, ug_a, dn, dn_a, k)
    y64, _, _, _ = ok.moe_block(x, gw, ug, ug_a, dn, dn_a, k, round_bf16=False)
    scale = np.abs(y64).max()
    np.testing.assert_allclose(y32, y64, rtol=1e-4, atol=1e-5 * scale)


def test_swiglu_known_values():
    """gate = 0 gives 0 whatever up is; gate below -7 is not clamped (only
    ``min(gate, 7)``); gate above 7 and |up| above 7 are clamped."""
    up = np.array([5.0, 2.0, 2.0, 9.0, -9.0, 1.0])
    gate = np.array([0.0, -9.0, 9.0, 1.0, 1.0, 7.0])
    out = ok.swiglu_act(up, gate)
    assert out[0] == 0.0
    np.testing.assert_allclose(out[1], 2.0 * -9.0 / (1.0 + math.exp(9.0)), rtol=1e-14)
    assert abs(out[1] - 2.0 * -7.0 / (1.0 + math.exp(7.0))) > 1e-4  # not a symmetric clamp
    np.testing.assert_allclose(out[2], 2.0 * 7.0 / (1.0 + math.exp(-7.0)), rtol=1e-14)
    np.testing.assert_allclose(out[3], 7.0 / (1.0 + math.exp(-1.0)), rtol=1e-14)
    np.testing.assert_allclose(out[4], -7.0 / (1.0 + math.exp(-1.0)), rtol=1e-14)
    np.testing.assert_allclose(out[5], out[2] / 2.0, rtol=1e-14)


def test_final_logits_brute_force():
    rng = np.random.default_rng(14)
    vocab, hid, g = 5, 128, 64
    codes = rng.integers(0, 16, (vocab, hid), dtype=np.uint32)
    sc = bf(rng.uniform(0.01, 0.03, (vocab, hid // g)))
    bs = bf(rng.uniform(-0.2, 0.0, (vocab, hid // g)))
    fn = rng.uniform(0.5, 1.5, hid)
    h = bf(rng.standard_normal((2, hid)))
    m = dict(cfg=dict(eps=1e-6, rtn_group=g), final_norm=fn, lm_head=(pack.pack_4bit(codes), sc, bs))
    got = od.final_logits(m, h)
    for b in range(2):
        rms = math.sqrt(math.fsum(float(v) * float(v) for v in h[b]) / hid + 1e-6)
        hn = bf(np.array([float(h[b, k]) / rms * fn[k] for k in range(hid)]))
        for v in range(vocab):
            want = math.fsum((int(codes[v, k]) * sc[v, k // g] + bs[v, k // g]) * hn[k] for k in range(hid))
            assert got[b, v] == bf(np.array([want]))[0]


def _tiny_model(rng, *, layers=2, hid=128, nq=4, nkv=2, d=64, e_n=4, inter=64, vocab=7, g=64,
                zero_q_k=True, zero_o=False, zero_experts=True):
    """A tiny oracle decoder; the chosen projections' alphas are zero."""
    c = dict(hidden=hid, heads=nq, kv_heads=nkv, head_dim=d, rotary_dim=d // 2, eps=1e-6,
             rtn_group=g, top_k=2)
    L = []
    qkv_rows = (nq + 2 * nkv) * d
    for _ in range(layers):
        qkv_a = rng.uniform(0.01, 0.05, qkv_rows)
        if zero_q_k:
            qkv_a[:(nq + nkv) * d] = 0.0
        o_a = np.zeros(hid) if zero_o else rng.uniform(0.01, 0.05, hid)
        ug_a = rng.uniform(0.01, 0.05, (e_n, 2 * inter))
        dn_a = np.zeros((e_n, hid)) if zero_experts else rng.uniform(0.01, 0.05, (e_n, hid))
        L.append(dict(
            qkv=pack.pack_2bit(rng.integers(0, 3, (qkv_rows, hid), dtype=np.uint32)), qkv_alpha=qkv_a,
            o=pack.pack_2bit(rng.integers(0, 3, (hid, nq * d), dtype=np.uint32)), o_alpha=o_a,
            input_ln=np.ones(hid), post_ln=np.ones(hid), q_norm=np.ones(d), k_norm=np.ones(d),
            moe=dict(gate_weight=bf(rng.standard_normal((e_n, hid)) * 0.1),
                     up_gate_packed=pack.pack_2bit(rng.integers(0, 3, (e_n, 2 * inter, hid), dtype=np.uint32)),
                     up_gate_alpha=ug_a,
                     down_packed=pack.pack_2bit(rng.integers(0, 3, (e_n, hid, inter), dtype=np.uint32)),
                     down_alpha=dn_a)))
    cos, sin = od.rope_tables(64, d // 2, 1e4)
    tab = lambda seed: (pack.pack_4bit(rng.integers(0, 16, (vocab, hid), dtype=np.uint32)),  # noqa: E731
                        bf(rng.uniform(0.01, 0.03, (vocab, hid // g))), bf(rng.uniform(-0.2, -0.1, (vocab, hid // g))))
    return dict(cfg=c, layers=L, embed=tab(1), lm_head=tab(2), final_norm=np.ones(hid), cos=cos, sin=sin)


def _cache(rng, m, batch, prefill, max_len=64):
    c = m["cfg"]
    shape = (batch, c["kv_heads"], max_len, c["head_dim"])
    k = [bf(rng.standard_normal(shape)) for _ in m["layers"]]
    v = [bf(rng.standard_normal(shape)) for _ in m["layers"]]
    for a in k + v:
        a[:, :, prefill:] = 0.0
    return dict(k=k, v=v, seqlen=np.full(batch, prefill, np.int64))


def test_decoder_layer_zero_experts_uniform_attention():
    """q and k rows zero -> every score is 0, attention is the mean of V over
    the positions read (the old ones and the one just written); expert down
    alphas zero -> the MoE adds nothing.  The layer's output is then
    bf16(h + bf16(O @ bf16(mean V))) computed here by loops."""
    rng = np.random.default_rng(15)
    m = _tiny_model(rng, layers=1)
    c = dict(m["cfg"], cos=m["cos"], sin=m["sin"])
    nq, nkv, d = c["heads"], c["kv_heads"], c["head_dim"]
    L = m["layers"][0]
    prefill = 9
    for window in (None, 4):
        L["window"] = window
        cache = _cache(np.random.default_rng(16), m, 2, prefill)
        old_v = [a.copy() for a in cache["v"]]
        h = bf(rng.standard_normal((2, c["hidden"])))
        out, (ids, probs) = od.decoder_layer(L, c, h, cache, 0)
        qkv_codes = pack.unpack_2bit(L["qkv"])
        o_codes = pack.unpack_2bit(L["o"])
        for b in range(2):
            rms = math.sqrt(math.fsum(float(t) ** 2 for t in h[b]) / c["hidden"] + c["eps"])
            qkv = bf(_scalar_gemv(qkv_codes, L["qkv_alpha"], h[b] / rms))
            # K written as RMSNorm of a zero row (zero), V as the raw v rows
            np.testing.assert_array_equal(cache["k"][0][b, :, prefill], 0.0)
            for kh in range(nkv):
                v_row = qkv[(nq + nkv + kh) * d:(nq + nkv + kh + 1) * d]
                np.testing.assert_array_equal(cache["v"][0][b, kh, prefill], v_row)
                np.testing.assert_array_equal(cache["v"][0][b, kh, :prefill], old_v[0][b, kh, :prefill])
            start = 0 if window is None else prefill + 1 - window
            attn = np.concatenate([cache["v"][0][b, hh // (nq // nkv), start:prefill + 1].mean(axis=0)
                                   for hh in range(nq)])
            o = bf(_scalar_gemv(o_codes, L["o_alpha"], bf(attn)))
            np.testing.assert_array_equal(out[b], bf(h[b] + o))
        assert ids.shape == (2, c["top_k"]) and np.allclose(probs.sum(axis=-1), 1.0)


def test_decoder_step_skeleton_and_zero_layers():
    """With the O and expert alphas zero, every layer returns its input, so a
    step's logits are final_logits of the embedding rows, the cache position
    advances by one, and each layer's V row at the old position holds that
    layer's v projection."""
    rng = np.random.default_rng(17)
    m = _tiny_model(rng, layers=2, zero_o=True)
    cache = _cache(np.random.default_rng(18), m, 2, 5)
    ids = np.array([6, 1])
    logits, routing = od.decoder_step(m, cache, ids)
    packed, sc, bs = m["embed"]
    emb = np.zeros((2, m["cfg"]["hidden"]))
    codes = pack.unpack_4bit(packed)
    g = m["cfg"]["rtn_group"]
    for b, t in enumerate(ids):
        emb[b] = [float(np.float32(np.float32(codes[t, k]) * np.float32(sc[t, k // g]) + np.float32(bs[t, k // g])))
                  for k in range(emb.shape[1])]
    np.testing.assert_array_equal(logits, od.final_logits(m, bf(emb)))
    np.testing.assert_array_equal(cache["seqlen"], [6, 6])
    assert len(routing) == 2
    c = m["cfg"]
    for i, L in enumerate(m["layers"]):
        qkv = bf(ok.ternary_gemv(bf(emb), L["qkv"], L["qkv_alpha"], rms_weight=L["input_ln"], rms_eps=c["eps"]))
        v0 = (c["heads"] + c["kv_heads"]) * c["head_dim"]
        np.testing.assert_array_equal(cache["v"][i][:, 0, 5], qkv[:, v0:v0 + c["head_dim"]])
