"""The oracle's closed forms against independent checks (CPU).

Each closed form is pinned by something that a plausible mistake (wrong bit
order, sign, operand transposition, dropped term, wrong tie rule) would
fail: the reference's known-answer test, brute-force Python loops on tiny
inputs, or identities that fix the result.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np

from oracle import kernels as ok
from oracle import pack

KATS = json.loads((Path(__file__).parent / "golden" / "pack_kats.json").read_text())


def _rand_packed(rng, shape):
    return pack.pack_2bit(rng.integers(0, 3, shape, dtype=np.uint32))


def test_ternary_gemv_reference_kat():
    """tests/test_ternary_gemv.py:114-132: code 2 -> +alpha*x, code 0 -> -alpha*x."""
    e = KATS["ternary_gemv_lsb_first"]
    codes = np.full((e["n"], e["k"]), e["default_code"], np.uint32)
    for r, c, v in e["codes_set"]:
        codes[r, c] = v
    y = ok.ternary_gemv(np.arange(e["k"], dtype=np.float32), pack.pack_2bit(codes), np.array(e["alpha"]))
    np.testing.assert_allclose(y, e["y"], rtol=0, atol=1e-12)


def test_ternary_gemv_brute_force_and_code3():
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 4, (5, 32), dtype=np.uint32)  # includes code 3 (= +2)
    alpha = rng.uniform(0.5, 2.0, 5)
    x = rng.standard_normal((3, 32))
    y = ok.ternary_gemv(x, pack.pack_2bit(codes), alpha)
    for b in range(3):
        for n in range(5):
            want = alpha[n] * sum((int(codes[n, k]) - 1) * x[b, k] for k in range(32))
            assert abs(y[b, n] - want) < 1e-9
    # the packed_kn layout is the transpose of the words, same result
    y_kn = ok.ternary_gemv(x, pack.pack_2bit(codes).T.copy(), alpha, packed_kn=True)
    np.testing.assert_allclose(y_kn, y, rtol=0, atol=1e-12)


def test_ternary_gemv_rms_fold_equals_explicit_norm():
    rng = np.random.default_rng(1)
    packed = _rand_packed(rng, (7, 64))
    alpha = rng.uniform(0.01, 0.05, 7)
    x = rng.standard_normal((2, 64))
    w = rng.uniform(0.5, 1.5, 64)
    y = ok.ternary_gemv(x, packed, alpha, rms_weight=w, rms_eps=1e-6)
    normed = np.stack([xr / math.sqrt(float(np.mean(xr * xr)) + 1e-6) * w for xr in x])
    np.testing.assert_allclose(y, ok.ternary_gemv(normed, packed, alpha), rtol=1e-12, atol=1e-12)


def test_router_brute_force_and_ties():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 16))
    g = rng.standard_normal((6, 16))
    ids, wts, probs = ok.router_topk(x, g, 3)
    for t in range(4):
        logits = [sum(x[t, k] * g[e, k] for k in range(16)) for e in range(6)]
        m = max(logits)
        ex = [math.exp(v - m) for v in logits]
        p = [v / sum(ex) for v in ex]
        order = sorted(range(6), key=lambda e: (-p[e], e))[:3]
        assert ids[t].tolist() == order
        tot = sum(p[e] for e in order)
        np.testing.assert_allclose(wts[t], [p[e] / (tot + 1e-20) for e in order], rtol=1e-6)
    # exact ties resolve to the lowest expert index, in descending order
    g_tie = np.zeros((5, 4))
    g_tie[3] = g_tie[1] = [1, 0, 0, 0]
    ids, wts, _ = ok.router_topk(np.array([[1.0, 0, 0, 0]]), g_tie, 4)
    assert ids[0].tolist() == [1, 3, 0, 2]
    np.testing.assert_allclose(wts.sum(), 1.0, rtol=1e-6)


def test_router_bias_shifts_logits():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 8))
    g = rng.standard_normal((5, 8))
    b = np.array([0.0, 10.0, 0.0, -10.0, 0.0])
    ids, _, p = ok.router_topk(x, g, 1, bias=b)
    assert ids[:, 0].tolist() == [1, 1]
    _, _, p0 = ok.router_topk(x, g, 1)
    ratio = p[:, 1] / p[:, 0] / (p0[:, 1] / p0[:, 0])
    np.testing.assert_allclose(ratio, math.exp(10.0), rtol=1e-9)


def test_dispatch_brute_force():
    rng = np.random.default_rng(4)
    ids = rng.integers(0, 6, (9, 3))
    counts, offsets, pair_ids, inverse = ok.dispatch(ids, 6)
    flat = ids.reshape(-1)
    for e in range(6):
        lst = [p for p in range(flat.size) if flat[p] == e]
        assert counts[e] == len(lst)
        assert pair_ids[offsets[e]:offsets[e + 1]].tolist() == lst
    assert offsets[0] == 0 and offsets[-1] == flat.size
    np.testing.assert_array_equal(pair_ids[inverse], np.arange(flat.size))


def test_swiglu_closed_form_and_clamps():
    up = np.array([-9.0, -1.0, 0.5, 8.0, 3.0])
    gate = np.array([1.0, 9.0, -2.0, 2.0, 7.5])
    out = ok.swiglu_act(up, gate)
    want = []
    for u, g in zip(up, gate):
        u = min(max(u, -7.0), 7.0)
        g = min(g, 7.0)
        want.append(u * g / (1 + math.exp(-g)))
    np.testing.assert_allclose(out, want, rtol=1e-12)


def test_expert_kernels_match_per_expert_composition():
    rng = np.random.default_rng(5)
    e_n, hid, inter, topk, t = 4, 32, 16, 2, 3
    ug = _rand_packed(rng, (e_n, 2 * inter, hid))
    ug_a = rng.uniform(0.01, 0.05, (e_n, 2 * inter))
    dn = _rand_packed(rng, (e_n, hid, inter))
    dn_a = rng.uniform(0.01, 0.05, (e_n, hid))
    x = rng.standard_normal((t, hid))
    ids = np.array([[0, 3], [1, 1], [2, 0]])
    w = np.array([[0.6, 0.4], [0.5, 0.5], [0.2, 0.8]])
    h = ok.ternary_expert_swiglu(x, ug, ug_a, ids)
    y = ok.ternary_expert_down_sum(h, dn, dn_a, ids, w, residual=x)
    for ti in range(t):
        acc = x[ti].copy()
        for j in range(topk):
            e = ids[ti, j]
            up = ok.ternary_gemv(x[ti], ug[e, :inter], ug_a[e, :inter])
            gate = ok.ternary_gemv(x[ti], ug[e, inter:], ug_a[e, inter:])
            hh = ok.swiglu_act(up, gate)
            np.testing.assert_allclose(h[ti, j], hh, rtol=1e-12, atol=1e-15)
            acc += w[ti, j] * ok.ternary_gemv(hh, dn[e], dn_a[e])
        np.testing.assert_allclose(y[ti], acc, rtol=1e-12, atol=1e-12)
    eo = ok.ternary_expert_gemv(h, dn, dn_a, ids)
    np.testing.assert_allclose(ok.moe_reduce_add(eo, w, x), y, rtol=1e-12, atol=1e-12)


def test_rtn4_gemv_brute_force_and_embedding():
    rng = np.random.default_rng(6)
    codes = rng.integers(0, 16, (3, 128), dtype=np.uint32)
    packed = pack.pack_4bit(codes)
    scales = rng.uniform(0.01, 0.1, (3, 2)).astype(np.float32)
    biases = rng.uniform(-0.5, 0.0, (3, 2)).astype(np.float32)
    x = rng.standard_normal((2, 128))
    y = ok.rtn4_gemv(x, packed, scales, biases, group_size=64)
    for b in range(2):
        for n in range(3):
            want = sum((int(codes[n, k]) * float(scales[n, k // 64]) + float(biases[n, k // 64])) * x[b, k]
                       for k in range(128))
            assert abs(y[b, n] - want) < 1e-9
    emb = ok.rtn4_embedding(np.array([2, 0]), packed, scales, biases, group_size=64)
    assert emb[0, 70] == np.float32(codes[2, 70] * scales[2, 1] + biases[2, 1])
    y_kn = ok.rtn4_gemv(x, packed.T.copy(), scales.T.copy(), biases.T.copy(), group_size=64, packed_kn=True)
    np.testing.assert_allclose(y_kn, y, rtol=0, atol=1e-12)


def test_norms_known_values():
    x = np.array([[3.0, 4.0]])
    y = ok.rms_norm(x, np.array([1.0, 2.0]), eps=0.0)
    r = math.sqrt(12.5)
    np.testing.assert_allclose(y, [[3 / r, 8 / r]], rtol=1e-12)
    s, n = ok.add_rms_norm(np.array([[1.0, 1.0]]), np.array([[2.0, 3.0]]), np.ones(2), eps=0.0)
    np.testing.assert_allclose(s, [[3.0, 4.0]])
    np.testing.assert_allclose(n, [[3 / r, 4 / r]], rtol=1e-12)


def test_moe_block_composition():
    rng = np.random.default_rng(7)
    e_n, hid, inter = 4, 32, 16
    gw = rng.standard_normal((e_n, hid))
    ug = _rand_packed(rng, (e_n, 2 * inter, hid))
    ug_a = rng.uniform(0.01, 0.05, (e_n, 2 * inter))
    dn = _rand_packed(rng, (e_n, hid, inter))
    dn_a = rng.uniform(0.01, 0.05, (e_n, hid))
    x = rng.standard_normal((2, hid))
    y, ids, wts, _ = ok.moe_block(x, gw, ug, ug_a, dn, dn_a, 2, round_bf16=False)
    h = ok.ternary_expert_swiglu(x, ug, ug_a, ids)
    np.testing.assert_allclose(y, ok.ternary_expert_down_sum(h, dn, dn_a, ids, wts), rtol=1e-6, atol=1e-9)
