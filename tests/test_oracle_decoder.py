"""Pins for the decoder pieces of the oracle (CPU only).

RoPE and attention are checked through properties the mathematics fixes, so a
dropped term, a wrong sign or a wrong head-to-KV mapping in the oracle fails:
rotate-half RoPE (reference src/maple_run/model.py:48-92) preserves the norm,
is the identity at position 0, and makes q(a).k(b) depend on a - b only;
GQA (src/maple_run/kernels/decode_attn.py:167-359) gives the mean of V for
equal scores, picks V's row for a dominant key, maps query head h to KV head
h // group, and reads only the last ``window`` positions.
"""

from __future__ import annotations

import numpy as np

from oracle import decoder as od


def _rope(x, pos, rot=32, theta=1e4):
    cos, sin = od.rope_tables(pos + 1, rot, theta)
    return od.head_norm_rope(x, np.ones(x.size), cos[pos].astype(np.float64),
                             sin[pos].astype(np.float64), rot, 0.0)


def test_rope_tables_match_angles():
    cos, sin = od.rope_tables(100, 32, 1e4)
    inv = 1e4 ** (-np.arange(0, 32, 2) / 32)
    ang = 77 * inv
    np.testing.assert_allclose(cos[77, :16], np.cos(ang), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(sin[77, 16:], np.sin(ang), rtol=1e-5, atol=1e-6)


def test_rope_identity_at_zero_and_norm_preserving():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(64)
    x /= np.sqrt(np.mean(x * x))  # unit RMS so the norm step is the identity
    np.testing.assert_allclose(_rope(x, 0), x, atol=1e-12)
    y = _rope(x, 1234)
    np.testing.assert_allclose(np.linalg.norm(y[:32]), np.linalg.norm(x[:32]), rtol=1e-5)
    np.testing.assert_array_equal(y[32:], x[32:])  # pass-through dims


def test_rope_scores_depend_on_relative_position_only():
    rng = np.random.default_rng(1)
    q, k = rng.standard_normal(64), rng.standard_normal(64)
    q /= np.sqrt(np.mean(q * q))
    k /= np.sqrt(np.mean(k * k))
    s1 = _rope(q, 40) @ _rope(k, 30)
    s2 = _rope(q, 1010) @ _rope(k, 1000)
    s3 = _rope(q, 41) @ _rope(k, 30)
    assert abs(s1 - s2) < 1e-4 * (1 + abs(s1))
    assert abs(s1 - s3) > 1e-3  # and it does depend on the offset


def test_rms_head_norm_scale():
    x = np.full(64, 3.0)
    y = od.head_norm_rope(x, np.full(64, 2.0), None, None, 0, 0.0)
    np.testing.assert_allclose(y, 2.0)


def test_gqa_uniform_scores_give_mean_and_group_mapping():
    nq, nkv, d, n = 8, 2, 4, 5
    q = np.zeros((nq, d))
    v = np.stack([np.arange(n * d, dtype=np.float64).reshape(n, d) + 1000 * g for g in range(nkv)])
    k = np.zeros((nkv, n, d))
    out = od.gqa(q, k, v, n, 1.0)
    for h in range(nq):
        np.testing.assert_allclose(out[h], v[h // (nq // nkv)].mean(axis=0))


def test_gqa_dominant_key_and_window():
    nq, nkv, d, n = 4, 1, 4, 10
    rng = np.random.default_rng(2)
    v = rng.standard_normal((nkv, n, d))
    k = np.zeros((nkv, n, d))
    k[0, 6] = 50.0
    q = np.ones((nq, d))
    out = od.gqa(q, k, v, n, 1.0)
    np.testing.assert_allclose(out, np.repeat(v[0, 6][None], nq, 0), atol=1e-12)
    # window 3 over kv_len 10 reads positions 7, 8, 9 only: key 6 is outside
    out_w = od.gqa(q, k, v, n, 1.0, window=3)
    np.testing.assert_allclose(out_w, np.repeat(v[0, 7:10].mean(0)[None], nq, 0), atol=1e-12)
