"""Pins for the decoder pieces of the oracle (CPU only).

RoPE and attention are checked through properties the mathematics fixes, so a
dropped term, a wrong sign or a wrong head-to-KV mapping in the oracle fails:
rotate-half RoPE (reference src/maple_run/model.py:48-92) preserves the norm,
is the identity at position 0, and makes q(a).k(b) depend on a - b only;
GQA (src/maple_run/kernels/decode_attn.py:167-359) gives the mean of V for
equal scores, picks V's row for a dominant key, maps query head h to KV head
h // group, and reads only the last ``window`` positions.

Those properties hold for either rotation direction and any score scale, so
known answers fix the rest: the rotation direction and the half split of
rotate-half (``_rotate_half`` = cat(-x2, x1), ``q cos + rotate_half(q) sin``,
model.py:48-61), the layer's score scale head_dim ** -0.5 (model.py:343,
through ``attend_row``), and P rounded to bf16 before P V with the sum over
the unrounded P (decode_attn.py:270-289).
"""

from __future__ import annotations

import math

import numpy as np
import pytest

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


def test_rope_known_answer_direction_and_pairing():
    """rotary_dim 2 at position p: (1, 0) -> (cos p, sin p) and (0, 1) ->
    (-sin p, cos p) (inv_freq_0 = theta^0 = 1).  rotary_dim 4 of head_dim 8:
    dim i pairs with dim i + 2 (the halves, not neighbours), dim 1 turning at
    theta^(-1/2) per position; dims 4.. pass through."""
    for p in (1, 5, 1000):
        for x, want in (((1.0, 0.0), (math.cos(p), math.sin(p))),
                        ((0.0, 1.0), (-math.sin(p), math.cos(p)))):
            xs = np.array(x) * math.sqrt(2.0)  # unit RMS: the norm step is the identity
            got = _rope(xs, p, rot=2)
            np.testing.assert_allclose(got / math.sqrt(2.0), want, atol=2e-6)
    theta, p = 1e4, 7
    w1 = p * theta ** -0.5
    x = np.zeros(8)
    x[1] = math.sqrt(8.0)  # unit RMS
    got = _rope(x, p, rot=4, theta=theta) / math.sqrt(8.0)
    want = np.zeros(8)
    want[1], want[3] = math.cos(w1), math.sin(w1)
    np.testing.assert_allclose(got, want, atol=2e-6)
    x = np.zeros(8)
    x[2] = math.sqrt(8.0)
    got = _rope(x, p, rot=4, theta=theta) / math.sqrt(8.0)
    want = np.zeros(8)
    want[0], want[2] = -math.sin(p), math.cos(p)
    np.testing.assert_allclose(got, want, atol=2e-6)


def test_gqa_rounds_p_to_bf16_and_sums_unrounded():
    """Two keys with p = (1, 1/3): P V uses bf16(1/3) = 171/512 and the sum
    uses 1 + 1/3, so with V = (0, 1) the output is (171/512) / (4/3)."""
    q = np.array([[1.0]])
    k = np.array([[[0.0], [math.log(1.0 / 3.0)]]])
    v = np.array([[[0.0], [1.0]]])
    out = od.gqa(q, k, v, 2, 1.0)
    assert abs(out[0, 0] - (171 / 512) * 0.75) < 1e-14


@pytest.mark.parametrize("d", [4, 64])
def test_attend_row_scale_is_inverse_sqrt_head_dim(d):
    """One query head over two positions: the cached key at position 0 is
    orthogonal to q (score 0), the new key equals q (q.k = d after the unit
    RMS norm), so the scores are (0, d * scale) = (0, sqrt(d)) for the
    reference's scale and the output is the softmax weights on V = (e_0, e_1),
    P rounded to bf16 as above."""
    c = dict(heads=1, kv_heads=1, head_dim=d, rotary_dim=0, eps=0.0,
             cos=np.ones((4, 1)), sin=np.zeros((4, 1)))
    L = dict(q_norm=np.ones(d), k_norm=np.ones(d))
    ones = np.ones(d)
    v_new = np.zeros(d)
    v_new[1] = 1.0
    row = np.concatenate([ones, ones, v_new])
    k_rows = np.zeros((1, 4, d))
    v_rows = np.zeros((1, 4, d))
    k_rows[0, 0] = np.where(np.arange(d) % 2 == 0, 1.0, -1.0)
    v_rows[0, 0, 0] = 1.0
    out = od.attend_row(row, L, c, k_rows, v_rows, 1)
    s1 = math.sqrt(d)
    p0 = math.exp(-s1)
    want = np.zeros(d)
    want[0] = float(od.bf(np.array([p0]))[0]) / (1.0 + p0)
    want[1] = 1.0 / (1.0 + p0)
    np.testing.assert_allclose(out, want, rtol=0, atol=1e-14)
    np.testing.assert_array_equal(k_rows[0, 1], ones)  # the new k written at pos 1
    np.testing.assert_array_equal(v_rows[0, 1], v_new)
