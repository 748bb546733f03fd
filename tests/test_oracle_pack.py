"""The oracle's packing formats against the reference's known answers (CPU).

Fixtures in ``tests/golden/pack_kats.json`` restate the words and values the
reference's own tests assert (``tests/test_pack.py``, ``tests/test_ternary_gemv.py``).
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import kernels as ok
from oracle import pack

KATS = json.loads((Path(__file__).parent / "golden" / "pack_kats.json").read_text())


def _codes(entry):
    shape = entry["shape"]
    c = np.full(shape, entry["default_code"], dtype=np.uint32)
    for k, v in entry["codes_nonone"].items():
        c[0, int(k)] = v
    return c


def test_pack_2bit_kat_k128():
    e = KATS["pack_2bit_k128"]
    codes = _codes(e)
    packed = pack.pack_2bit(codes)
    assert packed.dtype == np.uint32 and packed.shape == (1, 8)
    assert packed[0].tolist() == e["words"]
    np.testing.assert_array_equal(pack.unpack_2bit(packed), codes)


def test_pack_2bit_kat_one_word():
    e = KATS["pack_2bit_one_word"]
    codes = np.array(e["codes"], dtype=np.uint32).reshape(1, 16)
    packed = pack.pack_2bit(codes)
    assert int(packed[0, 0]) == e["word"]
    np.testing.assert_array_equal(pack.unpack_2bit(packed), codes)


def test_pack_4bit_kat():
    e = KATS["pack_4bit"]
    codes = _codes(e)
    packed = pack.pack_4bit(codes)
    assert packed.shape == (1, 8)
    assert int(packed[0, 0]) == e["word0"]
    np.testing.assert_array_equal(pack.unpack_4bit(packed), codes)


def test_pack_rejects_ragged_k():
    with pytest.raises(ValueError, match="multiple of 16"):
        pack.pack_2bit(np.zeros((1, 20), np.uint32))
    with pytest.raises(ValueError, match="multiple of 8"):
        pack.pack_4bit(np.zeros((1, 12), np.uint32))


def test_roundtrips_random():
    rng = np.random.default_rng(0)
    c2 = rng.integers(0, 4, (5, 7, 64), dtype=np.uint32)
    np.testing.assert_array_equal(pack.unpack_2bit(pack.pack_2bit(c2)), c2)
    c4 = rng.integers(0, 16, (3, 40), dtype=np.uint32)
    np.testing.assert_array_equal(pack.unpack_4bit(pack.pack_4bit(c4)), c4)


def test_unpack_2bit_closed_form():
    """code i of word w is (w >> 2i) & 3 -- checked word by word in Python."""
    rng = np.random.default_rng(1)
    words = rng.integers(0, 2**32, (3, 4), dtype=np.uint64).astype(np.uint32)
    codes = pack.unpack_2bit(words)
    for r in range(3):
        for wi in range(4):
            w = int(words[r, wi])
            assert [int(c) for c in codes[r, wi * 16:(wi + 1) * 16]] == [(w >> (2 * i)) & 3 for i in range(16)]


def _expected_ternary(w, scale=0.7):
    aw = np.abs(w.astype(np.float32))
    thr = scale * aw.mean(axis=-1, keepdims=True)
    return np.sign(w) * (aw > thr)


def test_ternarize_codes_match_sign_mask():
    rng = np.random.default_rng(0)
    w = rng.standard_normal((32, 128)).astype(np.float32)
    packed, alpha = pack.ternarize(w)
    assert packed.shape == (32, 8) and alpha.shape == (32,) and alpha.dtype == w.dtype
    codes = pack.unpack_2bit(packed)
    assert set(np.unique(codes).tolist()) == {0, 1, 2}
    np.testing.assert_array_equal(codes.astype(np.float32) - 1, _expected_ternary(w))


def test_ternarize_alpha_is_mean_abs_of_survivors():
    rng = np.random.default_rng(1)
    w = rng.standard_normal((8, 256)).astype(np.float32)
    _, alpha = pack.ternarize(w)
    aw = np.abs(w)
    mask = aw > 0.7 * aw.mean(axis=-1, keepdims=True)
    for r in range(8):
        assert alpha[r] == pytest.approx(float(aw[r][mask[r]].mean()), rel=1e-6)


def test_ternarize_zero_rows_and_group_check():
    e = KATS["ternarize_zero_rows"]
    packed, alpha = pack.ternarize(np.zeros(e["shape"], np.float32))
    np.testing.assert_array_equal(pack.unpack_2bit(packed), np.full(e["shape"], e["codes"], np.uint32))
    np.testing.assert_array_equal(alpha, np.full(e["shape"][0], e["alpha"], np.float32))
    with pytest.raises(ValueError, match="multiple"):
        pack.ternarize(np.ones((4, 64), np.float32))


def test_ternarize_3d_stack():
    rng = np.random.default_rng(2)
    w = rng.standard_normal((4, 16, 128)).astype(np.float32)
    packed, alpha = pack.ternarize(w)
    assert packed.shape == (4, 16, 8) and alpha.shape == (4, 16)
    np.testing.assert_array_equal(pack.unpack_2bit(packed).astype(np.float32) - 1, _expected_ternary(w))


def test_rtn_roundtrip_within_half_scale():
    rng = np.random.default_rng(3)
    w = rng.standard_normal((16, 64)).astype(np.float32)
    packed, scales, biases = pack.quantize_rtn(w)
    assert packed.shape == (16, 8) and scales.shape == (16, 1)
    rec = pack.dequantize_rtn(packed, scales, biases)
    codes = pack.unpack_4bit(packed)
    assert codes.min() >= 0 and codes.max() <= 15
    assert np.all(np.abs(rec - w) <= 0.5 * scales + 1e-5)


def test_rtn_group_min_max_reconstructed_exactly():
    """bias is the group minimum (code 0) and the maximum is code 15."""
    rng = np.random.default_rng(4)
    w = rng.standard_normal((3, 256)).astype(np.float32)
    packed, scales, biases = pack.quantize_rtn(w, group_size=128)
    codes = pack.unpack_4bit(packed).reshape(3, 2, 128)
    g = w.reshape(3, 2, 128)
    np.testing.assert_array_equal(biases, g.min(-1))
    np.testing.assert_array_equal(codes[np.arange(3)[:, None], np.arange(2)[None, :], g.argmax(-1)], 15)
    np.testing.assert_array_equal(codes[np.arange(3)[:, None], np.arange(2)[None, :], g.argmin(-1)], 0)


def test_bf16_round_known_values():
    vals = np.array([1.0, 1.0 + 2**-8, 1.0 + 3 * 2**-8, -2.5, 1e-40, np.inf], np.float32)
    out = ok.bf16_round(vals)
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7: ties go to the even mantissa (1.0);
    # 1 + 3*2^-8 ties between 1+2^-7 and 1+2^-6: even is 1 + 2^-6.
    np.testing.assert_array_equal(out[:4], np.array([1.0, 1.0, 1.0 + 2**-6, -2.5], np.float32))
    assert out[5] == np.inf


def _pairwise_f32(a: np.ndarray) -> np.float32:
    """NumPy's float32 pairwise summation restated step by step -- the order
    the device ternarisation (csrc/ternarize.hip) uses for its means and sums."""
    n = len(a)
    if n < 8:
        r = np.float32(0)
        for x in a:
            r = np.float32(r + x)
        return r
    if n <= 128:
        r = [np.float32(a[j]) for j in range(8)]
        i = 8
        while i < n - n % 8:
            for j in range(8):
                r[j] = np.float32(r[j] + a[i + j])
            i += 8
        res = np.float32(np.float32(np.float32(r[0] + r[1]) + np.float32(r[2] + r[3]))
                         + np.float32(np.float32(r[4] + r[5]) + np.float32(r[6] + r[7])))
        while i < n:
            res = np.float32(res + a[i])
            i += 1
        return res
    n2 = n // 2
    n2 -= n2 % 8
    return np.float32(_pairwise_f32(a[:n2]) + _pairwise_f32(a[n2:]))


@pytest.mark.parametrize("k", [128, 384, 640, 768, 2048, 4096])
def test_pairwise_order_is_numpys(k):
    """The summation order the device ternarisation follows gives the bits of
    NumPy's float32 np.sum and np.mean over a row (the reference's mean|w| and
    sum(|w| * mask)); a first-element start, a plausible alternative, differs."""
    rng = np.random.default_rng(k)
    differs = 0
    for t in range(24):
        a = np.abs(rng.standard_normal(k).astype(np.float32) * np.float32(10.0 ** rng.uniform(-3, 3)))
        s = _pairwise_f32(a)
        assert s == np.sum(a[None, :], axis=-1)[0]
        assert np.float32(s / np.float32(k)) == np.mean(a[None, :], axis=-1, keepdims=True)[0, 0]
        differs += np.float32(a[0] + _pairwise_f32(a[1:])) != s
    assert differs > 0
