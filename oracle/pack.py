"""Packing formats of the hot path (NumPy restatement; test infrastructure).

Follows reference ``src/maple_run/pack.py``:

* 2-bit ternary codes, 16 per uint32, LSB first: code i of a word sits in bits
  ``2i .. 2i+1``; the value is ``code - 1`` (``pack.py:17-45``).
* 4-bit RTN codes, 8 per uint32, LSB first, nibble i in bits ``4i .. 4i+3``
  (``pack.py:19-20,48-64``).
* Affine RTN ``w ~= q * scale + bias`` with ``bias`` = group minimum
  (``pack.py:67-117``).
* Row-wise ternarisation (``pack.py:120-149``).

Pinned by the reference's known-answer words (``tests/test_pack.py:26-52,
102-111``, kept as fixtures in ``tests/golden/pack_kats.json``), round-trip
identities, and the closed-form invariants of ``tests/test_pack.py:55-136``.
"""

from __future__ import annotations

import numpy as np

THRESHOLD_SCALE = 0.7   # pack.py:12
TERNARY_GROUP = 128     # pack.py:13 (K must be a multiple of this to ternarize)
HEAD_GROUP = 64         # pack.py:14 (default RTN group)
HEAD_BITS = 4           # pack.py:15


def pack_2bit(codes: np.ndarray) -> np.ndarray:
    """Pack codes in ``[0, 4)`` along the last axis, 16 per uint32, LSB first.

    Follows ``pack.py:23-38``: code ``i`` of each group of 16 lands in bits
    ``2i..2i+1``.  Written as a shift-and-OR loop rather than a sum.
    """
    *lead, k = codes.shape
    if k % 16:
        raise ValueError(f"2-bit packing requires the last axis to be a multiple of 16; got {k}.")
    c = codes.astype(np.uint32, copy=False).reshape(*lead, k // 16, 16)
    out = np.zeros((*lead, k // 16), dtype=np.uint32)
    for i in range(16):
        out |= (c[..., i] & np.uint32(3)) << np.uint32(2 * i)
    return out


def unpack_2bit(packed: np.ndarray) -> np.ndarray:
    """Inverse of ``pack_2bit`` (``pack.py:41-45``): ``nwords`` -> ``16*nwords`` codes."""
    p = np.asarray(packed).astype(np.uint32, copy=False)
    shifts = np.arange(0, 32, 2, dtype=np.uint32)
    codes = (p[..., None] >> shifts) & np.uint32(3)
    return codes.reshape(*p.shape[:-1], p.shape[-1] * 16)


def pack_4bit(codes: np.ndarray) -> np.ndarray:
    """Pack codes in ``[0, 16)``, 8 per uint32, LSB first (``pack.py:48-57``)."""
    *lead, k = codes.shape
    if k % 8:
        raise ValueError(f"4-bit packing requires the last axis to be a multiple of 8; got {k}.")
    c = codes.astype(np.uint32, copy=False).reshape(*lead, k // 8, 8)
    out = np.zeros((*lead, k // 8), dtype=np.uint32)
    for i in range(8):
        out |= (c[..., i] & np.uint32(15)) << np.uint32(4 * i)
    return out


def unpack_4bit(packed: np.ndarray) -> np.ndarray:
    """Inverse of ``pack_4bit`` (``pack.py:60-64``)."""
    p = np.asarray(packed).astype(np.uint32, copy=False)
    shifts = np.arange(0, 32, 4, dtype=np.uint32)
    codes = (p[..., None] >> shifts) & np.uint32(15)
    return codes.reshape(*p.shape[:-1], p.shape[-1] * 8)


def quantize_rtn(weight: np.ndarray, group_size: int = HEAD_GROUP, bits: int = HEAD_BITS):
    """Affine round-to-nearest along the last axis (``pack.py:67-100``).

    Per group: ``scale = (max - min) / 15``, ``bias = min``,
    ``q = clip(rint((w - min) / scale), 0, 15)``; a constant group gets
    ``scale = 0`` and ``q = 0``.  Returns ``(packed, scales, biases)`` with
    float32 scales/biases of shape ``[..., K / group_size]``.
    """
    if bits != HEAD_BITS:
        raise ValueError(f"Only {HEAD_BITS}-bit RTN is implemented; got {bits}.")
    k = weight.shape[-1]
    if k % group_size:
        raise ValueError(
            f"RTN conversion requires the last axis to be a multiple of {group_size}; got {k}."
        )
    levels = np.float32(15.0)
    w = weight.astype(np.float32, copy=False)
    g = w.reshape(*w.shape[:-1], k // group_size, group_size)
    lo = g.min(axis=-1, keepdims=True)
    hi = g.max(axis=-1, keepdims=True)
    scale = (hi - lo) / levels
    flat = scale == 0
    q = np.clip(np.rint((g - lo) / np.where(flat, np.float32(1.0), scale)), 0, levels)
    q = np.where(flat, 0, q)
    packed = pack_4bit(q.reshape(*w.shape[:-1], k).astype(np.uint32))
    return packed, scale[..., 0].astype(np.float32), lo[..., 0].astype(np.float32)


def dequantize_rtn(packed, scales, biases, group_size: int = HEAD_GROUP, bits: int = HEAD_BITS):
    """``q * scale + bias`` per group, float32 (``pack.py:103-117``)."""
    if bits != HEAD_BITS:
        raise ValueError(f"Only {HEAD_BITS}-bit RTN is implemented; got {bits}.")
    q = unpack_4bit(packed).astype(np.float32)
    k = q.shape[-1]
    g = q.reshape(*q.shape[:-1], k // group_size, group_size)
    rec = g * np.asarray(scales, np.float32)[..., None] + np.asarray(biases, np.float32)[..., None]
    return rec.reshape(q.shape)


def ternarize(weight: np.ndarray, threshold_scale: float = THRESHOLD_SCALE):
    """Row-wise ternarisation (``pack.py:120-149``).

    ``thr = threshold_scale * mean|w|`` per row; ``mask = |w| > thr``;
    ``alpha = sum(|w| * mask) / max(sum(mask), 1)`` cast back to the weight
    dtype; codes ``sign(w) * mask + 1`` packed 16 per uint32.
    """
    if weight.shape[-1] % TERNARY_GROUP:
        raise ValueError(
            "Ternary conversion requires the reduction dim to be a multiple of "
            f"{TERNARY_GROUP}; got {weight.shape[-1]}."
        )
    w = weight.astype(np.float32, copy=False)
    aw = np.abs(w)
    thr = np.float32(threshold_scale) * aw.mean(axis=-1, keepdims=True)
    keep = (aw > thr).astype(np.float32)
    alpha = (aw * keep).sum(axis=-1) / np.maximum(keep.sum(axis=-1), 1)
    codes = (np.sign(w) * keep + 1).astype(np.uint32)
    return pack_2bit(codes), alpha.astype(weight.dtype, copy=False)


def ternary_values(packed: np.ndarray) -> np.ndarray:
    """Dequantised ternary values ``code - 1`` as float64 (code 3 -> +2, as in
    ``ternary_gemv.py:126-128``)."""
    return unpack_2bit(packed).astype(np.float64) - 1.0
