"""Device-side ternarisation, the converter's step (reference
``src/maple_run/pack.py:120-149``), through ``ma_ternarize``.

``ternarize(weight)`` takes a CUDA tensor ``[..., N, K]`` (float32, bfloat16
or float16; K a multiple of 128) and returns ``(packed uint32 [..., N, K /
16], row_alpha [..., N])`` in the weight's dtype: per row thr =
threshold_scale * mean|w|, mask = |w| > thr, alpha = sum(|w| * mask) /
max(sum(mask), 1), codes sign(w) * mask + 1 packed 16 per uint32, least
significant first.  The means and sums follow NumPy's float32 pairwise order,
so the outputs are the bits of the reference's NumPy converter.
"""

from __future__ import annotations

import torch

from . import _lib

DEFAULT_THRESHOLD_SCALE = 0.7  # pack.py:12
GROUP_SIZE = 128               # pack.py:13


def ternarize(weight: torch.Tensor, threshold_scale: float = DEFAULT_THRESHOLD_SCALE):
    if weight.shape[-1] % GROUP_SIZE:
        raise ValueError(
            f"Ternary conversion requires the reduction dim to be a multiple of {GROUP_SIZE}; "
            f"got {weight.shape[-1]}.")
    if not weight.is_cuda:
        raise RuntimeError("ternarize requires a CUDA tensor.")
    k_in = int(weight.shape[-1])
    w = weight.contiguous()
    rows = w.numel() // k_in
    packed = torch.empty(*weight.shape[:-1], k_in // 16, device=w.device, dtype=torch.uint32)
    alpha = torch.empty(*weight.shape[:-1], device=w.device, dtype=w.dtype)
    _lib.call("ma_ternarize", _lib.ptr(w), _lib.dtype_code(w, "weight"), rows, k_in,
              float(threshold_scale), _lib.ptr(packed), _lib.ptr(alpha), _lib.stream_of(w))
    return packed, alpha
