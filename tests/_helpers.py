"""Comparison helpers shared by the GPU parity tests."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch

# bf16 carries 8 significant bits: one ulp is 2^-7 of the leading power of two,
# so 2^-8 relative is half an ulp to one ulp depending on the mantissa.
BF16_RTOL = 2.0 ** -8


def np_f(t: torch.Tensor) -> np.ndarray:
    """Device tensor -> float64 NumPy (exact for bf16/fp32)."""
    return t.detach().float().cpu().numpy().astype(np.float64)


def np_u32(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.int32).cpu().numpy().view(np.uint32)


def assert_bf16_close(y, ref, *, rtol=BF16_RTOL, atol_frac=1e-3, what=""):
    """Elementwise ``|y - ref| <= rtol*|ref| + atol_frac*max|ref|`` and
    ``max|y - ref| / max|ref| <= 1e-2`` (the path's stated bf16 tolerance)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    assert y.shape == ref.shape, (what, y.shape, ref.shape)
    scale = max(float(np.abs(ref).max()), 1e-30)
    err = np.abs(y - ref)
    bound = rtol * np.abs(ref) + atol_frac * scale
    bad = err > bound
    assert not bad.any(), (
        f"{what}: {int(bad.sum())} of {bad.size} elements outside tolerance; worst "
        f"err {err.max():.4g} at ref scale {scale:.4g}"
    )
    assert err.max() / scale <= 1e-2, f"{what}: max rel err {err.max() / scale:.3g}"


def assert_f32_close(y, ref, *, rtol=1e-4, atol=1e-4, what=""):
    np.testing.assert_allclose(np.asarray(y, np.float64), np.asarray(ref, np.float64),
                               rtol=rtol, atol=atol, err_msg=what)


def tie_safe_rows(probs: np.ndarray, k: int, gap: float = 1e-5) -> np.ndarray:
    """Rows whose top-(k+1) sorted probabilities are separated by more than
    ``gap`` (relative): there the ids are fixed regardless of float32
    summation order, so they must match exactly."""
    p = np.sort(probs.reshape(-1, probs.shape[-1]), axis=-1)[:, ::-1][:, : k + 1]
    d = (p[:, :-1] - p[:, 1:]) / np.maximum(p[:, :-1], 1e-30)
    return (d > gap).all(axis=1)


# Router bias of the Zipf(1.1)-skewed workloads (64 experts, top-8) and the
# expert load it is fitted to: tests/golden/make_zipf_bias.py.
ZIPF = json.loads((Path(__file__).parent / "golden" / "zipf_bias_e64.json").read_text())


def zipf_bias(device) -> torch.Tensor:
    return torch.tensor(ZIPF["bias"], dtype=torch.float32, device=device)


def load_tv_distance(ids: np.ndarray, n_experts: int = 64) -> float:
    """Total-variation distance between the share of (token, slot) pairs each
    expert received and the fixture's target shares."""
    c = np.bincount(np.asarray(ids).reshape(-1), minlength=n_experts).astype(np.float64)
    return 0.5 * float(np.abs(c / c.sum() - np.asarray(ZIPF["target_share"])).sum())
