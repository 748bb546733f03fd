"""RMSNorm, residual + RMSNorm and the MoE top-k combine, one launch each.

Drop-ins for reference ``src/maple_run/kernels/fused_norm.py``: ``rms_norm``
(:105-125), ``add_rms_norm`` (:128-161), ``moe_reduce_add`` (:164-202).
"""

from __future__ import annotations

import torch

from .. import _lib


def _rows_and_n(x: torch.Tensor) -> tuple[int, int]:
    n = int(x.shape[-1])
    return (int(x.numel() // n) if n else 0), n


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm over the last dim; compute in fp32, store in ``x.dtype``."""
    if not x.is_cuda:
        raise RuntimeError("rms_norm requires CUDA tensors.")
    rows, n = _rows_and_n(x)
    x_mat = x.reshape(rows, n).contiguous()
    y = torch.empty_like(x_mat)
    w = weight.reshape(-1)
    if w.numel() != n:
        raise ValueError(f"rms_norm weight has {w.numel()} elements, expected {n}.")
    w = w.contiguous()
    _lib.call(
        "ma_rms_norm", _lib.ptr(x_mat), _lib.dtype_code(x_mat, "x"), rows, n,
        _lib.ptr(w), _lib.dtype_code(w, "weight"), float(eps), _lib.ptr(y), _lib.stream_of(x),
    )
    return y.reshape(x.shape)


def add_rms_norm(
    x: torch.Tensor, y: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6
) -> tuple[torch.Tensor, torch.Tensor]:
    """``residual = x + y`` and ``norm = rms_norm(residual)`` in one launch."""
    if not x.is_cuda or not y.is_cuda:
        raise RuntimeError("add_rms_norm requires CUDA tensors.")
    if x.shape != y.shape:
        raise ValueError(f"add_rms_norm shape mismatch {tuple(x.shape)} vs {tuple(y.shape)}.")
    if x.dtype != y.dtype:
        raise TypeError(f"add_rms_norm dtype mismatch {x.dtype} vs {y.dtype}.")
    rows, n = _rows_and_n(x)
    x_mat = x.reshape(rows, n).contiguous()
    y_mat = y.reshape(rows, n).contiguous()
    residual = torch.empty_like(x_mat)
    normed = torch.empty_like(x_mat)
    w = weight.reshape(-1)
    if w.numel() != n:
        raise ValueError(f"add_rms_norm weight has {w.numel()} elements, expected {n}.")
    w = w.contiguous()
    _lib.call(
        "ma_add_rms_norm", _lib.ptr(x_mat), _lib.ptr(y_mat), _lib.dtype_code(x_mat, "x"), rows, n,
        _lib.ptr(w), _lib.dtype_code(w, "weight"), float(eps), _lib.ptr(residual),
        _lib.ptr(normed), _lib.stream_of(x),
    )
    return residual.reshape(x.shape), normed.reshape(x.shape)


def moe_reduce_add(
    expert_out: torch.Tensor,
    topk_weight: torch.Tensor,
    residual: torch.Tensor | None = None,
) -> torch.Tensor:
    """``y = (expert_out * topk_weight).sum(topk) [+ residual]`` in one launch."""
    if expert_out.ndim < 2:
        raise ValueError("expert_out must be [..., topk, N].")
    if not expert_out.is_cuda:
        raise RuntimeError("moe_reduce_add requires CUDA tensors.")
    topk = int(expert_out.shape[-2])
    n = int(expert_out.shape[-1])
    if tuple(topk_weight.shape) != tuple(expert_out.shape[:-1]):
        raise ValueError("topk_weight must match expert_out without the last dim.")
    tokens = int(expert_out.numel() // (topk * n)) if topk * n else 0
    x = expert_out.reshape(tokens, topk, n).contiguous()
    w = topk_weight.reshape(tokens, topk).float().contiguous()
    y = torch.empty(tokens, n, device=expert_out.device, dtype=expert_out.dtype)
    res = None
    if residual is not None:
        res = residual.reshape(tokens, n).contiguous()
    _lib.call(
        "ma_moe_reduce_add", _lib.ptr(x), _lib.dtype_code(x, "expert_out"), tokens, topk, n,
        _lib.ptr(w), _lib.ptr(res), _lib.dtype_code(res, "residual") if res is not None else 0,
        _lib.ptr(y), _lib.stream_of(expert_out),
    )
    return y.reshape(*expert_out.shape[:-2], n)
