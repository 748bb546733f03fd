"""Indexed stacked-expert ternary kernels: selected experts only, weights 3-D uint32.

Drop-ins for reference ``src/maple_run/kernels/ternary_expert.py``:
``ternary_expert_gemv`` (:125-234), ``ternary_expert_swiglu`` (:403-468) and
``ternary_expert_down_sum`` (:471-556), same signatures, shapes, dtypes and
exceptions.  One HIP launch each; expert ids stay on the device.
"""

from __future__ import annotations

import torch

from .. import _lib

_CODES_PER_WORD = 16
MLP_CLAMP = 7.0


def _expert_nk(packed_weight: torch.Tensor, packed_kn: bool) -> tuple[int, int, int]:
    """Return n_exp, n_out, nwords."""
    if packed_kn:
        n_exp, nwords, n_out = packed_weight.shape
    else:
        n_exp, n_out, nwords = packed_weight.shape
    return int(n_exp), int(n_out), int(nwords)


def _ids_arg(ids: torch.Tensor) -> tuple[torch.Tensor, int]:
    # The kernels' fast paths read int32 ids (the router's output dtype).
    if ids.dtype != torch.int32:
        ids = ids.to(torch.int32)
    return ids.contiguous(), 0


def _rows(t: torch.Tensor, k: int) -> torch.Tensor:
    m = t.reshape(-1, k)
    return m if m.stride(-1) == 1 else m.contiguous()


def ternary_expert_gemv(
    x: torch.Tensor,
    packed_weight: torch.Tensor,
    row_alpha: torch.Tensor,
    expert_ids: torch.Tensor,
    *,
    packed_kn: bool = False,
) -> torch.Tensor:
    """Indexed packed GEMV for stacked experts; returns ``expert_ids.shape + (N,)``.

    ``x`` is either one row per token (``[..., K]`` with ``expert_ids``
    ``[..., topk]``) or one row per slot (``x.shape[:-1] == expert_ids.shape``).
    """
    if packed_weight.ndim != 3:
        raise ValueError(
            f"packed_weight must be 3-D [E, N, K/16]; got shape {tuple(packed_weight.shape)}."
        )
    if packed_weight.dtype != torch.uint32:
        raise TypeError(
            f"packed_weight must be uint32 codes, got {packed_weight.dtype}; "
            "refusing to run a dense-weight path."
        )
    if not x.is_cuda or not packed_weight.is_cuda or not row_alpha.is_cuda:
        raise RuntimeError("ternary_expert_gemv requires CUDA tensors.")
    if not expert_ids.is_cuda:
        raise RuntimeError("expert_ids must be a CUDA tensor (no GPU→CPU routing).")
    n_exp, n_out, nwords = _expert_nk(packed_weight, packed_kn)
    k_in = nwords * _CODES_PER_WORD
    if x.shape[-1] != k_in:
        raise ValueError(f"x last dim {x.shape[-1]} != packed K ({k_in}).")
    if tuple(row_alpha.shape) != (n_exp, n_out):
        raise ValueError(f"row_alpha shape {tuple(row_alpha.shape)} != {(n_exp, n_out)}.")
    id_shape = tuple(expert_ids.shape)
    if tuple(x.shape[:-1]) == id_shape:
        x_div = 1
    elif tuple(x.shape[:-1]) == id_shape[:-1]:
        x_div = id_shape[-1]
        tokens = int(x.numel() // k_in)
        if tokens * x_div != expert_ids.numel():
            raise ValueError(f"x leading {x.shape[:-1]} incompatible with expert_ids {id_shape}.")
    else:
        raise ValueError(f"x shape {tuple(x.shape)} incompatible with expert_ids {id_shape}.")
    slots = int(expert_ids.numel())
    x_mat = _rows(x, k_in)
    ids, ids64 = _ids_arg(expert_ids.reshape(slots))
    y = torch.empty(slots, n_out, device=x.device, dtype=x.dtype)
    pw = packed_weight.contiguous()
    alpha = row_alpha.contiguous()
    _lib.call(
        "ma_ternary_expert_gemv",
        _lib.ptr(x_mat), _lib.dtype_code(x_mat, "x"), x_mat.stride(0) if x_mat.shape[0] else k_in,
        x_div, _lib.ptr(pw), n_exp, n_out, nwords, int(bool(packed_kn)),
        _lib.ptr(alpha), _lib.dtype_code(alpha, "row_alpha"), _lib.ptr(ids), ids64, slots,
        _lib.ptr(y), n_out, _lib.stream_of(x),
    )
    return y.reshape(*id_shape, n_out)


def ternary_expert_swiglu(
    x: torch.Tensor,
    packed_weight: torch.Tensor,
    row_alpha: torch.Tensor,
    expert_ids: torch.Tensor,
    *,
    packed_kn: bool = False,
) -> torch.Tensor:
    """Indexed up+gate GEMV with SiLU/clamp fused. Packed rows are ``[up; gate]``.

    ``x`` is per-token ``[..., K]``; ``expert_ids`` is ``[..., topk]``.
    Returns activated expert hidden ``[..., topk, N]`` with ``N = packed N / 2``.
    """
    if packed_weight.ndim != 3 or packed_weight.dtype != torch.uint32:
        raise ValueError("packed_weight must be uint32 [E, 2N, K/16] or [E, K/16, 2N].")
    if not x.is_cuda or not packed_weight.is_cuda or not expert_ids.is_cuda:
        raise RuntimeError("ternary_expert_swiglu requires CUDA tensors.")
    n_exp, n_rows, nwords = _expert_nk(packed_weight, packed_kn)
    if n_rows % 2 != 0:
        raise ValueError(f"packed up_gate rows must be even, got {n_rows}.")
    n_out = n_rows // 2
    k_in = nwords * _CODES_PER_WORD
    if x.shape[-1] != k_in:
        raise ValueError(f"x last dim {x.shape[-1]} != packed K ({k_in}).")
    if tuple(row_alpha.shape) != (n_exp, n_rows):
        raise ValueError(f"row_alpha shape {tuple(row_alpha.shape)} != {(n_exp, n_rows)}.")
    id_shape = tuple(expert_ids.shape)
    if tuple(x.shape[:-1]) != id_shape[:-1]:
        raise ValueError(f"x shape {tuple(x.shape)} incompatible with expert_ids {id_shape}.")
    topk = id_shape[-1]
    tokens = int(x.numel() // k_in)
    x_mat = _rows(x, k_in)
    ids, ids64 = _ids_arg(expert_ids.reshape(tokens * topk))
    y = torch.empty(tokens * topk, n_out, device=x.device, dtype=x.dtype)
    pw = packed_weight.contiguous()
    alpha = row_alpha.contiguous()
    _lib.call(
        "ma_ternary_expert_swiglu",
        _lib.ptr(x_mat), _lib.dtype_code(x_mat, "x"), x_mat.stride(0) if tokens else k_in,
        tokens, topk, _lib.ptr(pw), n_exp, n_rows, nwords, int(bool(packed_kn)),
        _lib.ptr(alpha), _lib.dtype_code(alpha, "row_alpha"), _lib.ptr(ids), ids64,
        _lib.ptr(y), n_out, _lib.stream_of(x),
    )
    return y.reshape(*id_shape, n_out)


def ternary_expert_down_sum(
    x: torch.Tensor,
    packed_weight: torch.Tensor,
    row_alpha: torch.Tensor,
    expert_ids: torch.Tensor,
    topk_weight: torch.Tensor,
    residual: torch.Tensor | None = None,
    *,
    packed_kn: bool = False,
    round_slots: bool = False,
) -> torch.Tensor:
    """Down-proj GEMV, weighted sum over top-k, optional residual add. One launch.

    ``x`` and ``expert_ids`` / ``topk_weight`` share leading dims ``[..., topk]``.
    Returns ``[..., N]`` (top-k reduced).

    ``round_slots`` (not in the reference's signature): the MoE block's
    composition instead -- each slot's output rounded to ``x.dtype`` before
    the float32 weighted sum, the residual added last, i.e.
    ``moe_reduce_add(ternary_expert_gemv(...), topk_weight, residual)``
    (``model.py:470-473``) in one launch (``ma_ternary_expert_down_combine``).
    """
    if packed_weight.ndim != 3 or packed_weight.dtype != torch.uint32:
        raise ValueError("packed_weight must be uint32 [E, N, K/16] or [E, K/16, N].")
    if not x.is_cuda or not packed_weight.is_cuda or not expert_ids.is_cuda:
        raise RuntimeError("ternary_expert_down_sum requires CUDA tensors.")
    n_exp, n_out, nwords = _expert_nk(packed_weight, packed_kn)
    k_in = nwords * _CODES_PER_WORD
    if x.shape[-1] != k_in:
        raise ValueError(f"x last dim {x.shape[-1]} != packed K ({k_in}).")
    if tuple(row_alpha.shape) != (n_exp, n_out):
        raise ValueError(f"row_alpha shape {tuple(row_alpha.shape)} != {(n_exp, n_out)}.")
    if expert_ids.shape != topk_weight.shape or tuple(x.shape[:-1]) != tuple(expert_ids.shape):
        raise ValueError("x / expert_ids / topk_weight leading dims must match.")
    topk = int(expert_ids.shape[-1])
    tokens = int(expert_ids.numel() // topk)
    x_mat = _rows(x, k_in)
    ids, ids64 = _ids_arg(expert_ids.reshape(tokens * topk))
    wts = topk_weight.reshape(tokens * topk).float().contiguous()
    y = torch.empty(tokens, n_out, device=x.device, dtype=x.dtype)
    res = None
    if residual is not None:
        res = residual.reshape(-1)
        if res.numel() != tokens * n_out:
            raise ValueError(f"residual shape {tuple(residual.shape)} != {tuple(y.shape)}.")
        res = res.contiguous()
    pw = packed_weight.contiguous()
    alpha = row_alpha.contiguous()
    _lib.call(
        "ma_ternary_expert_down_combine" if round_slots else "ma_ternary_expert_down_sum",
        _lib.ptr(x_mat), _lib.dtype_code(x_mat, "x"), x_mat.stride(0) if x_mat.shape[0] else k_in,
        _lib.ptr(pw), n_exp, n_out, nwords, int(bool(packed_kn)),
        _lib.ptr(alpha), _lib.dtype_code(alpha, "row_alpha"), _lib.ptr(ids), ids64,
        _lib.ptr(wts), _lib.ptr(res), _lib.dtype_code(res, "residual") if res is not None else 0,
        tokens, topk, _lib.ptr(y), n_out, _lib.stream_of(x),
    )
    return y.reshape(*tuple(expert_ids.shape[:-1]), n_out)
