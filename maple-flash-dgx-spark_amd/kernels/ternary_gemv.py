"""Packed ternary GEMV ``y = x @ W`` with ``W`` kept as packed uint32 codes.

Drop-in for reference ``src/maple_run/kernels/ternary_gemv.py:261-388``: same
signature, argument meaning, output shape/dtype and exceptions.  The work is
``ma_ternary_gemv`` (one launch) or, for the RMS-folded form at 17 tokens and
more, ``ma_ternary_gemv_ws`` (operand build + GEMM), HIP on gfx950, on the
current stream.
"""

from __future__ import annotations

import torch

from .. import _lib

_CODES_PER_WORD = 16


def ternary_gemv(
    x: torch.Tensor,
    packed_weight: torch.Tensor,
    row_alpha: torch.Tensor,
    *,
    rms_weight: torch.Tensor | None = None,
    rms_eps: float = 1e-6,
    packed_kn: bool = False,
) -> torch.Tensor:
    """Decode GEMV ``y = x @ W`` with ``W`` kept as packed uint32 codes.

    Parameters
    ----------
    x:
        Activations ``[K]`` or ``[B, K]`` (any leading dims are flattened).
    packed_weight:
        ``uint32`` codes ``[N, K/16]`` (``packed_kn=False``) or ``[K/16, N]``.
    row_alpha:
        Per-output-row scale ``[N]``.
    rms_weight:
        If set, RMSNorm ``x`` in-kernel (fused input RMSNorm + GEMV).
    packed_kn:
        If True, packed codes are stored ``[nwords, N]``.
    """
    if not x.is_cuda or not packed_weight.is_cuda or not row_alpha.is_cuda:
        raise RuntimeError("ternary_gemv requires CUDA tensors (packed weights stay on GPU).")
    if packed_weight.dtype != torch.uint32:
        raise TypeError(
            f"packed_weight must be uint32 codes, got {packed_weight.dtype}; "
            "refusing to run a dense-weight path."
        )
    if packed_weight.ndim != 2:
        raise ValueError(
            f"packed_weight must be 2-D [N, K/16] or [K/16, N]; got shape "
            f"{tuple(packed_weight.shape)}. Stacked experts are a later fused kernel."
        )
    if packed_kn:
        nwords, n_out = packed_weight.shape
    else:
        n_out, nwords = packed_weight.shape
    k_in = nwords * _CODES_PER_WORD
    alpha = row_alpha.reshape(-1)
    if alpha.numel() != n_out:
        raise ValueError(
            f"row_alpha has {alpha.numel()} elements, expected one per output row ({n_out})."
        )
    if x.shape[-1] != k_in:
        raise ValueError(f"x last dim {x.shape[-1]} != packed K ({k_in}).")

    leading = x.shape[:-1]
    batch = int(x.numel() // k_in) if k_in else 0
    x_mat = x.reshape(batch, k_in)
    if x_mat.stride(-1) != 1:
        x_mat = x_mat.contiguous()
    y = torch.empty(batch, n_out, device=x.device, dtype=x.dtype)
    rms_w = None
    if rms_weight is not None:
        rms_w = rms_weight.reshape(-1)
        if rms_w.numel() != k_in:
            raise ValueError(f"rms_weight has {rms_w.numel()} elements, expected {k_in}.")
        rms_w = rms_w.contiguous()
    pw = packed_weight.contiguous()
    alpha = alpha.contiguous()
    args = (
        _lib.ptr(x_mat), _lib.dtype_code(x_mat, "x"), batch, x_mat.stride(0) if batch else k_in,
        _lib.ptr(pw), n_out, nwords, int(bool(packed_kn)),
        _lib.ptr(alpha), _lib.dtype_code(alpha, "row_alpha"),
        _lib.ptr(rms_w), _lib.dtype_code(rms_w, "rms_weight") if rms_w is not None else 0,
        float(rms_eps),
        _lib.ptr(y), n_out,
    )
    # With the RMSNorm folded in, from 17 tokens the MFMA GEMM's two-launch form
    # builds each token's operands once into a workspace (the query says 0 where
    # no workspace is used).
    ws_bytes = _lib.load().ma_ternary_gemv_workspace_bytes(batch, nwords, int(rms_w is not None))
    if ws_bytes:
        ws = torch.empty(ws_bytes, device=x.device, dtype=torch.uint8)
        _lib.call("ma_ternary_gemv_ws", *args, _lib.ptr(ws), ws_bytes, _lib.stream_of(x))
    else:
        _lib.call("ma_ternary_gemv", *args, _lib.stream_of(x))
    return y.reshape(*leading, n_out)


def ternary_gemv_combine(pending, packed_weight: torch.Tensor, row_alpha: torch.Tensor, *,
                         rms_weight: torch.Tensor, rms_eps: float = 1e-6):
    """A grouped MoE combine left pending by ``moe_grouped(..., combine=False)``
    run in front of the next RMS-folded GEMM (``ma_ternary_gemv_combine_ws``):
    ``x = sum_j w[t, j] * slot_out[inverse[t, j]] + residual`` (bf16, the
    values ``moe_grouped`` would have returned), ``y = ternary_gemv(x, W,
    alpha, rms_weight)``.  Returns ``(x, y)``.  Needs ``combine_gemv_supported``."""
    n_out, nwords = packed_weight.shape
    tokens, hidden = pending.tokens, pending.hidden
    if hidden != nwords * _CODES_PER_WORD:
        raise ValueError(f"combined rows have {hidden} values, the GEMM takes {nwords * _CODES_PER_WORD}.")
    x = torch.empty(tokens, hidden, device=pending.slot_out.device, dtype=torch.bfloat16)
    y = torch.empty(tokens, n_out, device=x.device, dtype=torch.bfloat16)
    rms_w = rms_weight.reshape(-1).contiguous()
    alpha = row_alpha.reshape(-1).contiguous()
    pw = packed_weight.contiguous()
    ws_bytes = _lib.load().ma_ternary_gemv_workspace_bytes(tokens, nwords, 1)
    ws = torch.empty(max(int(ws_bytes), 1), device=x.device, dtype=torch.uint8)
    _lib.call(
        "ma_ternary_gemv_combine_ws",
        _lib.ptr(pending.slot_out), _lib.ptr(pending.inverse), _lib.ptr(pending.weights),
        pending.top_k, _lib.ptr(pending.residual), _lib.ptr(x), tokens,
        _lib.ptr(pw), n_out, nwords, _lib.ptr(alpha),
        _lib.dtype_code(alpha, "row_alpha"), _lib.ptr(rms_w), _lib.dtype_code(rms_w, "rms_weight"),
        float(rms_eps), _lib.ptr(y), n_out, _lib.ptr(ws), ws.numel(), _lib.stream_of(x),
    )
    return x, y


def combine_gemv_supported(tokens: int, top_k: int, packed_weight: torch.Tensor) -> bool:
    """Where ``ternary_gemv_combine`` runs: 17+ tokens, top-k <= 8, K a
    multiple of 256 (row-major packed codes)."""
    return tokens >= 17 and 1 <= top_k <= 8 and packed_weight.ndim == 2 and packed_weight.shape[1] % 16 == 0
