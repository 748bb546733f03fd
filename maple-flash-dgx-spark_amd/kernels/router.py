"""Fused MoE router: logits GEMV + softmax + top-k + renormalize.

Drop-in for reference ``src/maple_run/kernels/router.py:141-217`` with one
addition: an optional ``bias`` (float32 ``[E]``) added to the logits before the
softmax, used by the skewed-routing workloads; ``bias=None`` is the reference.
"""

from __future__ import annotations

import torch

from .. import _lib, workspace


def router_wait_timed_out(device: torch.device | int = 0) -> bool:
    """True if a single-launch router call on ``device`` timed out waiting for
    its logits since its workspace was zeroed (the kernel records it instead
    of hanging).  Syncs."""
    return "router" in workspace.timed_out_kinds(device)


def router_topk(
    x: torch.Tensor,
    gate_weight: torch.Tensor,
    top_k: int,
    *,
    bias: torch.Tensor | None = None,
    pairs: bool = False,
):
    """Router logits -> softmax -> top-k -> renormalized weights.

    Returns ``(topk_idx int32 [..., top_k], topk_weight float32 [..., top_k])``
    in descending probability order, ties to the lowest expert index.  With
    ``pairs`` (bf16 ``x``, K a multiple of 16), a third item ``(x_pairs,
    x_corr)``: ``x`` in the form the grouped experts read, written by the same
    launch as the top-k (``moe_grouped(..., x_pairs=...)`` then skips its own
    x' launch; same bits).
    """
    if not x.is_cuda or not gate_weight.is_cuda:
        raise RuntimeError("router_topk requires CUDA tensors.")
    if gate_weight.ndim != 2:
        raise ValueError(f"gate_weight must be 2-D [E, K], got {tuple(gate_weight.shape)}.")
    n_exp, k_in = gate_weight.shape
    if x.shape[-1] != k_in:
        raise ValueError(f"x last dim {x.shape[-1]} != router K ({k_in}).")
    if top_k > n_exp:
        raise ValueError(f"top_k={top_k} exceeds {n_exp} experts.")
    leading = x.shape[:-1]
    tokens = int(x.numel() // k_in)
    x_mat = x.reshape(tokens, k_in)
    if x_mat.stride(-1) != 1:
        x_mat = x_mat.contiguous()
    w = gate_weight.contiguous()
    b = None
    if bias is not None:
        b = bias.reshape(-1).float().contiguous()
        if b.numel() != n_exp:
            raise ValueError(f"bias has {b.numel()} elements, expected {n_exp}.")
    idx = torch.empty(tokens, top_k, device=x.device, dtype=torch.int32)
    wt = torch.empty(tokens, top_k, device=x.device, dtype=torch.float32)
    nbytes = int(_lib.load().ma_router_workspace_bytes(tokens, n_exp))
    # zero-filled once; the single-launch decode router leaves it zero again
    ws = workspace.get("router", x.device, nbytes, min_bytes=1 << 16)
    ldx = x_mat.stride(0) if tokens else k_in
    if pairs:
        xp = torch.empty(tokens, k_in // 2, device=x.device, dtype=torch.uint32)
        xc = torch.empty(tokens, device=x.device, dtype=torch.float32)
        _lib.call(
            "ma_router_topk_pairs",
            _lib.ptr(x_mat), _lib.dtype_code(x_mat, "x"), tokens, ldx,
            _lib.ptr(w), _lib.dtype_code(w, "gate_weight"), n_exp, k_in, _lib.ptr(b), int(top_k),
            _lib.ptr(idx), _lib.ptr(wt), _lib.ptr(xp), _lib.ptr(xc), _lib.ptr(ws), ws.numel(),
            _lib.stream_of(x),
        )
        return idx.reshape(*leading, top_k), wt.reshape(*leading, top_k), (xp, xc)
    _lib.call(
        "ma_router_topk",
        _lib.ptr(x_mat), _lib.dtype_code(x_mat, "x"), tokens, ldx,
        _lib.ptr(w), _lib.dtype_code(w, "gate_weight"), n_exp, k_in, _lib.ptr(b), int(top_k),
        _lib.ptr(idx), _lib.ptr(wt), _lib.ptr(ws), ws.numel(), _lib.stream_of(x),
    )
    return idx.reshape(*leading, top_k), wt.reshape(*leading, top_k)
