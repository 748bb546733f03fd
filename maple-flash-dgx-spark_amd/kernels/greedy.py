"""Greedy token choice on the device (reference ``src/maple_run/generate.py:146-148``:
``torch.argmax(logits, dim=-1)``, the lowest index on ties)."""

from __future__ import annotations

import torch

from .. import _lib, workspace


def greedy_argmax(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Row-wise argmax of ``logits [..., V]`` (bf16 or float32) as int64
    ``[...]``; written into ``out`` when given (graph-safe: no allocation
    once the stream's workspace exists).  Each row is read by many
    workgroups (``ma_argmax_rows_ws``; the one-workgroup-per-row
    ``ma_argmax_rows`` gives the same ids)."""
    if not logits.is_cuda:
        raise RuntimeError("greedy_argmax requires CUDA tensors.")
    v = logits.shape[-1]
    x = logits.reshape(-1, v)
    if x.stride(1) != 1:
        x = x.contiguous()
    rows = x.shape[0]
    if out is None:
        out = torch.empty(logits.shape[:-1], device=logits.device, dtype=torch.int64)
    if out.dtype != torch.int64 or out.numel() != rows or not out.is_contiguous():
        raise ValueError("out must be a contiguous int64 tensor with one entry per row.")
    if rows == 0:
        return out
    nbytes = int(_lib.load().ma_argmax_workspace_bytes(rows))
    ws = workspace.get("argmax", logits.device, nbytes, (rows,))
    _lib.call("ma_argmax_rows_ws", _lib.ptr(x), _lib.dtype_code(x, "logits"), rows, v, x.stride(0),
              _lib.ptr(out), _lib.ptr(ws), ws.numel(), _lib.stream_of(logits))
    return out
