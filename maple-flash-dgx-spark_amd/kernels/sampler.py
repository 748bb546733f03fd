"""Fused top-k / temperature / nucleus sampling on the device.

Mirrors reference ``src/maple_run/kernels/sampler.py``: ``fused_sample``
(:106-145), ``fused_sample_batched`` (:148-199), ``sampler_workspace`` /
``batched_sampler_workspace`` (:202-232), ``MAX_TOP_K``; same arguments,
checks and exceptions.  Two HIP launches (``ma_fused_sample``): per-chunk
top-k candidates, then the merge, the temperature softmax over the top-k, the
nucleus cut and the inverse CDF at the caller's uniform.  Randomness stays
with the caller: one uniform in [0, 1) per row, so a seeded run and a graph
replay draw the same ids.

The workspace is one byte tensor (the reference passes a tuple of candidate
values, indices and the output); ``out`` is separate.
"""

from __future__ import annotations

import torch

from .. import _lib

MAX_TOP_K = 64


def _check(top_k: int, temperature: float, vocab: int) -> None:
    if not 0 < top_k <= MAX_TOP_K:
        raise ValueError(f"fused_sample needs 0 < top_k <= {MAX_TOP_K}, got {top_k}.")
    if top_k > vocab:
        raise ValueError(f"top_k {top_k} exceeds the vocabulary ({vocab}).")
    if temperature <= 0:
        raise ValueError("fused_sample needs temperature > 0 (greedy is argmax).")


def _workspace_bytes(rows: int, vocab: int, top_k: int) -> int:
    return int(_lib.load().ma_sampler_workspace_bytes(rows, vocab, top_k))


def sampler_workspace(vocab: int, top_k: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """``(workspace, out)`` for ``fused_sample`` so decode allocates nothing per token."""
    ws = torch.empty(_workspace_bytes(1, vocab, top_k), device=device, dtype=torch.uint8)
    return ws, torch.empty((), device=device, dtype=torch.int64)


def batched_sampler_workspace(vocab: int, top_k: int, batch: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """``fused_sample_batched`` scratch for up to ``batch`` rows (narrower calls
    use the front of it)."""
    ws = torch.empty(_workspace_bytes(batch, vocab, top_k), device=device, dtype=torch.uint8)
    return ws, torch.empty(batch, device=device, dtype=torch.int64)


def _launch(x: torch.Tensor, uniform: torch.Tensor, temperature: float, top_p: float, top_k: int,
            ws: torch.Tensor, out: torch.Tensor) -> None:
    rows, vocab = x.shape
    if x.stride(1) != 1:
        raise ValueError("logits rows must be contiguous.")
    if uniform.dtype != torch.float32 or not uniform.is_cuda:
        raise TypeError("uniform must be a float32 CUDA tensor.")
    if out.dtype != torch.int64 or not out.is_contiguous() or out.numel() < rows:
        raise ValueError("out must be a contiguous int64 tensor with one entry per row.")
    if ws.dtype != torch.uint8 or not ws.is_contiguous():
        raise TypeError("the sampler workspace must be a contiguous uint8 tensor.")
    _lib.call("ma_fused_sample", _lib.ptr(x), _lib.dtype_code(x, "logits"), rows, vocab, x.stride(0),
              _lib.ptr(uniform), int(top_k), float(1.0 / float(temperature)), float(top_p),
              _lib.ptr(ws), ws.numel(), _lib.ptr(out), _lib.stream_of(x))


def fused_sample(logits: torch.Tensor, uniform: torch.Tensor, *, temperature: float, top_p: float,
                 top_k: int, workspace: tuple[torch.Tensor, torch.Tensor] | None = None) -> torch.Tensor:
    """Sample one token id from 1-D ``logits``; ``uniform`` is a scalar in [0, 1).

    Top-k on the logits, temperature softmax over those, nucleus ``top_p``,
    then the draw.  Returns a 0-D int64 CUDA tensor."""
    if logits.ndim != 1:
        raise ValueError(f"fused_sample expects 1-D logits, got {tuple(logits.shape)}.")
    _check(top_k, temperature, int(logits.shape[0]))
    if not logits.is_cuda:
        raise RuntimeError("fused_sample requires CUDA tensors.")
    x = logits.reshape(1, -1)
    if workspace is None:
        workspace = sampler_workspace(int(x.shape[1]), top_k, logits.device)
    ws, out = workspace
    _launch(x, uniform.reshape(1), temperature, top_p, top_k, ws, out.reshape(-1))
    return out


def fused_sample_batched(logits: torch.Tensor, uniform: torch.Tensor, *, temperature: float,
                         top_p: float, top_k: int,
                         workspace: tuple[torch.Tensor, torch.Tensor] | None = None) -> torch.Tensor:
    """One id per row of ``logits [B, vocab]``; ``uniform`` is ``[B]``.  Row
    ``b`` draws exactly what it draws alone with the same uniform.  Returns
    int64 ``[B]``."""
    if logits.ndim != 2:
        raise ValueError(f"fused_sample_batched expects [B, vocab], got {tuple(logits.shape)}.")
    bsz, vocab = logits.shape
    _check(top_k, temperature, int(vocab))
    if uniform.numel() != bsz:
        raise ValueError(f"uniform has {uniform.numel()} draws, expected {bsz}.")
    if not logits.is_cuda:
        raise RuntimeError("fused_sample_batched requires CUDA tensors.")
    if workspace is None:
        workspace = batched_sampler_workspace(int(vocab), top_k, int(bsz), logits.device)
    ws, out = workspace
    _launch(logits, uniform.reshape(-1), temperature, top_p, top_k, ws, out.reshape(-1))
    return out[:bsz]
