"""Decode-step attention: QK RMSNorm + partial RoPE + KV write, then GQA.

Mirrors reference ``src/maple_run/kernels/decode_attn.py``: ``apply_qkv_decode``
(:362-439) and ``decode_gqa_attn`` (:470-592).  Differences at the boundary:
``apply_qkv_decode`` takes the float32 RoPE tables and gathers the row for
``seqlen[b]`` itself (the reference takes the gathered bf16 cos/sin), and the
GQA workspace is allocated here per call.  head_dim must be 64.
"""

from __future__ import annotations

import torch

from .. import _lib


def apply_qkv_decode(
    qkv: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    cos_table: torch.Tensor,
    sin_table: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    seqlen: torch.Tensor,
    *,
    num_heads: int,
    num_kv_heads: int,
    head_dim: int,
    rotary_dim: int,
    use_rope: bool = True,
    eps: float = 1e-6,
) -> torch.Tensor:
    """QK RMSNorm + RoPE + store K/V at ``seqlen``; returns q ``[B, H, 1, D]``."""
    if qkv.ndim != 2:
        raise ValueError(f"apply_qkv_decode expects [B, qkv], got {tuple(qkv.shape)}.")
    if qkv.dtype != torch.bfloat16 or k_cache.dtype != torch.bfloat16:
        raise TypeError("apply_qkv_decode runs on bf16 activations and caches.")
    bsz = qkv.shape[0]
    if k_cache.shape[0] != bsz or v_cache.shape[0] != bsz:
        raise ValueError(f"KV cache batch {k_cache.shape[0]} != qkv batch {bsz}.")
    if seqlen.numel() != bsz:
        raise ValueError(f"seqlen has {seqlen.numel()} entries, expected {bsz}.")
    if qkv.stride(1) != 1:
        raise ValueError("apply_qkv_decode needs a row-contiguous qkv.")
    q_out = torch.empty(bsz, num_heads, 1, head_dim, device=qkv.device, dtype=qkv.dtype)
    sl = seqlen.reshape(-1).to(torch.int64).contiguous()
    _lib.call(
        "ma_qk_norm_rope_store",
        _lib.ptr(qkv), qkv.stride(0), bsz, num_heads, num_kv_heads, head_dim,
        _lib.ptr(q_weight.float().contiguous()), _lib.ptr(k_weight.float().contiguous()),
        _lib.ptr(cos_table), _lib.ptr(sin_table), int(cos_table.shape[0]), int(rotary_dim),
        int(bool(use_rope)), float(eps), _lib.ptr(sl), _lib.ptr(k_cache), _lib.ptr(v_cache),
        int(k_cache.shape[2]), _lib.ptr(q_out), _lib.stream_of(qkv),
    )
    return q_out


def decode_gqa_attn(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    seqlen: torch.Tensor,
    *,
    scale: float,
    window: int | None = None,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """q ``[B, H, 1, D]`` against the first ``seqlen[b] + 1`` cached positions."""
    bsz, n_heads, _, head_dim = q.shape
    n_kv, max_len = int(k_cache.shape[1]), int(k_cache.shape[2])
    out = torch.empty(bsz, n_heads, 1, head_dim, device=q.device, dtype=q.dtype)
    nbytes = int(_lib.load().ma_gqa_workspace_bytes(bsz, n_kv, max_len))
    if workspace is None or workspace.numel() < nbytes:
        workspace = torch.empty(nbytes, device=q.device, dtype=torch.uint8)
    sl = seqlen.reshape(-1).to(torch.int64).contiguous()
    _lib.call(
        "ma_decode_gqa_attn",
        _lib.ptr(q.contiguous()), bsz, n_heads, n_kv, head_dim, _lib.ptr(k_cache),
        _lib.ptr(v_cache), _lib.ptr(sl), max_len, int(window or 0), float(scale),
        _lib.ptr(out), _lib.ptr(workspace), workspace.numel(), _lib.stream_of(q),
    )
    return out
