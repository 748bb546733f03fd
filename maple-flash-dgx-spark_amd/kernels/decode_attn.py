"""Decode-step attention: QK RMSNorm + partial RoPE + KV write, then GQA.

Mirrors reference ``src/maple_run/kernels/decode_attn.py``:
``apply_qkv_decode`` (:362-439) and ``decode_gqa_attn`` (:470-592), same
arguments and checks.  Differences at the boundary:

* ``decode_gqa_attn``'s ``workspace`` is one zero-initialised byte tensor from
  ``gqa_workspace`` (the reference passes a tuple of three float tensors); the
  splits are merged inside the same launch.
* ``decode_attention`` has no single reference counterpart: it is the decode
  branch of ``MapleAttention`` (``model.py:368-414``: RoPE gather,
  ``apply_qkv_decode``, ``decode_gqa_attn``) in one launch, reading the
  float32 RoPE tables at ``seqlen[b]`` itself.

head_dim must be 64 or 128 and at most 16 query heads may share a KV head.
"""

from __future__ import annotations

import torch

from .. import _lib, workspace


def _check_rows(what, bsz, k_cache, v_cache, seqlen, row_map):
    if row_map is None and (k_cache.shape[0] != bsz or v_cache.shape[0] != bsz):
        raise ValueError(f"KV cache batch {k_cache.shape[0]} != {what} batch {bsz}.")
    if seqlen.numel() != bsz:
        raise ValueError(f"seqlen has {seqlen.numel()} entries, expected {bsz}.")
    if row_map is not None and row_map.numel() != bsz:
        raise ValueError(f"row_map has {row_map.numel()} entries, expected {bsz}.")
    if k_cache.dtype != torch.bfloat16 or v_cache.dtype != torch.bfloat16:
        raise TypeError("the KV cache must be bf16.")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("the KV cache must be contiguous [rows, n_kv, max_len, head_dim].")


def _i64(t: torch.Tensor | None) -> torch.Tensor | None:
    return None if t is None else t.reshape(-1).to(torch.int64).contiguous()


def _norm_weights(q_weight, k_weight):
    if q_weight.dtype != k_weight.dtype:
        raise TypeError("q_norm and k_norm weights must share a dtype.")
    return q_weight.reshape(-1).contiguous(), k_weight.reshape(-1).contiguous()


def o_projection_supported(batch: int, num_heads: int, num_kv_heads: int, head_dim: int,
                           max_len: int, window: int | None, o_rows: int) -> bool:
    """True if ``decode_attention(..., o_linear=...)`` can compute an output
    projection of ``o_rows`` rows in its launch for these sizes."""
    return bool(_lib.load().ma_decode_attn_o_supported(batch, num_heads, num_kv_heads, head_dim,
                                                         max_len, int(window or 0), o_rows))


def attention_form(batch: int, num_kv_heads: int, head_dim: int, max_len: int, window: int | None = None,
                   fused: bool = True, with_o: bool = False) -> str:
    """``"xcd"`` if the attention launch for these sizes keeps every split of
    a (row, KV head) on one XCD (merged through that XCD's L2), ``"grid"``
    for the cross-XCD form; both give the same bits."""
    f = _lib.load().ma_decode_attn_form(batch, num_kv_heads, head_dim, max_len, int(window or 0),
                                        int(fused), int(with_o))
    if f < 0:
        raise ValueError("attention_form: bad sizes")
    return "xcd" if f == 1 else "grid"


def gqa_workspace(batch: int, num_kv_heads: int, max_len: int, device, head_dim: int = 64) -> torch.Tensor:
    """Zeroed workspace for ``decode_gqa_attn`` / ``decode_attention``; keep
    one per cache so decode allocates nothing inside a graph."""
    nbytes = int(_lib.load().ma_gqa_workspace_bytes(batch, num_kv_heads, max_len, head_dim))
    if nbytes == 0:
        raise ValueError(f"head_dim {head_dim} unsupported (64 or 128).")
    return workspace.register_attention(torch.zeros(nbytes, device=device, dtype=torch.uint8))


def apply_qkv_decode(
    qkv: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    seqlen: torch.Tensor,
    *,
    row_map: torch.Tensor | None = None,
    num_heads: int,
    num_kv_heads: int,
    head_dim: int,
    rotary_dim: int,
    use_rope: bool,
    use_qk_norm: bool,
    eps: float,
) -> torch.Tensor:
    """QK RMSNorm + optional RoPE + store K/V at ``seqlen``. Returns Q ``[B, H, 1, D]``.

    ``cos``/``sin`` hold one row per batch row (``[B, rotary_dim]`` or
    ``[B, 1, rotary_dim]``, as gathered by the rotary embedding).
    """
    if qkv.ndim != 2:
        raise ValueError(f"apply_qkv_decode expects [B, qkv], got {tuple(qkv.shape)}.")
    if not use_qk_norm:
        raise ValueError("apply_qkv_decode requires QK RMSNorm.")
    if qkv.dtype != torch.bfloat16:
        raise TypeError("apply_qkv_decode runs on bf16 activations.")
    bsz = qkv.shape[0]
    _check_rows("qkv", bsz, k_cache, v_cache, seqlen, row_map)
    if qkv.stride(1) != 1:
        raise ValueError("apply_qkv_decode needs a row-contiguous qkv.")
    q_out = torch.empty(bsz, num_heads, 1, head_dim, device=qkv.device, dtype=qkv.dtype)
    cos2 = cos.reshape(bsz, -1).contiguous()
    sin2 = sin.reshape(bsz, -1).to(cos2.dtype).contiguous()
    qw, kw = _norm_weights(q_weight, k_weight)
    sl, rm = _i64(seqlen), _i64(row_map)
    _lib.call(
        "ma_qk_norm_rope_store",
        _lib.ptr(qkv), qkv.stride(0), bsz, num_heads, num_kv_heads, head_dim,
        _lib.ptr(qw), _lib.ptr(kw), _lib.dtype_code(qw, "q_weight"), _lib.ptr(cos2), _lib.ptr(sin2),
        _lib.dtype_code(cos2, "cos"), cos2.shape[1], 0, int(rotary_dim), int(bool(use_rope)), float(eps),
        _lib.ptr(sl), _lib.ptr(rm), _lib.ptr(k_cache),
        _lib.ptr(v_cache), int(k_cache.shape[0]), int(k_cache.shape[2]), _lib.ptr(q_out),
        _lib.stream_of(qkv),
    )
    return q_out


def decode_gqa_attn(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    seqlen: torch.Tensor,
    *,
    row_map: torch.Tensor | None = None,
    scale: float,
    window: int | None,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """GQA attention for ``q_len=1``. ``seqlen[b]`` is the index just written (kv_len-1)."""
    if q.ndim != 4 or q.shape[2] != 1:
        raise ValueError(f"decode_gqa_attn expects q [B, H, 1, D], got {tuple(q.shape)}.")
    bsz, n_q, _, head_dim = q.shape
    _check_rows("q", bsz, k_cache, v_cache, seqlen, row_map)
    n_kv, max_len = int(k_cache.shape[1]), int(k_cache.shape[2])
    if n_q % n_kv != 0:
        raise ValueError(f"n_q={n_q} not divisible by n_kv={n_kv}.")
    out = torch.empty_like(q)
    nbytes = int(_lib.load().ma_gqa_workspace_bytes(bsz, n_kv, max_len, head_dim))
    if workspace is None:
        workspace = gqa_workspace(bsz, n_kv, max_len, q.device, head_dim)
    elif workspace.numel() < nbytes:
        raise ValueError(f"workspace holds {workspace.numel()} bytes, needs {nbytes}.")
    sl, rm = _i64(seqlen), _i64(row_map)
    _lib.call(
        "ma_decode_gqa_attn",
        _lib.ptr(q.contiguous()), bsz, n_q, n_kv, head_dim, _lib.ptr(k_cache), _lib.ptr(v_cache),
        int(k_cache.shape[0]), max_len, _lib.ptr(sl), _lib.ptr(rm),
        int(window or 0), float(scale), _lib.ptr(out), _lib.ptr(workspace), workspace.numel(),
        _lib.stream_of(q),
    )
    return out


def decode_attention(
    qkv: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    cos_table: torch.Tensor,
    sin_table: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    seqlen: torch.Tensor,
    workspace: torch.Tensor,
    *,
    row_map: torch.Tensor | None = None,
    num_heads: int,
    num_kv_heads: int,
    head_dim: int,
    rotary_dim: int,
    use_rope: bool = True,
    eps: float = 1e-6,
    scale: float,
    window: int | None = None,
    o_linear: tuple | None = None,
):
    """``apply_qkv_decode`` + ``decode_gqa_attn`` in one launch, with the RoPE
    rows read from the float32 tables ``[n_pos, rotary_dim]`` at ``seqlen[b]``.
    Returns the attention output ``[B, H, 1, D]`` bf16.

    ``o_linear = (packed [N, H*D/16] uint32, alpha [N])`` (batch 1, H*D = 2048):
    the same launch also computes the output projection
    ``ternary_gemv(out.reshape(1, -1), packed, alpha)`` (the same bits) and the
    call returns ``(out, o [1, N])``."""
    if qkv.ndim != 2 or qkv.stride(1) != 1 or qkv.dtype != torch.bfloat16:
        raise ValueError("decode_attention expects a row-contiguous bf16 qkv [B, qkv].")
    bsz = qkv.shape[0]
    _check_rows("qkv", bsz, k_cache, v_cache, seqlen, row_map)
    n_kv, max_len = int(k_cache.shape[1]), int(k_cache.shape[2])
    if sin_table.dtype != cos_table.dtype or sin_table.stride(0) != cos_table.stride(0):
        raise ValueError("cos and sin tables must share dtype and layout.")
    out = torch.empty(bsz, num_heads, 1, head_dim, device=qkv.device, dtype=qkv.dtype)
    qw, kw = _norm_weights(q_weight, k_weight)
    sl, rm = _i64(seqlen), _i64(row_map)
    o_w = o_a = o = None
    o_rows = 0
    if o_linear is not None:
        o_w, o_a = o_linear
        if o_w.dtype != torch.uint32:
            raise TypeError("o_linear packed weight must be torch.uint32")
        if o_w.ndim != 2 or o_w.shape[1] * 16 != num_heads * head_dim:
            raise ValueError("o_linear packed weight must be [N, num_heads * head_dim / 16]")
        o_rows = int(o_w.shape[0])
        o_a = o_a.contiguous()
        o = torch.empty(bsz, o_rows, device=qkv.device, dtype=qkv.dtype)
    _lib.call(
        "ma_decode_attn_fused",
        _lib.ptr(qkv), qkv.stride(0), bsz, num_heads, num_kv_heads, head_dim,
        _lib.ptr(qw), _lib.ptr(kw), _lib.dtype_code(qw, "q_weight"), _lib.ptr(cos_table), _lib.ptr(sin_table),
        _lib.dtype_code(cos_table, "cos_table"), cos_table.stride(0), int(cos_table.shape[0]), int(rotary_dim),
        int(bool(use_rope)), float(eps), _lib.ptr(sl), _lib.ptr(rm),
        _lib.ptr(k_cache), _lib.ptr(v_cache), int(k_cache.shape[0]), max_len, int(window or 0),
        float(scale), _lib.ptr(out), _lib.ptr(workspace), workspace.numel(),
        _lib.ptr(o_w), _lib.ptr(o_a), _lib.dtype_code(o_a, "row_alpha") if o_a is not None else 0,
        o_rows, _lib.ptr(o), _lib.stream_of(qkv),
    )
    if o_linear is not None:
        return out, o
    return out
