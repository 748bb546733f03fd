"""4-bit RTN embedding lookup and GEMV (lm_head / embeddings).

Drop-ins for reference ``src/maple_run/kernels/rtn4.py``: ``rtn4_embedding``
(:27-47), ``rtn4_gemv`` (:285-415) and ``rtn4_indexed_gemv`` (:418-611, the
FlashHead probe GEMV).  Dequant is ``code * scale + bias`` per
group, 8 LSB-first codes per uint32.  Unlike the reference, every batch size
works with group 64 and 128 (the reference rejects group 128 above batch 16,
``rtn4.py:79-81,349-353``).
"""

from __future__ import annotations

import torch

from .. import _lib, workspace

_CODES_PER_WORD = 8
HEAD_GROUP_SIZE = 64


def rtn4_embedding(
    input_ids: torch.Tensor,
    packed_weight: torch.Tensor,
    scales: torch.Tensor,
    biases: torch.Tensor,
    group_size: int = HEAD_GROUP_SIZE,
) -> torch.Tensor:
    """Gather packed rows for ``input_ids`` and dequant those rows only (float32)."""
    if packed_weight.dtype != torch.uint32:
        raise TypeError(f"packed_weight must be uint32 codes, got {packed_weight.dtype}.")
    if not input_ids.is_cuda or not packed_weight.is_cuda:
        raise RuntimeError("rtn4_embedding requires CUDA tensors.")
    vocab, nwords = packed_weight.shape
    k = nwords * _CODES_PER_WORD
    ids = input_ids.reshape(-1)
    if ids.dtype not in (torch.int32, torch.int64):
        ids = ids.to(torch.int64)
    ids = ids.contiguous()
    out = torch.empty(ids.numel(), k, device=packed_weight.device, dtype=torch.float32)
    sc, bs = scales.contiguous(), biases.contiguous()
    _lib.call(
        "ma_rtn4_embedding",
        _lib.ptr(ids), int(ids.dtype == torch.int64), ids.numel(),
        _lib.ptr(packed_weight.contiguous()), vocab, nwords,
        _lib.ptr(sc), _lib.dtype_code(sc, "scales"), _lib.ptr(bs), _lib.dtype_code(bs, "biases"),
        int(group_size), _lib.ptr(out), _lib.stream_of(packed_weight),
    )
    return out.reshape(*input_ids.shape, k)


def rtn4_gemv(
    x: torch.Tensor,
    packed_weight: torch.Tensor,
    scales: torch.Tensor,
    biases: torch.Tensor,
    group_size: int = HEAD_GROUP_SIZE,
    *,
    packed_kn: bool = False,
) -> torch.Tensor:
    """Decode GEMV ``y = x @ W`` with 4-bit packed ``W`` (affine RTN)."""
    if packed_weight.dtype != torch.uint32:
        raise TypeError(
            f"packed_weight must be uint32 codes, got {packed_weight.dtype}; "
            "refusing to run a dense-weight path."
        )
    if packed_weight.ndim != 2:
        raise ValueError(
            f"packed_weight must be 2-D [N, K/8] or [K/8, N]; got shape "
            f"{tuple(packed_weight.shape)}."
        )
    if not x.is_cuda or not packed_weight.is_cuda:
        raise RuntimeError("rtn4_gemv requires CUDA tensors.")
    if packed_kn:
        nwords, n_out = packed_weight.shape
        n_groups = nwords * _CODES_PER_WORD // group_size
        if tuple(scales.shape) != (n_groups, n_out) or tuple(biases.shape) != (n_groups, n_out):
            raise ValueError(
                f"packed_kn scales/biases expected {(n_groups, n_out)}, "
                f"got {tuple(scales.shape)} and {tuple(biases.shape)}."
            )
    else:
        n_out, nwords = packed_weight.shape
        n_groups = nwords * _CODES_PER_WORD // group_size
        if tuple(scales.shape) != (n_out, n_groups) or tuple(biases.shape) != (n_out, n_groups):
            raise ValueError(
                f"scales/biases expected {(n_out, n_groups)}, got {tuple(scales.shape)} "
                f"and {tuple(biases.shape)}."
            )
    k_in = nwords * _CODES_PER_WORD
    if x.shape[-1] != k_in:
        raise ValueError(f"x last dim {x.shape[-1]} != packed K ({k_in}).")
    if k_in % group_size:
        raise ValueError(f"K={k_in} is not a whole number of RTN groups (group_size={group_size}).")
    leading = x.shape[:-1]
    batch = int(x.numel() // k_in)
    x_mat = x.reshape(batch, k_in)
    if x_mat.stride(-1) != 1:
        x_mat = x_mat.contiguous()
    y = torch.empty(batch, n_out, device=x.device, dtype=x.dtype)
    pw, sc, bs = packed_weight.contiguous(), scales.contiguous(), biases.contiguous()
    args = (
        _lib.ptr(x_mat), _lib.dtype_code(x_mat, "x"), batch, x_mat.stride(0) if batch else k_in,
        _lib.ptr(pw), n_out, nwords, int(bool(packed_kn)),
        _lib.ptr(sc), _lib.dtype_code(sc, "scales"), _lib.ptr(bs), _lib.dtype_code(bs, "biases"),
        int(group_size), _lib.ptr(y), n_out,
    )
    # Batched calls in groups of 128 build their x' operands once into a
    # per-stream workspace (ma_rtn4_gemv_ws); others need none.
    nbytes = 0 if packed_kn else int(_lib.load().ma_rtn4_gemv_workspace_bytes(batch, nwords, int(group_size)))
    if nbytes:
        ws = workspace.get("rtn4", x.device, nbytes, (nwords, int(group_size)))
        _lib.call("ma_rtn4_gemv_ws", *args, _lib.ptr(ws), ws.numel(), _lib.stream_of(x))
    else:
        _lib.call("ma_rtn4_gemv", *args, _lib.stream_of(x))
    return y.reshape(*leading, n_out)


def rtn4_indexed_gemv(
    x: torch.Tensor,
    packed_weight: torch.Tensor,
    scales: torch.Tensor,
    biases: torch.Tensor,
    cluster_ids: torch.Tensor,
    group_size: int = HEAD_GROUP_SIZE,
) -> torch.Tensor:
    """GEMV over the rows of the probed clusters: ``packed_weight`` is
    ``[n_clusters, cluster_size, nwords]`` (the head's rows grouped by
    cluster), ``cluster_ids`` ``[n_probes]``; the output ``[..., n_probes *
    cluster_size]`` is cluster-major, so entry ``p * cluster_size + m`` is
    row ``m`` of cluster ``cluster_ids[p]`` -- the same values ``rtn4_gemv``
    gives for those rows."""
    if packed_weight.dtype != torch.uint32:
        raise TypeError(f"packed_weight must be uint32 codes, got {packed_weight.dtype}; "
                        "refusing to run a dense-weight path.")
    if packed_weight.ndim != 3:
        raise ValueError("packed_weight must be 3-D [n_clusters, cluster_size, nwords]; got shape "
                         f"{tuple(packed_weight.shape)}.")
    if not x.is_cuda or not packed_weight.is_cuda:
        raise RuntimeError("rtn4_indexed_gemv requires CUDA tensors.")
    if cluster_ids.ndim != 1:
        raise ValueError(f"cluster_ids must be 1-D [n_probes]; got shape {tuple(cluster_ids.shape)}.")
    n_clusters, cluster_size, nwords = packed_weight.shape
    n_groups = nwords * _CODES_PER_WORD // group_size
    expect = (n_clusters, cluster_size, n_groups)
    if tuple(scales.shape) != expect or tuple(biases.shape) != expect:
        raise ValueError(f"scales/biases expected {expect}, got {tuple(scales.shape)} and {tuple(biases.shape)}.")
    k_in = nwords * _CODES_PER_WORD
    if x.shape[-1] != k_in:
        raise ValueError(f"x last dim {x.shape[-1]} != packed K ({k_in}).")
    leading = x.shape[:-1]
    batch = int(x.numel() // k_in)
    x_mat = x.reshape(batch, k_in).contiguous()
    n_probes = int(cluster_ids.numel())
    ids = cluster_ids.to(torch.int32).contiguous()
    y = torch.empty(batch, n_probes * cluster_size, device=x.device, dtype=x.dtype)
    sc, bs = scales.contiguous(), biases.contiguous()
    _lib.call("ma_rtn4_indexed_gemv", _lib.ptr(x_mat), _lib.dtype_code(x_mat, "x"), batch, k_in,
              _lib.ptr(packed_weight.contiguous()), n_clusters, cluster_size, nwords,
              _lib.ptr(sc), _lib.dtype_code(sc, "scales"), _lib.ptr(bs), _lib.dtype_code(bs, "biases"),
              int(group_size), _lib.ptr(ids), n_probes, _lib.ptr(y), n_probes * cluster_size,
              _lib.stream_of(x))
    return y.reshape(*leading, n_probes * cluster_size)
