"""Token-to-expert dispatch: per-expert lists of (token, slot) pairs.

No reference counterpart (the reference grids over pairs,
``src/maple_run/kernels/ternary_expert.py:210,443``).  Definition: pairs
``p = token * top_k + slot`` stably sorted by expert id.
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from .. import _lib


class Dispatch(NamedTuple):
    counts: torch.Tensor    # int32 [E]
    offsets: torch.Tensor   # int32 [E + 1], exclusive scan of counts
    pair_ids: torch.Tensor  # int32 [T * k], pairs grouped by expert, ascending in token
    inverse: torch.Tensor   # int32 [T * k], position of each pair in pair_ids


def moe_dispatch(expert_ids: torch.Tensor, n_experts: int) -> Dispatch:
    """Build the per-expert pair lists for ``expert_ids`` ``[..., top_k]`` on device."""
    if not expert_ids.is_cuda:
        raise RuntimeError("moe_dispatch requires a CUDA tensor (no GPU→CPU routing).")
    ids = expert_ids.reshape(-1)
    if ids.dtype not in (torch.int32, torch.int64):
        ids = ids.to(torch.int32)
    ids = ids.contiguous()
    n = int(ids.numel())
    dev = expert_ids.device
    counts = torch.empty(n_experts, device=dev, dtype=torch.int32)
    offsets = torch.empty(n_experts + 1, device=dev, dtype=torch.int32)
    pair_ids = torch.empty(n, device=dev, dtype=torch.int32)
    inverse = torch.empty(n, device=dev, dtype=torch.int32)
    _lib.call(
        "ma_moe_dispatch",
        _lib.ptr(ids), int(ids.dtype == torch.int64), n, int(n_experts),
        _lib.ptr(counts), _lib.ptr(offsets), _lib.ptr(pair_ids), _lib.ptr(inverse),
        _lib.stream_of(ids),
    )
    return Dispatch(counts, offsets, pair_ids, inverse)
