"""Packed layer objects over the HIP kernels.

The class names, constructor arguments and methods are those of reference
``src/maple_run/linear.py:16-111`` (the drop-in contract: ``model.py`` builds
and calls them).  Each object owns contiguous device copies of its codes and
scales, in the checkpoint's row-major ``[rows, words]`` order that the kernels
read one row slice at a time, and forwards to one kernel call.
``add_adapter_delta`` stands in for the reference's adapter hook
(``src/maple_run/eggroll/perturb.py:277-292``): the decode path here never
attaches an adapter, so it hands ``y`` back unless a layer carries one.
"""

from __future__ import annotations

import torch

from .kernels.rtn4 import HEAD_GROUP_SIZE, rtn4_embedding, rtn4_gemv
from .kernels.ternary_expert import (
    ternary_expert_down_sum,
    ternary_expert_gemv,
    ternary_expert_swiglu,
)
from .kernels.ternary_gemv import ternary_gemv


def add_adapter_delta(layer, y, x, **_kwargs):
    """``y`` plus the layer's adapter term, when one is attached as ``layer._adapter``."""
    adapter = getattr(layer, "_adapter", None)
    return y if adapter is None else adapter(y, x, **_kwargs)


def _codes(t: torch.Tensor) -> torch.Tensor:
    if t.dtype != torch.uint32:
        raise TypeError(f"packed codes must be torch.uint32, got {t.dtype}.")
    return t.contiguous()


class PackedTernaryLinear:
    """A ternary projection: 2-bit codes ``[rows, K/16]`` and one scale per row;
    ``forward(x, rms_weight=None)`` optionally folds the input RMSNorm."""

    def __init__(self, packed_weight, row_alpha):
        self.packed_weight = _codes(packed_weight)
        self.row_alpha = row_alpha.contiguous()

    def forward(self, x, rms_weight=None, rms_eps: float = 1e-6):
        y = ternary_gemv(x, self.packed_weight, self.row_alpha, rms_weight=rms_weight, rms_eps=rms_eps)
        return add_adapter_delta(self, y, x, rms_weight=rms_weight, rms_eps=rms_eps)

    __call__ = forward


class PackedTernaryExperts:
    """All experts of one projection stacked as ``[experts, rows, K/16]``; the
    kernels pick each slot's expert on the device from ``expert_ids``."""

    def __init__(self, packed_weight, row_alpha):
        self.packed_weight = _codes(packed_weight)
        self.row_alpha = row_alpha.contiguous()

    def forward(self, x, expert_ids):
        y = ternary_expert_gemv(x, self.packed_weight, self.row_alpha, expert_ids)
        return add_adapter_delta(self, y, x, expert_ids=expert_ids)

    def swiglu(self, x, expert_ids):
        """Up and gate rows of each selected expert, then SwiGLU."""
        y = ternary_expert_swiglu(x, self.packed_weight, self.row_alpha, expert_ids)
        return add_adapter_delta(self, y, x, expert_ids=expert_ids)

    def down_sum(self, x, expert_ids, topk_weight, residual=None):
        """Down projection of every slot, combined with the routing weights."""
        return ternary_expert_down_sum(x, self.packed_weight, self.row_alpha, expert_ids, topk_weight,
                                       residual=residual)

    __call__ = forward


class PackedRTN4Linear:
    """The 4-bit affine head: codes ``[vocab, K/8]`` with a scale and a bias per
    group of ``group_size`` inputs."""

    def __init__(self, packed_weight, scales, biases, group_size: int = HEAD_GROUP_SIZE):
        self.packed_weight = _codes(packed_weight)
        self.scales = scales.contiguous()
        self.biases = biases.contiguous()
        self.group_size = int(group_size)

    def forward(self, x):
        y = rtn4_gemv(x, self.packed_weight, self.scales, self.biases, group_size=self.group_size)
        return add_adapter_delta(self, y, x)

    __call__ = forward


class PackedRTN4Embedding:
    """Token embedding from the same 4-bit format: ``forward(ids)`` returns the
    dequantised float32 rows of those ids only."""

    def __init__(self, packed_weight, scales, biases, group_size: int = HEAD_GROUP_SIZE):
        self.packed_weight = _codes(packed_weight)
        self.scales = scales.contiguous()
        self.biases = biases.contiguous()
        self.group_size = int(group_size)
        rows, words = self.packed_weight.shape
        if self.scales.shape != (rows, words * 8 // self.group_size):
            raise ValueError(f"embedding scales {tuple(self.scales.shape)} do not match "
                             f"{rows} rows in groups of {self.group_size}.")

    def forward(self, input_ids):
        return rtn4_embedding(input_ids, self.packed_weight, self.scales, self.biases,
                              group_size=self.group_size)

    __call__ = forward
