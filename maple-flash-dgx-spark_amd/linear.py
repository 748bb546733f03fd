"""Packed linear layers that hold codes + scales and call the HIP kernels.

Mirror of reference ``src/maple_run/linear.py:16-111``.  Codes stay in the
checkpoint's ``[N, nwords]`` order; weights are made contiguous once here.
``add_adapter_delta`` is the reference's adapter hook
(``src/maple_run/eggroll/perturb.py:277-292``); with no adapter attached it
returns ``y`` untouched, which is the only case on this path.
"""

from __future__ import annotations

from .kernels.rtn4 import HEAD_GROUP_SIZE, rtn4_embedding, rtn4_gemv
from .kernels.ternary_expert import (
    ternary_expert_down_sum,
    ternary_expert_gemv,
    ternary_expert_swiglu,
)
from .kernels.ternary_gemv import ternary_gemv


def add_adapter_delta(layer, y, x, **_kwargs):
    """No-op unless a low-rank adapter is attached as ``layer._adapter``."""
    adapter = getattr(layer, "_adapter", None)
    if adapter is None:
        return y
    return adapter(y, x, **_kwargs)


class PackedTernaryLinear:
    """Codes ``[N, nwords]`` + per-row alpha; ``forward(x, rms_weight=None)``."""

    def __init__(self, packed_weight, row_alpha):
        self.packed_weight = packed_weight.contiguous()
        self.row_alpha = row_alpha.contiguous()

    def forward(self, x, rms_weight=None, rms_eps: float = 1e-6):
        y = ternary_gemv(x, self.packed_weight, self.row_alpha, rms_weight=rms_weight,
                         rms_eps=rms_eps)
        return add_adapter_delta(self, y, x, rms_weight=rms_weight, rms_eps=rms_eps)

    __call__ = forward


class PackedTernaryExperts:
    """Stacked experts ``[E, N, nwords]``; one fused launch over selected ids."""

    def __init__(self, packed_weight, row_alpha):
        self.packed_weight = packed_weight.contiguous()
        self.row_alpha = row_alpha.contiguous()

    def forward(self, x, expert_ids):
        y = ternary_expert_gemv(x, self.packed_weight, self.row_alpha, expert_ids)
        return add_adapter_delta(self, y, x, expert_ids=expert_ids)

    def swiglu(self, x, expert_ids):
        y = ternary_expert_swiglu(x, self.packed_weight, self.row_alpha, expert_ids)
        return add_adapter_delta(self, y, x, expert_ids=expert_ids)

    def down_sum(self, x, expert_ids, topk_weight, residual=None):
        return ternary_expert_down_sum(x, self.packed_weight, self.row_alpha, expert_ids,
                                       topk_weight, residual=residual)

    __call__ = forward


class PackedRTN4Linear:
    """4-bit head in ``[N, nwords]`` order."""

    def __init__(self, packed_weight, scales, biases, group_size: int = HEAD_GROUP_SIZE):
        self.packed_weight = packed_weight.contiguous()
        self.scales = scales.contiguous()
        self.biases = biases.contiguous()
        self.group_size = group_size

    def forward(self, x):
        y = rtn4_gemv(x, self.packed_weight, self.scales, self.biases, group_size=self.group_size)
        return add_adapter_delta(self, y, x)

    __call__ = forward


class PackedRTN4Embedding:
    def __init__(self, packed_weight, scales, biases, group_size: int = HEAD_GROUP_SIZE):
        self.packed_weight = packed_weight
        self.scales = scales
        self.biases = biases
        self.group_size = group_size

    def forward(self, input_ids):
        return rtn4_embedding(input_ids, self.packed_weight, self.scales, self.biases,
                              group_size=self.group_size)

    __call__ = forward
