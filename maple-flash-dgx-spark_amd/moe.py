"""The MoE FFN block on the HIP kernels (reference ``src/maple_run/model.py:448-474``).

``MapleSparseMoeBlock`` keeps the reference composition and call signature:
router -> fused up+gate SwiGLU -> down -> top-k combine (+ residual), with no
host sync and no per-expert Python loop.  The down projection and the combine
run as one launch (``ternary_expert_down_sum``), which skips the reference's
bf16 rounding of each slot's down output before the combine
(``model.py:470-473``); the result stays within bf16 tolerance of the
reference composition.
"""

from __future__ import annotations

import torch

from .kernels.router import router_topk
from .kernels.ternary_expert import ternary_expert_down_sum, ternary_expert_swiglu
from .synthetic import MoELayer


def moe_block(x: torch.Tensor, layer: MoELayer, top_k: int, residual: torch.Tensor | None = None):
    """One MoE layer on ``x [..., H]``; returns ``(y, ids, weights)``."""
    hidden = x.shape[-1]
    xf = x.reshape(-1, hidden)
    ids, wts = router_topk(xf, layer.gate_weight, top_k, bias=layer.router_bias)
    h = ternary_expert_swiglu(xf, layer.up_gate_packed, layer.up_gate_alpha, ids)
    res = None if residual is None else residual.reshape(-1, hidden)
    y = ternary_expert_down_sum(h, layer.down_packed, layer.down_alpha, ids, wts, residual=res)
    return y.reshape(x.shape), ids, wts


class MapleSparseMoeBlock:
    """Top-k softmax router + fused packed SwitchGLU (``model.py:448-474``)."""

    def __init__(self, gate_weight, up_gate, down, top_k: int, moe_intermediate: int,
                 router_bias: torch.Tensor | None = None):
        self.gate_weight = gate_weight
        self.up_gate = up_gate
        self.down = down
        self.top_k = top_k
        self.moe_intermediate = moe_intermediate
        self.router_bias = router_bias

    def __call__(self, hidden_states: torch.Tensor, residual: torch.Tensor | None = None):
        shape = hidden_states.shape
        hidden = shape[-1]
        x = hidden_states.reshape(-1, hidden)
        topk_idx, topk_weight = router_topk(x, self.gate_weight, self.top_k, bias=self.router_bias)
        hidden_e = self.up_gate.swiglu(x, topk_idx)
        res = None if residual is None else residual.reshape(-1, hidden)
        y = self.down.down_sum(hidden_e, topk_idx, topk_weight, residual=res)
        return y.view(shape)
