"""HIP kernels of the hot path, exported under the reference's names
(``src/maple_run/kernels/__init__.py:5-39``), plus ``moe_dispatch``.

Importing this package does not load the HIP library; the first kernel call
does (and raises if it has not been built).  The functions are bound eagerly
so that ``ternary_gemv`` names the function even after its submodule of the
same name has been imported.
"""

from __future__ import annotations

from .decode_attn import apply_qkv_decode, decode_attention, decode_gqa_attn, gqa_workspace
from .dispatch import moe_dispatch
from .fused_norm import add_rms_norm, moe_reduce_add, rms_norm
from .greedy import greedy_argmax
from .router import router_topk
from .rtn4 import rtn4_embedding, rtn4_gemv, rtn4_indexed_gemv
from .ternary_expert import ternary_expert_down_sum, ternary_expert_gemv, ternary_expert_swiglu
from .ternary_gemv import ternary_gemv

__all__ = [
    "ternary_gemv",
    "ternary_expert_gemv",
    "ternary_expert_swiglu",
    "ternary_expert_down_sum",
    "router_topk",
    "moe_dispatch",
    "rtn4_gemv",
    "rtn4_embedding",
    "rtn4_indexed_gemv",
    "rms_norm",
    "add_rms_norm",
    "moe_reduce_add",
    "apply_qkv_decode",
    "decode_gqa_attn",
    "decode_attention",
    "gqa_workspace",
    "greedy_argmax",
]
