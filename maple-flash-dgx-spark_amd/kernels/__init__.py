"""HIP kernels of the hot path, exported under the reference's names
(``src/maple_run/kernels/__init__.py:5-39``), plus ``moe_dispatch``."""

from __future__ import annotations

__all__ = [
    "ternary_gemv",
    "ternary_expert_gemv",
    "ternary_expert_swiglu",
    "ternary_expert_down_sum",
    "router_topk",
    "moe_dispatch",
    "rtn4_gemv",
    "rtn4_embedding",
    "rms_norm",
    "add_rms_norm",
    "moe_reduce_add",
]

_WHERE = {
    "ternary_gemv": "ternary_gemv",
    "ternary_expert_gemv": "ternary_expert",
    "ternary_expert_swiglu": "ternary_expert",
    "ternary_expert_down_sum": "ternary_expert",
    "router_topk": "router",
    "moe_dispatch": "dispatch",
    "rtn4_gemv": "rtn4",
    "rtn4_embedding": "rtn4",
    "rms_norm": "fused_norm",
    "add_rms_norm": "fused_norm",
    "moe_reduce_add": "fused_norm",
}


def __getattr__(name: str):
    mod = _WHERE.get(name)
    if mod is None:
        raise AttributeError(f"module {__name__!r} has no attribute {name}")
    import importlib

    fn = getattr(importlib.import_module(f"{__name__}.{mod}"), name)
    # Importing a submodule binds its name on this package; a function that
    # shares its module's name (ternary_gemv) must win.
    globals()[name] = fn
    return fn
