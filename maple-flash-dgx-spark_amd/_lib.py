"""ctypes binding of ``libmaple_amd.so`` (the C ABI in ``include/maple_amd.h``).

The library is loaded after ``torch`` so that it binds to the HIP runtime torch
already mapped (both carry the SONAME ``libamdhip64.so.7``).  There is no
fallback: if the library is missing, every call raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libmaple_amd.so")
# The same library with the one-launch MoE layer's phase stamps compiled in
# (ma_moe_phase_stamps); for timelines only, never loaded unless asked for.
STAMPED_LIB_PATH = Path(__file__).resolve().with_name("libmaple_amd_stamps.so")

F32, BF16, F16 = 0, 1, 2
_DTYPES = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float
_Z = ctypes.c_size_t
_PL = ctypes.POINTER(ctypes.c_int64)

# name -> argtypes (restype is int unless listed in _RESTYPES)
_SIGNATURES = {
    "ma_version": [],
    "ma_last_error": [],
    "ma_ternary_gemv": [_P, _I, _L, _L, _P, _L, _L, _I, _P, _I, _P, _I, _F, _P, _L, _P],
    "ma_ternary_gemv_workspace_bytes": [_L, _L, _I],
    "ma_ternary_gemv_ws": [_P, _I, _L, _L, _P, _L, _L, _I, _P, _I, _P, _I, _F, _P, _L, _P, _Z, _P],
    "ma_router_workspace_bytes": [_L, _L],
    "ma_router_topk": [_P, _I, _L, _L, _P, _I, _L, _L, _P, _I, _P, _P, _P, _Z, _P],
    "ma_router_topk_pairs": [_P, _I, _L, _L, _P, _I, _L, _L, _P, _I, _P, _P, _P, _P, _P, _Z, _P],
    "ma_moe_dispatch": [_P, _I, _L, _I, _P, _P, _P, _P, _P],
    "ma_ternary_expert_gemv": [_P, _I, _L, _L, _P, _L, _L, _L, _I, _P, _I, _P, _I, _L, _P, _L, _P],
    "ma_ternary_expert_swiglu": [_P, _I, _L, _L, _L, _P, _L, _L, _L, _I, _P, _I, _P, _I, _P, _L, _P],
    "ma_ternary_expert_down_sum": [_P, _I, _L, _P, _L, _L, _L, _I, _P, _I, _P, _I, _P, _P, _I,
                                   _L, _L, _P, _L, _P],
    "ma_ternary_expert_down_combine": [_P, _I, _L, _P, _L, _L, _L, _I, _P, _I, _P, _I, _P, _P, _I,
                                       _L, _L, _P, _L, _P],
    "ma_moe_reduce_add": [_P, _I, _L, _L, _L, _P, _P, _I, _P, _P],
    "ma_rms_norm": [_P, _I, _L, _L, _P, _I, _F, _P, _P],
    "ma_add_rms_norm": [_P, _P, _I, _L, _L, _P, _I, _F, _P, _P, _P],
    "ma_rtn4_gemv": [_P, _I, _L, _L, _P, _L, _L, _I, _P, _I, _P, _I, _L, _P, _L, _P],
    "ma_rtn4_gemv_ws": [_P, _I, _L, _L, _P, _L, _L, _I, _P, _I, _P, _I, _L, _P, _L, _P, _Z, _P],
    "ma_rtn4_gemv_workspace_bytes": [_L, _L, _L],
    "ma_rtn4_embedding": [_P, _I, _L, _P, _L, _L, _P, _I, _P, _I, _L, _P, _P],
    "ma_grouped_workspace_bytes": [_L, _L, _L],
    "ma_qk_norm_rope_store": [_P, _L, _L, _I, _I, _I, _P, _P, _I, _P, _P, _I, _L, _L, _I, _I, _F,
                              _P, _P, _P, _P, _L, _L, _P, _P],
    "ma_gqa_workspace_bytes": [_L, _I, _L, _I],
    "ma_decode_gqa_attn": [_P, _L, _I, _I, _I, _P, _P, _L, _L, _P, _P, _L, _F, _P, _P, _Z, _P],
    "ma_decode_attn_fused": [_P, _L, _L, _I, _I, _I, _P, _P, _I, _P, _P, _I, _L, _L, _I, _I, _F,
                             _P, _P, _P, _P, _L, _L, _L, _F, _P, _P, _Z, _P, _P, _I, _L, _P, _P],
    "ma_decode_attn_o_supported": [_L, _I, _I, _I, _L, _L, _L],
    "ma_decode_attn_form": [_L, _I, _I, _L, _L, _I, _I],
    "ma_moe_fused_workspace_bytes": [_L, _L, _L, _L],
    "ma_moe_fused": [_P, _P, _P, _I, _F, _P, _P, _P, _L, _L, _L, _L, _P, _P, _P, _P, _I, _P, _P, _P,
                     _P, _Z, _P, _P, _I, _P, _F, _L, _P, _P, _L, _P],
    # x, attn, o_w, o_alpha, norm_w, norm_dt, eps, gate, bias, E, H, I, K, ug, ug_a, dn, dn_a, adt, y, ids,
    # wts, ws, ws_bytes, nx_w, nx_a, nx_adt, nx_rms, nx_eps, nx_rows, nx_out, pf, pf_bytes, stream
    "ma_moe_fused_o": [_P, _P, _P, _P, _P, _I, _F, _P, _P, _L, _L, _L, _L, _P, _P, _P, _P, _I, _P, _P,
                       _P, _P, _Z, _P, _P, _I, _P, _F, _L, _P, _P, _L, _P],
    "ma_moe_fused_timed_out": [_P, _P, _P],
    "ma_moe_fused_resident": [_L, _L, _L, _L, _PL, _PL],
    "ma_moe_fused_form": [_L, _L, _L, _L],
    "ma_moe_phase_stamps": [_P, _P, _P],
    "ma_xcd_forms_disable": [_I, _I],
    "ma_moe_route_workspace_bytes": [_L, _L],
    "ma_moe_route": [_P, _P, _L, _L, _P, _I, _F, _P, _P, _L, _I, _P, _P, _P, _P, _P, _P, _P, _P,
                     _P, _P, _P, _Z, _P],
    "ma_argmax_rows": [_P, _I, _L, _L, _L, _P, _P],
    "ma_argmax_workspace_bytes": [_L],
    "ma_argmax_rows_ws": [_P, _I, _L, _L, _L, _P, _P, _Z, _P],
    "ma_ternarize": [_P, _I, _L, _L, _F, _P, _P, _P],
    "ma_ternary_gemv_combine_ws": [_P, _P, _P, _L, _P, _P, _L, _P, _L, _L, _P, _I, _P, _I, _F, _P, _L,
                                   _P, _Z, _P],
    "ma_moe_grouped": [_P, _L, _P, _P, _L, _L, _P, _P, _P, _P, _I, _L, _L, _L, _P, _P, _P, _P, _P,
                       _I, _P, _L, _P, _P, _Z, _P],
    "ma_moe_grouped_noalloc_max_bytes": [],
    "ma_sampler_workspace_bytes": [_L, _L, _I],
    "ma_fused_sample": [_P, _I, _L, _L, _L, _P, _I, _F, _F, _P, _Z, _P, _P],
    "ma_rtn4_indexed_gemv": [_P, _I, _L, _L, _P, _L, _L, _L, _P, _I, _P, _I, _L, _P, _L, _P, _L, _P],
    "ma_flash_head_workspace_bytes": [_L, _L],
    "ma_flash_head": [_P, _P, _P, _P, _I, _L, _L, _P, _P, _P, _I, _L, _L, _P, _L, _P, _P, _P, _P, _L, _L,
                      _L, _P, _P, _P, _Z, _P],
    "ma_moe_grouped_noalloc": [_P, _L, _P, _P, _L, _L, _P, _P, _P, _P, _I, _L, _L, _L, _P, _P, _P, _P,
                               _P, _I, _P, _L, _P, _P],
}
_RESTYPES = {"ma_last_error": ctypes.c_char_p, "ma_router_workspace_bytes": _Z,
             "ma_ternary_gemv_workspace_bytes": _Z,
             "ma_grouped_workspace_bytes": _Z, "ma_gqa_workspace_bytes": _Z, "ma_argmax_workspace_bytes": _Z,
             "ma_moe_fused_workspace_bytes": _Z, "ma_moe_route_workspace_bytes": _Z,
             "ma_moe_grouped_noalloc_max_bytes": _Z, "ma_sampler_workspace_bytes": _Z,
             "ma_flash_head_workspace_bytes": _Z, "ma_rtn4_gemv_workspace_bytes": _Z}

_lib = None


def declared_symbols() -> list[str]:
    return list(_SIGNATURES)


def use_stamped_library() -> None:
    """Make ``load`` bind the stamped variant instead (before the first load)."""
    global LIB_PATH
    if _lib is not None and LIB_PATH != STAMPED_LIB_PATH:
        raise RuntimeError("the maple_amd library is already loaded; select the stamped one first")
    LIB_PATH = STAMPED_LIB_PATH


def load() -> ctypes.CDLL:
    """Load and declare the library once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"maple_amd HIP library not found at {LIB_PATH}; build it with "
                "`python maple-flash-dgx-spark_amd/build.py` (there is no CPU fallback)."
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                continue
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        _lib = lib
    return _lib


def dtype_code(t: torch.Tensor, what: str) -> int:
    code = _DTYPES.get(t.dtype)
    if code is None:
        raise TypeError(f"{what} must be float32, bfloat16 or float16; got {t.dtype}.")
    return code


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


_ERRORS = {1: ValueError, 2: TypeError, 3: RuntimeError}


def call(name: str, *args) -> int:
    """Call ``name``; map a non-zero status to the reference's exception type."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status != 0:
        msg = lib.ma_last_error().decode(errors="replace")
        raise _ERRORS.get(status, RuntimeError)(msg or f"{name} failed with status {status}")
    return status
