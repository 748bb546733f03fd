"""The C ABI: the built library loads and exports every declared symbol (CPU).

No compute call is made here (no GPU); the GPU tests call through the same
entry points.
"""

from __future__ import annotations

import ctypes

import torch
import re
from pathlib import Path

import pytest

from maple_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "maple_amd.h"


def declared_in_header() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(ma_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_path():
    names = declared_in_header()
    for must in ("ma_ternary_gemv", "ma_router_topk", "ma_moe_dispatch", "ma_ternary_expert_swiglu",
                 "ma_ternary_expert_gemv", "ma_ternary_expert_down_sum", "ma_moe_reduce_add",
                 "ma_rtn4_gemv", "ma_rtn4_embedding", "ma_rms_norm", "ma_add_rms_norm"):
        assert must in names


def test_library_exports_every_declared_symbol():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in declared_in_header() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_covers_header():
    assert set(declared_in_header()) <= set(_lib.declared_symbols())


def test_version_and_error_string():
    lib = _lib.load()
    assert lib.ma_version() >= 100
    assert isinstance(lib.ma_last_error(), bytes)


def test_size_errors_map_without_a_gpu():
    """Bad sizes are rejected on the host before any launch: status -> ValueError."""
    with pytest.raises(ValueError, match="bad sizes"):
        _lib.call("ma_ternary_gemv", None, 1, -1, 16, None, 4, 1, 0, None, 0, None, 0, 1e-6,
                  None, 4, None)
    with pytest.raises(ValueError, match="top_k"):
        _lib.call("ma_router_topk", None, 1, 1, 16, None, 1, 4, 16, None, 5, None, None, None, 0, None)
    with pytest.raises(ValueError, match="n_experts"):
        _lib.call("ma_moe_dispatch", None, 0, 8, 0, None, None, None, None, None)
    with pytest.raises(ValueError, match="groups"):
        _lib.call("ma_rtn4_gemv", None, 1, 1, 96, None, 4, 12, 0, None, 1, None, 1, 64, None, 4, None)
    # 2^22 tokens x hidden 2048: x' holds 2^32 uint32 words, past the batched
    # kernels' 32-bit copy offsets (rejected before any launch; the pointers
    # are never dereferenced)
    fake = 0x10000
    with pytest.raises(ValueError, match="split the batch"):
        _lib.call("ma_moe_grouped", fake, 2048, None, None, 1 << 22, 8, fake, fake, fake, fake,
                  _lib.dtype_code(torch.empty(0, dtype=torch.bfloat16), "a"), 64, 2048, 768, fake, fake,
                  fake, fake, None, 0, None, 0, fake, fake, 1 << 62, None)


def test_stamped_variant_exports_the_same_symbols_and_its_stamps_fit():
    """libmaple_amd_stamps.so (the one-launch layer with phase stamps) exports
    everything the header declares; only it reports a stamp layout, and the
    stamp rows lie inside the workspace ma_moe_fused_workspace_bytes sizes."""
    if not _lib.STAMPED_LIB_PATH.exists():
        pytest.fail(f"{_lib.STAMPED_LIB_PATH} not built; run __graft_entry__.build()")
    st = ctypes.CDLL(str(_lib.STAMPED_LIB_PATH))
    missing = [n for n in declared_in_header() if not hasattr(st, n)]
    assert not missing, f"declared but not exported: {missing}"
    off, words, wgs = ctypes.c_size_t(), ctypes.c_int(), ctypes.c_int()
    fn = st.ma_moe_phase_stamps
    fn.argtypes = [ctypes.c_void_p] * 3
    assert fn(ctypes.byref(off), ctypes.byref(words), ctypes.byref(wgs)) == 0
    assert words.value == 16 and wgs.value == 256 and off.value % 256 == 0
    size = st.ma_moe_fused_workspace_bytes
    size.argtypes = [ctypes.c_int64] * 4
    size.restype = ctypes.c_size_t
    for inter in (768, 512):
        assert off.value + 4 * words.value * wgs.value <= size(64, 2048, inter, 8)
    plain = _lib.load()
    assert plain.ma_moe_phase_stamps(ctypes.byref(off), ctypes.byref(words), ctypes.byref(wgs)) != 0
