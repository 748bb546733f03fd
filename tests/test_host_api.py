"""Host-side argument checks of the drop-in wrappers, mirroring the
reference's exception types and message stems (CPU; no kernel runs).

Reference: tests/test_ternary_gemv.py:198-206, tests/test_ternary_expert.py:114-127,
tests/test_rtn4.py:255-263; wrapper checks in src/maple_run/kernels/*.py.
"""

from __future__ import annotations

import pytest
import torch

from maple_amd.kernels import (
    moe_dispatch,
    rtn4_gemv,
    router_topk,
    ternary_expert_gemv,
    ternary_expert_swiglu,
    ternary_gemv,
)


def test_ternary_gemv_requires_device_tensors():
    x = torch.randn(128)
    w = torch.zeros(16, 8, dtype=torch.uint32)
    with pytest.raises(RuntimeError, match="CUDA"):
        ternary_gemv(x, w, torch.ones(16))


def test_expert_rejects_2d_and_non_uint32_before_device_check():
    x = torch.randn(2, 128)
    ids = torch.zeros(2, 2, dtype=torch.int32)
    with pytest.raises(ValueError, match="3-D"):
        ternary_expert_gemv(x, torch.zeros(16, 8, dtype=torch.uint32), torch.ones(16), ids)
    with pytest.raises(TypeError, match="uint32"):
        ternary_expert_gemv(x, torch.randn(4, 16, 8).bfloat16(), torch.ones(4, 16), ids)
    with pytest.raises(RuntimeError, match="CUDA"):
        ternary_expert_gemv(x, torch.zeros(4, 16, 8, dtype=torch.uint32), torch.ones(4, 16), ids)


def test_swiglu_rejects_non_uint32():
    with pytest.raises(ValueError, match="uint32"):
        ternary_expert_swiglu(torch.randn(1, 128), torch.randn(4, 16, 8), torch.ones(4, 16),
                              torch.zeros(1, 2, dtype=torch.int32))


def test_rtn4_rejects_dense_weight_and_bad_rank():
    x = torch.randn(128)
    with pytest.raises(TypeError, match="uint32"):
        rtn4_gemv(x, torch.randn(16, 16).bfloat16(), torch.ones(16, 2), torch.ones(16, 2))
    with pytest.raises(ValueError, match="2-D"):
        rtn4_gemv(x, torch.zeros(2, 16, 16, dtype=torch.uint32), torch.ones(16, 2), torch.ones(16, 2))


def test_router_and_dispatch_require_device():
    with pytest.raises(RuntimeError, match="CUDA"):
        router_topk(torch.randn(1, 16), torch.randn(4, 16), 2)
    with pytest.raises(RuntimeError, match="CUDA"):
        moe_dispatch(torch.zeros(3, 2, dtype=torch.int32), 4)
