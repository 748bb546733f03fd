"""ma_moe_grouped_noalloc (no workspace, no allocation) against ma_moe_grouped.

Both are called through the C ABI on the same inputs; the no-allocation form
stages in the library's own device array and runs the same kernels, so y and
h must be equal bit for bit.  Two calls in a row, the second smaller (the
array keeps the first call's contents): 200 tokens (1600 pairs, the
prefill-sized tiles) then 16 tokens (128 pairs, the decode-sized tiles);
then a call larger than the array is refused.
"""

from __future__ import annotations

import pytest
import torch

from maple_amd import _lib, synthetic
from maple_amd.kernels import moe_dispatch, router_topk
from maple_amd.moe import moe_grouped

pytestmark = pytest.mark.gpu

H, E, I, K = 2048, 64, 768, 8


def _noalloc(x, L, ids, wts, d, residual, h_out, y):
    tokens = x.shape[0]
    _lib.call(
        "ma_moe_grouped_noalloc",
        _lib.ptr(x), x.stride(0), None, None, tokens, K,
        _lib.ptr(L.up_gate_packed), _lib.ptr(L.up_gate_alpha), _lib.ptr(L.down_packed),
        _lib.ptr(L.down_alpha), _lib.dtype_code(L.up_gate_alpha, "row_alpha"), E, H, I,
        _lib.ptr(d.offsets), _lib.ptr(d.pair_ids), _lib.ptr(d.inverse),
        _lib.ptr(wts.reshape(-1).contiguous()), _lib.ptr(residual), _lib.dtype_code(residual, "residual"),
        _lib.ptr(h_out), I, _lib.ptr(y), _lib.stream_of(x))


def test_noalloc_equals_workspace_entry_point(dev):
    L = synthetic.make_moe_layer(H, E, I, seed=21, device=dev)
    assert int(_lib.load().ma_moe_grouped_noalloc_max_bytes()) == 16 << 20
    for step, tokens in enumerate((200, 16)):
        x = synthetic.randn_bf16((tokens, H), 900 + tokens, dev)
        res = synthetic.randn_bf16((tokens, H), 950 + tokens, dev)
        ids, wts = router_topk(x, L.gate_weight, K)
        d = moe_dispatch(ids, E)
        y_ref, h_ref = moe_grouped(x, L, ids, wts, res, return_h=True, dispatch=d)
        y = torch.empty_like(y_ref)
        h = torch.empty(tokens * K, I, device=dev, dtype=torch.bfloat16)
        _noalloc(x, L, ids, wts, d, res, h, y)
        torch.cuda.synchronize()
        assert torch.equal(h.reshape(h_ref.shape), h_ref), f"call {step} ({tokens} tokens): h"
        assert torch.equal(y, y_ref), f"call {step} ({tokens} tokens): y"


def test_noalloc_rejects_calls_beyond_its_array(dev):
    L = synthetic.make_moe_layer(H, E, I, seed=22, device=dev)
    tokens = 400  # 3200 pairs: 18 MB of staging > 16 MiB
    x = synthetic.randn_bf16((tokens, H), 990, dev)
    ids, wts = router_topk(x, L.gate_weight, K)
    d = moe_dispatch(ids, E)
    y = torch.empty(tokens, H, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="scratch"):
        _noalloc(x, L, ids, wts, d, x, None, y)
