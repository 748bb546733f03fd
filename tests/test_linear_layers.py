"""The packed layer objects (maple_amd.linear, the reference's linear.py
classes): construction checks on the CPU, and on the GPU each layer's call
equals the kernel it forwards to, bit for bit."""

from __future__ import annotations

import pytest
import torch

from maple_amd import linear, synthetic


def test_layers_refuse_non_uint32_codes_and_mismatched_scales():
    codes = torch.zeros(4, 2, dtype=torch.int32)
    with pytest.raises(TypeError):
        linear.PackedTernaryLinear(codes, torch.ones(4))
    with pytest.raises(TypeError):
        linear.PackedRTN4Linear(codes, torch.ones(4, 1), torch.ones(4, 1), group_size=16)
    u = codes.view(torch.uint32)
    with pytest.raises(ValueError):
        linear.PackedRTN4Embedding(u, torch.ones(4, 2), torch.ones(4, 2), group_size=16)
    emb = linear.PackedRTN4Embedding(u, torch.ones(4, 1), torch.ones(4, 1), group_size=16)
    assert emb.group_size == 16 and emb.packed_weight.is_contiguous()


def test_adapter_hook_is_identity_without_an_adapter():
    class L:
        pass

    y = torch.arange(3.0)
    assert linear.add_adapter_delta(L(), y, None) is y
    layer = L()
    layer._adapter = lambda y, x, **kw: y + 1
    assert torch.equal(linear.add_adapter_delta(layer, y, None), y + 1)


@pytest.mark.gpu
def test_layers_call_their_kernels(dev):
    from maple_amd.kernels import (rtn4_embedding, rtn4_gemv, ternary_expert_down_sum, ternary_expert_gemv,
                                   ternary_expert_swiglu, ternary_gemv)

    w, a = synthetic.ternary_linear(256, 512, 3, dev)
    x = synthetic.randn_bf16((3, 512), 4, dev)
    rms = torch.ones(512, device=dev)
    lin = linear.PackedTernaryLinear(w, a)
    assert torch.equal(lin(x, rms_weight=rms), ternary_gemv(x, w, a, rms_weight=rms))
    L = synthetic.make_moe_layer(256, 8, 128, seed=5, device=dev)
    ids = torch.tensor([[1, 6], [0, 3]], device=dev, dtype=torch.int32)
    wts = torch.tensor([[0.7, 0.3], [0.4, 0.6]], device=dev)
    xe = synthetic.randn_bf16((2, 256), 6, dev)
    ug = linear.PackedTernaryExperts(L.up_gate_packed, L.up_gate_alpha)
    dn = linear.PackedTernaryExperts(L.down_packed, L.down_alpha)
    assert torch.equal(ug(xe, ids), ternary_expert_gemv(xe, L.up_gate_packed, L.up_gate_alpha, ids))
    h = ug.swiglu(xe, ids)
    assert torch.equal(h, ternary_expert_swiglu(xe, L.up_gate_packed, L.up_gate_alpha, ids))
    assert torch.equal(dn.down_sum(h, ids, wts, residual=xe),
                       ternary_expert_down_sum(h, L.down_packed, L.down_alpha, ids, wts, residual=xe))
    hw, hs, hb = synthetic.rtn4_table(1000, 512, 64, 7, dev)
    head = linear.PackedRTN4Linear(hw, hs, hb, group_size=64)
    assert torch.equal(head(x), rtn4_gemv(x, hw, hs, hb, group_size=64))
    emb = linear.PackedRTN4Embedding(hw, hs, hb, group_size=64)
    tok = torch.tensor([0, 999, 17], device=dev)
    assert torch.equal(emb(tok), rtn4_embedding(tok, hw, hs, hb, group_size=64))
