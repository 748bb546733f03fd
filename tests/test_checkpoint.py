"""packed-ternary-v1 checkpoints (CPU): a decoder written with
``checkpoint.save_decoder`` reads back tensor for tensor through the
reference's loading rules (reference model.py:509-559, 664-832) -- the
``[q; k; v]`` and ``[up; gate]`` concatenation orders, the uint32 view of the
packed codes, bf16 router / alphas / RTN scales -- and configs the decoder
cannot run are refused."""

from __future__ import annotations

import dataclasses
import json

import pytest
import torch

from maple_amd import checkpoint
from maple_amd.model import DecoderConfig, SyntheticDecoder

SMALL = DecoderConfig(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64, experts=8, inter=256,
                      top_k=2, vocab=1024, rtn_group=128, lm_scale=(0.01, 0.02))


@pytest.fixture(scope="module")
def saved(tmp_path_factory):
    model = SyntheticDecoder(SMALL, "cpu", seed=5, max_len=64)
    d = tmp_path_factory.mktemp("packed")
    checkpoint.save_decoder(model, d)
    return model, d


def _tensors(model):
    out = {"final_norm": model.final_norm}
    for name, t in (("embed", model.embed), ("lm_head", model.lm_head)):
        for j, x in enumerate(t):
            out[f"{name}{j}"] = x
    for i, L in enumerate(model.layers):
        for f in ("qkv", "qkv_alpha", "o", "o_alpha", "input_ln", "post_ln", "q_norm", "k_norm"):
            out[f"{i}.{f}"] = getattr(L, f)
        for f in ("gate_weight", "up_gate_packed", "up_gate_alpha", "down_packed", "down_alpha"):
            out[f"{i}.moe.{f}"] = getattr(L.moe, f)
    return out


def test_round_trip_is_exact(saved):
    model, d = saved
    back = checkpoint.load_decoder(d, "cpu", max_len=64)
    # lm_scale only seeds the synthetic RTN tables (not part of a checkpoint);
    # the layer types come back spelled out, with the same attention per layer
    assert dataclasses.replace(back.cfg, lm_scale=SMALL.lm_scale, layer_types=()) == SMALL
    assert [back.cfg.layer_attention(i) for i in range(SMALL.layers)] == \
        [SMALL.layer_attention(i) for i in range(SMALL.layers)]
    a, b = _tensors(model), _tensors(back)
    assert a.keys() == b.keys()
    for k in a:
        assert a[k].dtype == b[k].dtype and a[k].shape == b[k].shape, k
        assert torch.equal(a[k], b[k]), k
    torch.testing.assert_close(back.cos, model.cos, rtol=0, atol=0)


def test_file_layout_follows_the_reference(saved):
    model, d = saved
    config, w = checkpoint.read_weights(d, "cpu")
    assert config["maple_run"]["format"] == "packed-ternary-v1"
    nq = SMALL.heads * SMALL.head_dim
    L0 = model.layers[0]
    # q rows first, then k, then v; the codes are stored as int32 words
    assert w["model.layers.0.self_attn.q_proj.weight"].dtype == torch.int32
    assert torch.equal(checkpoint.as_uint32(w["model.layers.0.self_attn.q_proj.weight"]), L0.qkv[:nq])
    # per expert: up rows, then gate rows
    up = checkpoint.as_uint32(w["model.layers.0.mlp.switch_mlp.up_proj.weight"])
    assert tuple(up.shape) == (SMALL.experts, SMALL.inter, SMALL.hidden // 16)
    assert torch.equal(up, L0.moe.up_gate_packed[:, :SMALL.inter])
    qkv, alpha = checkpoint.cat_qkv(dict(w), "model.layers.0")
    assert torch.equal(qkv, L0.qkv) and torch.equal(alpha.to(torch.bfloat16), L0.qkv_alpha)


def test_unconverted_and_unsupported_configs_are_refused(saved, tmp_path):
    _, d = saved
    config = json.loads((d / "config.json").read_text())
    with pytest.raises(ValueError, match="packed-ternary-v1"):
        checkpoint.require_packed_format({k: v for k, v in config.items() if k != "maple_run"})
    with pytest.raises(NotImplementedError):
        checkpoint.decoder_config(dict(config, layer_types=["chunked_attention", "full_attention"]))
    with pytest.raises(NotImplementedError):
        checkpoint.decoder_config(dict(config, use_qk_norm=False))
    with pytest.raises(NotImplementedError):
        checkpoint.decoder_config(dict(config, head_dim=128))
    # the reference's layer pattern: sliding layers with a window, NoPE global layers
    cfg = checkpoint.decoder_config(dict(config, layer_types=["sliding_attention", "full_attention"],
                                         sliding_window=64, nope_on_global_attention=True))
    assert cfg.layer_attention(0) == (64, True) and cfg.layer_attention(1) == (None, False)
