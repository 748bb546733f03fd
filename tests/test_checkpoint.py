"""packed-ternary-v1 checkpoints (CPU): a decoder written with
``checkpoint.save_decoder`` reads back tensor for tensor through the
reference's loading rules (reference model.py:509-559, 664-832) -- the
``[q; k; v]`` and ``[up; gate]`` concatenation orders, the uint32 view of the
packed codes, bf16 router and RTN scales/biases, float32 ``row_alpha`` kept as
written (model.py:728-748) -- and configs the decoder cannot run are
refused."""

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
        if k.endswith("alpha"):  # written as float32 and kept so: the same values
            assert b[k].dtype == torch.float32 and torch.equal(a[k].float(), b[k]), k
            continue
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
    assert torch.equal(qkv, L0.qkv) and torch.equal(alpha, L0.qkv_alpha.float())


def test_float32_alphas_stay_float32(tmp_path):
    """row_alpha values bf16 cannot hold come back unrounded (the reference
    keeps row_alpha in float32 and its kernels read it so)."""
    model = SyntheticDecoder(SMALL, "cpu", seed=6, max_len=64)
    g = torch.Generator().manual_seed(0)
    for L in model.layers:
        L.qkv_alpha = torch.rand(L.qkv_alpha.shape, generator=g) * 0.04 + 0.01
        L.moe.down_alpha = torch.rand(L.moe.down_alpha.shape, generator=g) * 0.04 + 0.01
    assert not torch.equal(model.layers[0].qkv_alpha, model.layers[0].qkv_alpha.bfloat16().float())
    checkpoint.save_decoder(model, tmp_path)
    back = checkpoint.load_decoder(tmp_path, "cpu", max_len=64)
    for L, B in zip(model.layers, back.layers):
        assert B.qkv_alpha.dtype == torch.float32 and torch.equal(B.qkv_alpha, L.qkv_alpha)
        assert B.moe.down_alpha.dtype == torch.float32 and torch.equal(B.moe.down_alpha, L.moe.down_alpha)


def test_rtn_group_defaults_to_64_and_must_cover_hidden(saved, tmp_path):
    _, d = saved
    config = json.loads((d / "config.json").read_text())
    meta = dict(config["maple_run"], rtn_4bit={"bits": 4})
    assert checkpoint.decoder_config(dict(config, maple_run=meta)).rtn_group == 64
    # the saved tables have group 128: a config claiming 64 is refused on load
    import shutil
    shutil.copytree(d, tmp_path / "c", dirs_exist_ok=True)
    (tmp_path / "c" / "config.json").write_text(json.dumps(dict(config, maple_run=meta)))
    with pytest.raises(ValueError, match="group_size"):
        checkpoint.load_decoder(tmp_path / "c", "cpu", max_len=64)


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
        checkpoint.decoder_config(dict(config, head_dim=96))
    # the reference's layer pattern: sliding layers with a window, NoPE global layers
    cfg = checkpoint.decoder_config(dict(config, layer_types=["sliding_attention", "full_attention"],
                                         sliding_window=64, nope_on_global_attention=True))
    assert cfg.layer_attention(0) == (64, True) and cfg.layer_attention(1) == (None, False)


def test_maple_preview_config_maps_to_the_kernels(saved):
    """Maple-Preview's shapes (docs/HANDOFF.md:190-199 of the reference): 24
    layers, hidden 2048, 16 query / 4 KV heads of 128, 256 experts top-8 with
    intermediate 512, vocab 151936, layer_types 3 sliding (window 512) : 1
    full, NoPE on the full layers, RTN group 64 when the converter names none."""
    _, d = saved
    config = json.loads((d / "config.json").read_text())
    meta = dict(config["maple_run"])
    meta.pop("rtn_4bit")
    maple = dict(config, hidden_size=2048, num_hidden_layers=24, num_attention_heads=16,
                 num_key_value_heads=4, head_dim=128, num_experts=256, num_experts_per_tok=8,
                 moe_intermediate_size=512, vocab_size=151936, partial_rotary_factor=0.5,
                 layer_types=["sliding_attention"] * 3 + ["full_attention"], sliding_window=512,
                 nope_on_global_attention=True, maple_run=meta)
    maple["layer_types"] = maple["layer_types"] * 6
    cfg = checkpoint.decoder_config(maple)
    assert (cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.qkv_rows) == (2048, 16, 4, 128, 3072)
    assert (cfg.experts, cfg.inter, cfg.top_k, cfg.rtn_group, cfg.rotary_dim) == (256, 512, 8, 64, 64)
    assert [cfg.layer_attention(i) for i in range(4)] == [(512, True)] * 3 + [(None, False)]
    assert cfg.layer_attention(23) == (None, False) and cfg.layer_attention(22) == (512, True)
