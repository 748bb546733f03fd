"""``packed-ternary-v1`` checkpoints for the decoder.

Reference: ``src/maple_run/model.py:509-559`` (the format check, the
``[q; k; v]`` and ``[up; gate]`` concatenations, the uint32 view),
``:636-660`` (the config keys), ``:664-832`` (``from_packed``: shards and
index, ``lm_head_flash.*`` dropped, the router and the RTN scales/biases held
in bf16 while ``row_alpha`` and the norms keep the float32 the converter
wrote, the RTN group from ``maple_run.rtn_4bit.group_size`` with 64 as the
default, the per-layer assembly) and ``src/maple_run/convert.py:181-303`` (tensor names,
``config.json["maple_run"]``).

A checkpoint directory holds ``config.json`` -- the model config plus a
``maple_run`` block whose ``format`` is ``packed-ternary-v1`` -- and
safetensors shards (listed by ``model.safetensors.index.json`` when there is
one).  Per layer ``model.layers.{i}.``:
  ``self_attn.{q,k,v,o}_proj.weight`` (packed 2-bit codes, uint32 words viewed
  as int32 in the file) and ``.row_alpha`` (float32);
  ``self_attn.{q,k}_norm.weight``, ``input_layernorm.weight``,
  ``post_attention_layernorm.weight``;
  ``mlp.gate.weight`` (router ``[E, H]``);
  ``mlp.switch_mlp.{up,gate,down}_proj.weight`` (stacked experts ``[E, N,
  K/16]``) and ``.row_alpha`` (``[E, N]``);
and ``model.word_embeddings.{weight,scales,biases}``, ``lm_head.{weight,
scales,biases}`` (4-bit RTN), ``model.norm.weight``.

Layers are ``full_attention`` or ``sliding_attention`` (the last
``sliding_window`` positions), full-attention layers without RoPE when
``nope_on_global_attention`` is set, all with QK-norm, head_dim 64 or 128
(the decode attention kernel's); other configs raise ``NotImplementedError``
instead of decoding wrongly.  With ``flash_head=True`` the ``lm_head_flash.*``
tensors (``model-flashhead.safetensors``) and the ``flash_head`` metadata
build a FlashHead for batch-1 decode (``model.py:750-770``,
``flash_head.py:373-463``).
"""

from __future__ import annotations

import json
from pathlib import Path

import torch

from . import synthetic
from .model import DecoderConfig, DecoderLayerWeights, SyntheticDecoder

FORMAT = "packed-ternary-v1"
HEAD_GROUP_SIZE = 64  # RTN group of the head when the config names none (pack.py:14)


def require_packed_format(config: dict) -> None:
    """``model.py:509-515``: only converted checkpoints load."""
    meta = config.get("maple_run") or {}
    if meta.get("format") != FORMAT:
        raise ValueError(
            "Checkpoint is not maple-run packed-ternary-v1 (config.json has no "
            "maple_run.format == 'packed-ternary-v1'); convert the bf16 dump first."
        )


def as_uint32(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.uint32 else t.view(torch.uint32)


def read_weights(model_dir, device, flash_head: bool = False) -> tuple[dict, dict]:
    """``(config, {name: tensor})`` of a checkpoint directory, tensors on
    ``device``; FlashHead tensors only when ``flash_head``."""
    from safetensors.torch import load_file

    model_dir = Path(model_dir).expanduser()
    config = json.loads((model_dir / "config.json").read_text())
    require_packed_format(config)
    index = model_dir / "model.safetensors.index.json"
    if index.exists():
        shards = sorted(set(json.loads(index.read_text())["weight_map"].values()))
    else:
        shards = sorted(p.name for p in model_dir.glob("*.safetensors"))
    weights: dict[str, torch.Tensor] = {}
    flash_shard = model_dir / "model-flashhead.safetensors"
    if flash_head and flash_shard.exists() and flash_shard.name not in shards:
        shards.append(flash_shard.name)
    for name in shards:
        if name == flash_shard.name and not flash_head:
            continue
        shard = load_file(str(model_dir / name), device=str(device))
        weights.update({k: v for k, v in shard.items() if flash_head or not k.startswith("lm_head_flash.")})
    return config, weights


def cat_qkv(weights: dict, prefix: str) -> tuple[torch.Tensor, torch.Tensor]:
    """``model.py:518-535``: q, k, v rows stacked in that order (popped)."""
    names = [f"{prefix}.self_attn.{p}_proj" for p in ("q", "k", "v")]
    packed = torch.cat([as_uint32(weights.pop(n + ".weight")) for n in names], dim=0)
    alpha = torch.cat([weights.pop(n + ".row_alpha") for n in names], dim=0)
    return packed, alpha


def cat_up_gate(weights: dict, prefix: str) -> tuple[torch.Tensor, torch.Tensor]:
    """``model.py:538-553``: per expert, the up rows then the gate rows (popped)."""
    names = [f"{prefix}.mlp.switch_mlp.{p}_proj" for p in ("up", "gate")]
    packed = torch.cat([as_uint32(weights.pop(n + ".weight")) for n in names], dim=1)
    alpha = torch.cat([weights.pop(n + ".row_alpha") for n in names], dim=1)
    return packed, alpha


def decoder_config(config: dict) -> DecoderConfig:
    """The ``DecoderConfig`` of a checkpoint config (keys of ``model.py:636-660``)."""
    layer_types = tuple(config.get("layer_types") or ())
    if any(t not in ("full_attention", "sliding_attention") for t in layer_types):
        raise NotImplementedError(f"layer types {sorted(set(layer_types))}: only full_attention "
                                  "and sliding_attention are supported")
    if layer_types and len(layer_types) != int(config["num_hidden_layers"]):
        raise ValueError("layer_types must name every layer")
    if not bool(config.get("use_qk_norm", True)):
        raise NotImplementedError("attention without QK-norm is not supported")
    if int(config["head_dim"]) not in (64, 128):
        raise NotImplementedError(f"head_dim {config['head_dim']}: the decode attention kernel is built "
                                  "for head_dim 64 and 128")
    meta = config.get("maple_run") or {}
    return DecoderConfig(
        hidden=int(config["hidden_size"]),
        layers=int(config["num_hidden_layers"]),
        heads=int(config["num_attention_heads"]),
        kv_heads=int(config["num_key_value_heads"]),
        head_dim=int(config["head_dim"]),
        experts=int(config["num_experts"]),
        inter=int(config["moe_intermediate_size"]),
        top_k=int(config["num_experts_per_tok"]),
        vocab=int(config["vocab_size"]),
        rtn_group=int((meta.get("rtn_4bit") or {}).get("group_size", HEAD_GROUP_SIZE)),
        rope_theta=float(config.get("rope_theta", 10000)),
        partial_rotary=float(config.get("partial_rotary_factor", 0.5)),
        eps=float(config.get("rms_norm_eps", 1e-6)),
        layer_types=layer_types,
        sliding_window=int(config.get("sliding_window", 512)),
        nope_on_global=bool(config.get("nope_on_global_attention", True)) and bool(layer_types),
    )


def load_decoder(model_dir, device="cuda", max_len: int = 4096 + 128, flash_head: bool = False,
                 **flags) -> SyntheticDecoder:
    """A decoder on the HIP kernels with a checkpoint's weights (``flags``:
    the ``SyntheticDecoder`` launch options; ``flash_head``: decode batch 1
    through the checkpoint's FlashHead)."""
    device = torch.device(device)
    config, w = read_weights(model_dir, device, flash_head)
    cfg = decoder_config(config)
    # model.py:728-748: float32 router rows and RTN scales/biases go to bf16;
    # row_alpha keeps the dtype it was written in (float32 from the converter)
    bf16 = lambda t: t.to(torch.bfloat16).contiguous()
    f32 = lambda t: t.to(torch.float32).contiguous()
    keep = lambda t: t.contiguous()
    for name in ("model.word_embeddings", "lm_head"):
        n_groups = int(w[name + ".scales"].shape[-1])
        if n_groups * cfg.rtn_group != cfg.hidden:
            raise ValueError(f"{name}: {n_groups} RTN scale groups per row do not cover hidden "
                             f"{cfg.hidden} with group_size {cfg.rtn_group}")
    layers = []
    for i in range(cfg.layers):
        p = f"model.layers.{i}"
        qkv, qkv_a = cat_qkv(w, p)
        up_gate, up_gate_a = cat_up_gate(w, p)
        moe = synthetic.MoELayer(
            gate_weight=bf16(w.pop(f"{p}.mlp.gate.weight")),
            up_gate_packed=up_gate.contiguous(),
            up_gate_alpha=keep(up_gate_a),
            down_packed=as_uint32(w.pop(f"{p}.mlp.switch_mlp.down_proj.weight")).contiguous(),
            down_alpha=keep(w.pop(f"{p}.mlp.switch_mlp.down_proj.row_alpha")),
        )
        layers.append(DecoderLayerWeights(
            qkv.contiguous(), keep(qkv_a),
            as_uint32(w.pop(f"{p}.self_attn.o_proj.weight")).contiguous(),
            keep(w.pop(f"{p}.self_attn.o_proj.row_alpha")),
            f32(w.pop(f"{p}.input_layernorm.weight")), f32(w.pop(f"{p}.post_attention_layernorm.weight")),
            f32(w.pop(f"{p}.self_attn.q_norm.weight")), f32(w.pop(f"{p}.self_attn.k_norm.weight")), moe))
    rtn = lambda n: (as_uint32(w.pop(n + ".weight")).contiguous(), bf16(w.pop(n + ".scales")),
                     bf16(w.pop(n + ".biases")))
    embed = rtn("model.word_embeddings")
    lm_head = rtn("lm_head")
    final_norm = f32(w.pop("model.norm.weight"))
    model = SyntheticDecoder.from_weights(cfg, device, layers, embed, lm_head, final_norm,
                                          max_len=max_len, **flags)
    if flash_head:
        from .flash_head import build_flash_head

        model.flash_head = build_flash_head(config=config, lm_head=lm_head, weights=w, device=device)
    return model


def save_decoder(model, model_dir) -> None:
    """Write a decoder's weights as a packed-ternary-v1 directory (one shard):
    the layout ``load_decoder`` and the reference's ``from_packed`` read."""
    from safetensors.torch import save_file

    c = model.cfg
    model_dir = Path(model_dir)
    model_dir.mkdir(parents=True, exist_ok=True)
    cpu = lambda t: t.detach().to("cpu").contiguous()
    codes = lambda t: cpu(t).view(torch.int32)
    f32 = lambda t: cpu(t).to(torch.float32)
    out: dict[str, torch.Tensor] = {}
    nq, nk = c.heads * c.head_dim, c.kv_heads * c.head_dim
    for i, L in enumerate(model.layers):
        p = f"model.layers.{i}"
        for name, r0, r1 in (("q", 0, nq), ("k", nq, nq + nk), ("v", nq + nk, nq + 2 * nk)):
            out[f"{p}.self_attn.{name}_proj.weight"] = codes(L.qkv[r0:r1])
            out[f"{p}.self_attn.{name}_proj.row_alpha"] = f32(L.qkv_alpha[r0:r1])
        out[f"{p}.self_attn.o_proj.weight"] = codes(L.o)
        out[f"{p}.self_attn.o_proj.row_alpha"] = f32(L.o_alpha)
        out[f"{p}.self_attn.q_norm.weight"] = f32(L.q_norm)
        out[f"{p}.self_attn.k_norm.weight"] = f32(L.k_norm)
        out[f"{p}.input_layernorm.weight"] = f32(L.input_ln)
        out[f"{p}.post_attention_layernorm.weight"] = f32(L.post_ln)
        m, inter = L.moe, L.moe.inter
        out[f"{p}.mlp.gate.weight"] = f32(m.gate_weight)
        out[f"{p}.mlp.switch_mlp.up_proj.weight"] = codes(m.up_gate_packed[:, :inter])
        out[f"{p}.mlp.switch_mlp.gate_proj.weight"] = codes(m.up_gate_packed[:, inter:])
        out[f"{p}.mlp.switch_mlp.up_proj.row_alpha"] = f32(m.up_gate_alpha[:, :inter])
        out[f"{p}.mlp.switch_mlp.gate_proj.row_alpha"] = f32(m.up_gate_alpha[:, inter:])
        out[f"{p}.mlp.switch_mlp.down_proj.weight"] = codes(m.down_packed)
        out[f"{p}.mlp.switch_mlp.down_proj.row_alpha"] = f32(m.down_alpha)
    for name, (wt, sc, bs) in (("model.word_embeddings", model.embed), ("lm_head", model.lm_head)):
        out[f"{name}.weight"] = codes(wt)
        out[f"{name}.scales"] = f32(sc)
        out[f"{name}.biases"] = f32(bs)
    out["model.norm.weight"] = f32(model.final_norm)
    save_file(out, str(model_dir / "model.safetensors"))
    config = {
        "model_type": "maple", "hidden_size": c.hidden, "num_hidden_layers": c.layers,
        "num_attention_heads": c.heads, "num_key_value_heads": c.kv_heads, "head_dim": c.head_dim,
        "num_experts": c.experts, "num_experts_per_tok": c.top_k, "moe_intermediate_size": c.inter,
        "vocab_size": c.vocab, "rms_norm_eps": c.eps, "rope_theta": c.rope_theta,
        "partial_rotary_factor": c.partial_rotary,
        "layer_types": list(c.layer_types) or ["full_attention"] * c.layers,
        "sliding_window": c.sliding_window, "use_qk_norm": True, "nope_on_global_attention": c.nope_on_global,
        "maple_run": {
            "format": FORMAT, "experts": "stacked_switch_mlp",
            "expert_template": "model.layers.{layer}.mlp.switch_mlp.{proj}.weight",
            "ternary": {"bits": 2, "pack": "uint32_lsb_first", "scale": "row_alpha"},
            "rtn_4bit": {"bits": 4, "group_size": c.rtn_group, "mode": "affine", "pack": "uint32_lsb_first"},
        },
    }
    (model_dir / "config.json").write_text(json.dumps(config, indent=2, sort_keys=True))
