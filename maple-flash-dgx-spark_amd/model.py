"""Synthetic packed decoder on the HIP kernels (decode path of reference
``src/maple_run/model.py``: ``MapleDecoderLayer`` :477-506,
``MapleForCausalLM.forward`` :848-886, ``KVCache`` :116-310).

One decode step, per layer:
  qkv   = ternary_gemv(hidden, W_qkv, rms_weight=input_ln)     (fused RMSNorm)
  attn  = decode_attention(qkv, ...)    QK-norm + RoPE, K/V written at seqlen,
                                        GQA over the cache (one launch)
  o     = ternary_gemv(attn, W_o)
  hidden, mlp_in = add_rms_norm(hidden, o, post_ln)
  hidden = moe_block(mlp_in, residual=hidden)
  (at batch 1, when the one-launch MoE kernel is built for the shape and
  fused_moe is left True, the last two lines are one launch:
  moe_fused(hidden, add=o, norm_weight=post_ln), which in forward() also
  computes the next layer's qkv line from its output, so only layer 0 runs
  the standalone QKV projection; from 17 tokens, with combine_next left True,
  the grouped MoE's top-k combine is left to the next layer's QKV projection,
  which builds hidden from the slot outputs in its operand launch)
then seqlen += 1, final rms_norm, RTN4 lm_head, greedy argmax.

Weights are random with the synthetic distributions (``synthetic.py``): every
projection packed ternary, norm weights 1, the lm_head and embedding 4-bit RTN
with group 128 and zero-centred dequantised values, RoPE on every layer over
half the head (rotary_dim 32, theta 1e4), full attention (no window).
"""

from __future__ import annotations

import dataclasses
from dataclasses import dataclass, field

import torch

from . import synthetic
from .kernels.decode_attn import decode_attention, gqa_workspace, o_projection_supported
from .kernels.fused_norm import rms_norm
from .kernels.greedy import greedy_argmax
from .kernels.rtn4 import rtn4_embedding, rtn4_gemv
from .kernels.ternary_gemv import combine_gemv_supported, ternary_gemv, ternary_gemv_combine
from .moe import PendingCombine, fused_form, fused_supported, moe_fused, moe_layer


@dataclass
class DecoderConfig:
    hidden: int = 2048
    layers: int = 24
    heads: int = 32
    kv_heads: int = 4
    head_dim: int = 64
    experts: int = 64
    inter: int = 768
    top_k: int = 8
    vocab: int = 151936
    rtn_group: int = 128
    rope_theta: float = 10000.0
    partial_rotary: float = 0.5
    eps: float = 1e-6
    lm_scale: tuple = (0.003, 0.006)
    # per-layer attention (model.py:646-649, 784-786): "full_attention" or
    # "sliding_attention" (the last sliding_window positions); empty = all full.
    # nope_on_global: full-attention layers skip RoPE.
    layer_types: tuple = ()
    sliding_window: int = 512
    nope_on_global: bool = False

    def layer_attention(self, i: int) -> tuple:
        """``(window or None, use_rope)`` of layer ``i``."""
        kind = self.layer_types[i] if self.layer_types else "full_attention"
        window = self.sliding_window if kind == "sliding_attention" else None
        return window, not (self.nope_on_global and kind == "full_attention")

    @property
    def qkv_rows(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim

    @property
    def rotary_dim(self) -> int:
        return int(self.head_dim * self.partial_rotary)


@dataclass
class DecoderLayerWeights:
    qkv: torch.Tensor
    qkv_alpha: torch.Tensor
    o: torch.Tensor
    o_alpha: torch.Tensor
    input_ln: torch.Tensor
    post_ln: torch.Tensor
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    moe: synthetic.MoELayer


def rope_tables(max_len: int, rotary_dim: int, theta: float, device):
    """float32 cos/sin ``[max_len, rotary_dim]`` built like ``model.py:66-92``
    (``inv_freq = theta^(-2i/rot)``, ``emb = cat(freqs, freqs)``)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, rotary_dim, 2, device=device, dtype=torch.float32) / rotary_dim))
    t = torch.arange(max_len, device=device, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().contiguous(), emb.sin().contiguous()


@dataclass
class KVCache:
    """Preallocated bf16 K/V per layer ``[rows, n_kv, max_len, D]``, one write
    position per slot (``model.py:116-143``) and the attention workspace
    (zeroed once; the kernels leave its barrier counters zero).

    Slots and cache rows (``model.py:145-156, 196-214``): ``seqlen`` is
    indexed by slot, K/V by cache row, and ``row_map[slot]`` names the row.
    With ``remap`` off the map is the identity; a scheduler turns it on to
    keep live sequences in the low slots by swapping indices (never K/V), so
    a decode step can run at a narrow width.  A step of width ``w`` covers
    slots ``[0, w)``."""

    k: list
    v: list
    seqlen: torch.Tensor
    max_len: int
    attn_ws: torch.Tensor = field(default=None)
    row_map: torch.Tensor = field(default=None)
    remap: bool = False

    def __post_init__(self):
        if self.row_map is None:
            self.row_map = torch.arange(self.rows, device=self.seqlen.device, dtype=torch.int64)

    @property
    def rows(self) -> int:
        return int(self.k[0].shape[0])

    def slot_rows(self, width: int):
        """``(seqlen, row_map)`` views for a step over slots ``[0, width)``;
        ``row_map`` is None when the kernels may read row == slot."""
        if not 0 < width <= self.rows:
            raise ValueError(f"step width {width} outside the cache's {self.rows} slots.")
        rm = self.row_map[:width] if (self.remap or width != self.rows) else None
        return self.seqlen[:width], rm

    def swap_slots(self, i: int, j: int) -> None:
        """Exchange two slots: their row map entries and write positions."""
        if i == j:
            return
        if not self.remap:
            raise RuntimeError("swap_slots needs cache.remap: without the map the kernels read "
                               "cache row == slot, and a swap would read another sequence's K/V.")
        for t in (self.row_map, self.seqlen):
            a = t[i].clone()
            t[i] = t[j]
            t[j] = a

    def reset_slot(self, slot: int) -> None:
        """Forget a slot's history so a new sequence can take it."""
        self.seqlen[slot] = 0

    def snapshot(self, steps: int | None = None) -> dict:
        """Write positions, slot map and a copy of the K/V that the next
        ``steps`` decode steps can overwrite (all of it when ``steps`` is
        None); ``restore`` puts them back (``model.py:276-291``)."""
        lo, hi = 0, self.max_len
        if steps is not None:
            sl = self.seqlen.cpu()
            lo = int(sl.min()) if sl.numel() else 0
            hi = min(self.max_len, int(sl.max()) + int(steps) + 1) if sl.numel() else 0
        return {"seqlen": self.seqlen.clone(), "row_map": self.row_map.clone(), "remap": self.remap,
                "span": (lo, hi), "k": [t[:, :, lo:hi].clone() for t in self.k],
                "v": [t[:, :, lo:hi].clone() for t in self.v]}

    def restore(self, snap: dict) -> None:
        self.seqlen.copy_(snap["seqlen"])
        self.row_map.copy_(snap["row_map"])
        self.remap = snap["remap"]
        lo, hi = snap["span"]
        for dst, src in zip(self.k, snap["k"]):
            dst[:, :, lo:hi].copy_(src)
        for dst, src in zip(self.v, snap["v"]):
            dst[:, :, lo:hi].copy_(src)


class SyntheticDecoder:
    def __init__(self, cfg: DecoderConfig, device, seed: int = 0, max_len: int = 4096 + 128,
                 fused_moe: bool = True, fused_o: bool = False, combine_next: bool = True,
                 o_in_moe: bool = False, prefetch_router: bool = True):
        self.cfg = cfg
        self.prefetch_router = prefetch_router
        self.fused_moe = fused_moe
        self.combine_next = combine_next
        self.fused_o = fused_o
        self.o_in_moe = o_in_moe
        self.device = torch.device(device)
        self.max_len = max_len
        c, dev, s = cfg, self.device, seed * 1000
        ones = lambda n: torch.ones(n, device=dev, dtype=torch.float32)
        self.layers = []
        for i in range(c.layers):
            qkv, qkv_a = synthetic.ternary_linear(c.qkv_rows, c.hidden, s + 10 * i + 1, dev)
            o, o_a = synthetic.ternary_linear(c.hidden, c.heads * c.head_dim, s + 10 * i + 2, dev)
            moe = synthetic.make_moe_layer(c.hidden, c.experts, c.inter, seed=s + 10 * i + 3, device=dev)
            self.layers.append(DecoderLayerWeights(qkv, qkv_a, o, o_a, ones(c.hidden), ones(c.hidden),
                                                   ones(c.head_dim), ones(c.head_dim), moe))
        lo, hi = c.lm_scale
        self.lm_head = synthetic.rtn4_table(c.vocab, c.hidden, c.rtn_group, s + 901, dev, lo, hi)
        self.embed = synthetic.rtn4_table(c.vocab, c.hidden, c.rtn_group, s + 902, dev, lo, hi)
        self.final_norm = ones(c.hidden)
        self.cos, self.sin = rope_tables(max_len, c.rotary_dim, c.rope_theta, dev)
        self.flash_head = None
        self._pack_read_ahead()

    @classmethod
    def from_weights(cls, cfg: DecoderConfig, device, layers: list, embed: tuple, lm_head: tuple,
                     final_norm: torch.Tensor, max_len: int = 4096 + 128, fused_moe: bool = True,
                     fused_o: bool = False, combine_next: bool = True,
                     o_in_moe: bool = False, prefetch_router: bool = True) -> "SyntheticDecoder":
        """A decoder over given weights (``checkpoint.load_decoder``) instead of
        the seeded synthetic ones."""
        self = cls.__new__(cls)
        self.cfg = cfg
        self.fused_moe, self.fused_o, self.combine_next = fused_moe, fused_o, combine_next
        self.o_in_moe = o_in_moe
        self.prefetch_router = prefetch_router
        self.device = torch.device(device)
        self.max_len = max_len
        self.layers = list(layers)
        self.embed, self.lm_head, self.final_norm = embed, lm_head, final_norm
        self.cos, self.sin = rope_tables(max_len, cfg.rotary_dim, cfg.rope_theta, self.device)
        self.flash_head = None
        self._pack_read_ahead()
        return self

    def _pack_read_ahead(self) -> None:
        """Lay out each layer's post-attention norm weights, QK-norm weights
        and router rows in one buffer (in that order, 256-byte aligned; the
        layer's tensors become views of it), which the previous layer's
        one-launch MoE kernel reads ahead into every XCD's L2 while it waits
        on its own hand-offs: bytes that are read at the start of the layer's
        launches and would otherwise come cold from HBM (the small ones first,
        so that a router larger than the read-ahead still leaves them in)."""
        self.read_ahead = []
        for i, L in enumerate(self.layers):
            parts = [L.post_ln, L.q_norm, L.k_norm, L.moe.gate_weight]
            offs, n = [], 0
            for t in parts:
                offs.append(n)
                n += -(-t.numel() * t.element_size() // 256) * 256
            buf = torch.empty(n, dtype=torch.uint8, device=L.post_ln.device)
            views = []
            for t, o in zip(parts, offs):
                v = buf[o:o + t.numel() * t.element_size()].view(t.dtype).view(t.shape)
                v.copy_(t)
                views.append(v)
            moe = dataclasses.replace(L.moe, gate_weight=views[3])
            self.layers[i] = dataclasses.replace(L, post_ln=views[0], q_norm=views[1], k_norm=views[2], moe=moe)
            self.read_ahead.append(buf)

    def make_cache(self, batch: int, prefill_len: int, seed: int = 0) -> KVCache:
        """Cache rows filled with seeded N(0, 1) bf16 K/V for ``prefill_len``
        positions; decoding then writes at ``prefill_len``."""
        c = self.cfg
        shape = (batch, c.kv_heads, self.max_len, c.head_dim)
        ks, vs = [], []
        for i in range(c.layers):
            k = synthetic.randn_bf16(shape, 50_000 + seed * 97 + 2 * i, self.device)
            v = synthetic.randn_bf16(shape, 50_001 + seed * 97 + 2 * i, self.device)
            k[:, :, prefill_len:] = 0
            v[:, :, prefill_len:] = 0
            ks.append(k)
            vs.append(v)
        seqlen = torch.full((batch,), prefill_len, device=self.device, dtype=torch.int64)
        ws = gqa_workspace(batch, c.kv_heads, self.max_len, self.device, c.head_dim)
        return KVCache(ks, vs, seqlen, self.max_len, ws)

    def _layer(self, i: int, hidden: torch.Tensor, cache: KVCache, routing=None,
               qkv: torch.Tensor | None = None, fuse_next: bool = True):
        """Layer ``i``; returns ``(y, next_qkv)``.  ``qkv``: this layer's input
        projection if an earlier launch already computed it.  ``next_qkv`` is
        layer ``i + 1``'s projection when the one-launch MoE kernel computed it
        from ``y`` (batch 1, ``fuse_next``), else None.  ``y`` is a
        ``PendingCombine`` where layer ``i + 1``'s QKV launch runs the MoE
        combine (``combine_next``, 17+ tokens); ``hidden`` may be one."""
        c, L = self.cfg, self.layers[i]
        if isinstance(hidden, PendingCombine):  # the previous layer's MoE combine runs here
            hidden, qkv = ternary_gemv_combine(hidden, L.qkv, L.qkv_alpha, rms_weight=L.input_ln,
                                               rms_eps=c.eps)
        bsz = hidden.shape[0]
        if qkv is None:
            qkv = ternary_gemv(hidden, L.qkv, L.qkv_alpha, rms_weight=L.input_ln, rms_eps=c.eps)
        window, use_rope = c.layer_attention(i)
        akw = dict(num_heads=c.heads, num_kv_heads=c.kv_heads, head_dim=c.head_dim,
                   rotary_dim=c.rotary_dim, eps=c.eps, scale=c.head_dim ** -0.5, window=window,
                   use_rope=use_rope)
        seqlen, row_map = cache.slot_rows(bsz)
        akw["row_map"] = row_map
        if bsz == 1 and self.fused_o and o_projection_supported(1, c.heads, c.kv_heads, c.head_dim,
                                                                cache.max_len, window, c.hidden):
            # attention and its output projection in one launch (measured: no
            # faster than two launches at 4096 positions -- the grid barrier
            # and the tail cost what the second launch does -- so off by default)
            _, o = decode_attention(qkv, L.q_norm, L.k_norm, self.cos, self.sin, cache.k[i], cache.v[i],
                                    seqlen, cache.attn_ws, o_linear=(L.o, L.o_alpha), **akw)
        else:
            attn = decode_attention(qkv, L.q_norm, L.k_norm, self.cos, self.sin, cache.k[i], cache.v[i],
                                    seqlen, cache.attn_ws, **akw)
            # o_in_moe: at batch 1 the XCD-split MoE launch computes the output
            # projection itself (same bits; measured 1,294 against 1,306 tok/s
            # with the separate launch, so off by default)
            o_moe = (bsz == 1 and self.o_in_moe and self.fused_moe and fused_supported(L.moe, c.top_k, hidden)
                     and fused_form(L.moe, c.top_k) == 1 and c.heads * c.head_dim == c.hidden
                     and L.o_alpha.dtype == L.moe.up_gate_alpha.dtype)
            o = None if o_moe else ternary_gemv(attn.reshape(bsz, -1), L.o, L.o_alpha)
        next_qkv = None
        if bsz == 1 and self.fused_moe and fused_supported(L.moe, c.top_k, hidden):
            # add + RMSNorm + router + experts + combine (+ the next layer's
            # RMS-folded QKV projection) in one launch
            nl = None
            if fuse_next and i + 1 < c.layers and self.layers[i + 1].qkv_alpha.dtype == L.moe.up_gate_alpha.dtype:
                n = self.layers[i + 1]
                nl = (n.qkv, n.qkv_alpha, n.input_ln, c.eps)
            # the next layer's norm weights and router rows are read ahead
            # into the caches while this launch waits for h
            pf = self.read_ahead[i + 1] if self.prefetch_router and i + 1 < c.layers else None
            out = moe_fused(hidden, L.moe, c.top_k, add=o, norm_weight=L.post_ln, eps=c.eps,
                            next_linear=nl,
                            o_linear=None if o is not None else (attn.reshape(1, -1), L.o, L.o_alpha),
                            prefetch=pf)
            y, ids = out[0], out[1]
            if nl is not None:
                next_qkv = out[3]
        else:
            # add + RMSNorm + router + dispatch in one launch from 4 tokens,
            # then the grouped experts
            defer = (self.combine_next and fuse_next and i + 1 < c.layers
                     and combine_gemv_supported(bsz, c.top_k, self.layers[i + 1].qkv))
            y, ids = moe_layer(hidden, L.moe, c.top_k, L.post_ln, c.eps, add=o.reshape(hidden.shape),
                               defer_combine=defer)
        if routing is not None:
            routing.append(ids)
        return y, next_qkv

    def layer_step(self, i: int, hidden: torch.Tensor, cache: KVCache, routing=None) -> torch.Tensor:
        """Layer ``i`` on its own (its QKV projection computed here)."""
        return self._layer(i, hidden, cache, routing, fuse_next=False)[0]

    def forward(self, input_ids: torch.Tensor, cache: KVCache, routing: list | None = None) -> torch.Tensor:
        """One decode step for ``input_ids [w]`` over cache slots ``[0, w)``;
        returns bf16 logits ``[w, vocab]``.  ``routing``, if a list, receives
        each layer's expert ids."""
        width = int(input_ids.numel())
        cache.slot_rows(width)
        hidden = self.embed_tokens(input_ids.reshape(-1))
        qkv = None
        for i in range(self.cfg.layers):
            hidden, qkv = self._layer(i, hidden, cache, routing, qkv)
        cache.seqlen[:width].add_(1)
        return self.head(hidden)

    def embed_tokens(self, input_ids: torch.Tensor) -> torch.Tensor:
        w, sc, bs = self.embed
        return rtn4_embedding(input_ids, w, sc, bs, group_size=self.cfg.rtn_group).to(torch.bfloat16)

    def head(self, hidden: torch.Tensor) -> torch.Tensor:
        """Final RMSNorm and the RTN4 lm_head: bf16 logits ``[B, vocab]``
        (at batch 1 through the FlashHead when one is attached: -inf outside
        the probed clusters and forced tokens, model.py:874-886)."""
        hidden = rms_norm(hidden, self.final_norm, self.cfg.eps)
        if self.flash_head is not None and hidden.shape[0] == 1:
            return self.flash_head(hidden).reshape(1, -1)
        w, sc, bs = self.lm_head
        return rtn4_gemv(hidden, w, sc, bs, group_size=self.cfg.rtn_group)

    def greedy_step(self, ids: torch.Tensor, cache: KVCache) -> torch.Tensor:
        """forward + argmax, writing the next ids back into ``ids`` (graph-safe)."""
        logits = self.forward(ids, cache)
        greedy_argmax(logits, out=ids)
        return logits

    def decode_bytes(self, batch: int, kv_len: int) -> int:
        """Algorithmic HBM bytes of one decode step: weights touched once; the
        experts a step touches counted as the expected number of distinct
        experts among ``batch`` rows of top-k picks under uniform routing,
        E (1 - (1 - k/E)^batch) (k at batch 1, all E at large batches); the
        KV read for every row over the positions each layer attends (the last
        ``sliding_window`` on sliding layers)."""
        c = self.cfg
        lay = (c.qkv_rows + c.hidden) * c.hidden // 4 + (c.qkv_rows + c.hidden) * 2
        router = c.experts * c.hidden * 2
        expert = (3 * c.inter * c.hidden) // 4 + (2 * c.inter + c.hidden) * 2
        hit = c.experts * (1.0 - (1.0 - c.top_k / c.experts) ** batch)
        experts = int(round(hit * expert))
        kv = 0
        for i in range(c.layers):
            window, _ = c.layer_attention(i)
            span = min(kv_len, window) if window else kv_len
            kv += batch * 2 * c.kv_heads * span * c.head_dim * 2
        head = c.vocab * c.hidden // 2 + 2 * c.vocab * (c.hidden // c.rtn_group) * 2
        return c.layers * (lay + router + experts) + kv + head
