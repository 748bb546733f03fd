"""Seeded synthetic weights and activations for the packed-ternary MoE workloads.

Distributions (one seed per tensor):

* ternary codes iid uniform over {0, 1, 2} (values {-1, 0, +1}), packed 16 per
  uint32 LSB first (reference ``src/maple_run/pack.py:17-45``);
* per-row scales ``alpha ~ U(0.01, 0.05)`` in bf16;
* router weight ``~ N(0, 0.02)`` in bf16, activations ``~ N(0, 1)`` in bf16;
* the optional router bias that skews expert load towards a Zipf(s) law.

Everything is generated on the target device with ``torch.Generator`` so the
full-size layers (about 200 MB of codes per MoE layer) are cheap to build.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def pack_codes(codes: torch.Tensor) -> torch.Tensor:
    """Pack int codes ``[..., K]`` in [0, 4) to uint32 ``[..., K/16]``, LSB first."""
    *lead, k = codes.shape
    c = codes.reshape(*lead, k // 16, 16).to(torch.int64)
    shifts = torch.arange(0, 32, 2, device=codes.device, dtype=torch.int64)
    words = (c << shifts).sum(dim=-1)
    return words.to(torch.int32).view(torch.uint32)


def pack_codes4(codes: torch.Tensor) -> torch.Tensor:
    """Pack int codes ``[..., K]`` in [0, 16) to uint32 ``[..., K/8]``, LSB first."""
    *lead, k = codes.shape
    c = codes.reshape(*lead, k // 8, 8).to(torch.int64)
    shifts = torch.arange(0, 32, 4, device=codes.device, dtype=torch.int64)
    words = (c << shifts).sum(dim=-1)
    return words.to(torch.int32).view(torch.uint32)


def ternary_packed(shape, seed: int, device, chunk_rows: int = 4096) -> torch.Tensor:
    """iid U{0,1,2} codes of ``shape = (..., N, K)`` packed to ``(..., N, K/16)``."""
    *lead, n, k = shape
    g = _gen(seed, device)
    rows = int(math.prod(lead)) * n
    out = torch.empty(rows, k // 16, device=device, dtype=torch.int32)
    for r0 in range(0, rows, chunk_rows):
        r1 = min(rows, r0 + chunk_rows)
        codes = torch.randint(0, 3, (r1 - r0, k), generator=g, device=device, dtype=torch.int32)
        out[r0:r1] = pack_codes(codes).view(torch.int32)
    return out.view(torch.uint32).reshape(*lead, n, k // 16)


def uniform_bf16(shape, lo: float, hi: float, seed: int, device) -> torch.Tensor:
    g = _gen(seed, device)
    return (torch.rand(shape, generator=g, device=device) * (hi - lo) + lo).to(torch.bfloat16)


def randn_bf16(shape, seed: int, device, std: float = 1.0) -> torch.Tensor:
    g = _gen(seed, device)
    return (torch.randn(shape, generator=g, device=device) * std).to(torch.bfloat16)


@dataclass
class MoELayer:
    """One MoE FFN: router, stacked ``[up; gate]`` experts and down experts."""

    gate_weight: torch.Tensor       # bf16 [E, H]
    up_gate_packed: torch.Tensor    # uint32 [E, 2I, H/16], rows [up; gate]
    up_gate_alpha: torch.Tensor     # bf16 [E, 2I]
    down_packed: torch.Tensor       # uint32 [E, H, I/16]
    down_alpha: torch.Tensor        # bf16 [E, H]
    router_bias: torch.Tensor | None = None  # float32 [E] or None

    @property
    def n_experts(self) -> int:
        return int(self.gate_weight.shape[0])

    @property
    def hidden(self) -> int:
        return int(self.gate_weight.shape[1])

    @property
    def inter(self) -> int:
        return int(self.up_gate_packed.shape[1] // 2)

    def expert_bytes(self) -> int:
        """Packed codes + alphas of one expert (bytes)."""
        e = self.n_experts
        return (self.up_gate_packed.numel() + self.down_packed.numel()) * 4 // e + (
            self.up_gate_alpha.numel() + self.down_alpha.numel()) * 2 // e


def make_moe_layer(hidden: int = 2048, n_experts: int = 64, inter: int = 768, seed: int = 0,
                   device="cuda", router_std: float = 0.02) -> MoELayer:
    s = int(seed) * 16
    return MoELayer(
        gate_weight=randn_bf16((n_experts, hidden), s + 1, device, std=router_std),
        up_gate_packed=ternary_packed((n_experts, 2 * inter, hidden), s + 2, device),
        up_gate_alpha=uniform_bf16((n_experts, 2 * inter), 0.01, 0.05, s + 3, device),
        down_packed=ternary_packed((n_experts, hidden, inter), s + 4, device),
        down_alpha=uniform_bf16((n_experts, hidden), 0.01, 0.05, s + 5, device),
    )


def zipf_router_bias(n_experts: int, s: float = 1.1, gamma: float = 1.0, seed: int = 0) -> torch.Tensor:
    """Logit bias ``b_e = gamma * log p_{pi(e)}`` with ``p_r ~ r^-s`` over ranks
    1..E and ``pi`` a seeded permutation (float32, CPU)."""
    g = torch.Generator().manual_seed(int(seed))
    perm = torch.randperm(n_experts, generator=g)
    ranks = torch.arange(1, n_experts + 1, dtype=torch.float64)
    p = ranks ** (-s)
    p = p / p.sum()
    return (gamma * torch.log(p[perm])).to(torch.float32)


def ternary_linear(n_out: int, k_in: int, seed: int, device):
    """``(packed [N, K/16] uint32, alpha [N] bf16)`` with the synthetic distributions."""
    return (
        ternary_packed((n_out, k_in), seed * 2 + 1, device),
        uniform_bf16((n_out,), 0.01, 0.05, seed * 2 + 2, device),
    )


def rtn4_table(n_out: int, k_in: int, group: int, seed: int, device, scale_lo: float = 0.002,
               scale_hi: float = 0.004):
    """4-bit RTN table: codes iid U{0..15}, ``scale ~ U(lo, hi)``, ``bias = -7.5 * scale``
    (zero-centred dequantised weights), scales/biases bf16 ``[N, K/group]``."""
    g = _gen(seed, device)
    words = torch.empty(n_out, k_in // 8, device=device, dtype=torch.int32)
    for r0 in range(0, n_out, 8192):
        r1 = min(n_out, r0 + 8192)
        codes = torch.randint(0, 16, (r1 - r0, k_in), generator=g, device=device, dtype=torch.int32)
        words[r0:r1] = pack_codes4(codes).view(torch.int32)
    sc = torch.rand((n_out, k_in // group), generator=g, device=device) * (scale_hi - scale_lo) + scale_lo
    sc = sc.to(torch.bfloat16)
    bs = (-7.5 * sc.float()).to(torch.bfloat16)
    return words.view(torch.uint32), sc, bs


def to_numpy_u32(t: torch.Tensor):
    """uint32 tensor -> NumPy uint32 array (via an int32 view)."""
    import numpy as np

    return t.view(torch.int32).cpu().numpy().view(np.uint32)


def flash_head_for(lm_head: tuple, n_clusters: int, n_probes: int, seed: int, device, force=()):
    """A FlashHead over ``lm_head`` with synthetic cluster data: a seeded token
    permutation split into ``n_clusters`` equal clusters and random RTN4
    centroid rows (group 64).  For timing the FlashHead path; real clusters
    come from the converter's k-means."""
    from .flash_head import FlashHead

    w, sc, bs = lm_head
    vocab, nwords = int(w.shape[0]), int(w.shape[1])
    if vocab % n_clusters:
        raise ValueError(f"{n_clusters} clusters do not divide the vocabulary ({vocab}).")
    g = _gen(seed, device)
    tm = torch.randperm(vocab, generator=g, device=device).to(torch.int32).reshape(n_clusters, -1)
    cw, cs, cb = rtn4_table(n_clusters, nwords * 8, 64, seed + 1, device)
    order = tm.reshape(-1).to(torch.int64)
    fid = torch.tensor(list(force), device=device, dtype=torch.int64)
    rows = lambda t: t.view(torch.int32).index_select(0, fid).view(torch.uint32)  # noqa: E731
    return FlashHead(
        centroids_weight=cw, centroids_scales=cs, centroids_biases=cb, token_map=tm,
        head_weight=w.view(torch.int32).index_select(0, order).view(torch.uint32).reshape(n_clusters, -1, nwords),
        head_scales=sc.index_select(0, order).reshape(n_clusters, vocab // n_clusters, -1),
        head_biases=bs.index_select(0, order).reshape(n_clusters, vocab // n_clusters, -1),
        force_ids=fid, force_weight=rows(w) if len(force) else None,
        force_scales=sc.index_select(0, fid) if len(force) else None,
        force_biases=bs.index_select(0, fid) if len(force) else None,
        n_probes=n_probes, vocab_size=vocab, group_size=int(nwords * 8 // sc.shape[1]), device=device,
        centroid_group_size=64)
