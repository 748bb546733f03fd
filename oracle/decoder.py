"""Synthetic decoder step, NumPy (test infrastructure only).

Restates the decode path of reference ``src/maple_run/model.py``
(``MapleAttention`` decode branch :368-414, ``MapleDecoderLayer`` :477-506,
``MapleForCausalLM.forward`` :848-886) and of
``src/maple_run/kernels/decode_attn.py`` (QK RMSNorm + partial rotate-half
RoPE :15-163, GQA :166-359).  Values are float64; every tensor the reference
stores in bf16 is rounded with ``bf16_round`` at the same point.
"""

from __future__ import annotations

import numpy as np

from . import kernels as ok

bf = lambda a: ok.bf16_round(a).astype(np.float64)  # noqa: E731


def rope_tables(max_len: int, rotary_dim: int, theta: float):
    """float32 cos/sin ``[max_len, rotary_dim]`` (``model.py:66-92``)."""
    inv_freq = (1.0 / (np.float32(theta) ** (np.arange(0, rotary_dim, 2, dtype=np.float32)
                                             / np.float32(rotary_dim)))).astype(np.float32)
    t = np.arange(max_len, dtype=np.float32)
    freqs = np.outer(t, inv_freq).astype(np.float32)
    emb = np.concatenate([freqs, freqs], axis=-1)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


def head_norm_rope(x, w, cos_row, sin_row, rotary_dim, eps, use_rope=True):
    """RMSNorm one head, then rotate-half RoPE on its first ``rotary_dim`` dims
    (``decode_attn.py:29-60``); cos/sin already rounded to bf16."""
    x = np.asarray(x, np.float64)
    y = x / np.sqrt(np.mean(x * x) + eps) * np.asarray(w, np.float64)
    if use_rope and rotary_dim:
        half = rotary_dim // 2
        lo, hi = y[:half].copy(), y[half:rotary_dim].copy()
        y[:half] = lo * cos_row[:half] - hi * sin_row[:half]
        y[half:rotary_dim] = hi * cos_row[half:rotary_dim] + lo * sin_row[half:rotary_dim]
    return y


def gqa(q, k_cache, v_cache, kv_len, scale, window=None):
    """Attention of one row's query heads over positions [start, kv_len)
    (``decode_attn.py:236-289``): scores ``K q * scale``, ``p = exp(s - max)``,
    the sum ``l`` over the unrounded ``p``, and ``P`` rounded to bf16 (the
    cache dtype) before ``P V`` (``:282-289``); output ``(bf16(P) V) / l``.
    The reference takes the max per tile of positions as it streams (running
    max); here it is the max over all positions, the same thing when every
    position sits in one tile, and otherwise a different bf16 rounding point
    of P (relative error 2^-9 of a term either way)."""
    nq, d = q.shape
    nkv = k_cache.shape[0]
    group = nq // nkv
    start = max(0, kv_len - window) if window else 0
    out = np.zeros((nq, d))
    for h in range(nq):
        K = np.asarray(k_cache[h // group, start:kv_len], np.float64)
        V = np.asarray(v_cache[h // group, start:kv_len], np.float64)
        s = K @ q[h] * scale
        p = np.exp(s - s.max())
        out[h] = (bf(p) @ V) / p.sum()
    return out


def attend_row(qkv_row, L: dict, c: dict, k_rows, v_rows, pos: int):
    """The attention of one batch row at position ``pos`` (``model.py:368-414``
    decode branch, ``decode_attn.py:15-163,166-359``): the ``[q; k; v]`` row
    split into heads; q and the new k RMS-normalised per head and roped
    (rotate-half over the first ``rotary_dim`` dims, skipped on NoPE layers);
    the new k and v written at ``pos`` of this row's cache ``k_rows`` /
    ``v_rows`` ``[n_kv, max_len, D]``; GQA over positions up to ``pos`` at
    scale ``head_dim ** -0.5`` (``model.py:343``).  Returns the attention
    output ``[heads * head_dim]`` in float64 (not yet rounded)."""
    nq, nkv, d = c["heads"], c["kv_heads"], c["head_dim"]
    rot, eps = c["rotary_dim"], c["eps"]
    use_rope = L.get("use_rope", True)
    cs = bf(c["cos"][pos]) if rot else None
    sn = bf(c["sin"][pos]) if rot else None
    q = np.stack([bf(head_norm_rope(qkv_row[hh * d:(hh + 1) * d], L["q_norm"], cs, sn, rot, eps, use_rope=use_rope))
                  for hh in range(nq)])
    for kh in range(nkv):
        o0 = (nq + kh) * d
        k_rows[kh, pos] = bf(head_norm_rope(qkv_row[o0:o0 + d], L["k_norm"], cs, sn, rot, eps, use_rope=use_rope))
        o1 = (nq + nkv + kh) * d
        v_rows[kh, pos] = qkv_row[o1:o1 + d]
    kv_len = min(pos + 1, k_rows.shape[1])
    return gqa(q, k_rows, v_rows, kv_len, d ** -0.5, window=L.get("window")).reshape(-1)


def decoder_layer(L: dict, c: dict, h, cache: dict, i: int, *, router_ids=None):
    """One decoder layer on bf16 hidden ``h [B, hidden]`` (``model.py:477-506``):
    fused-RMS QKV, QK-norm + RoPE with the K/V write at ``seqlen``, GQA, O
    projection, add + RMSNorm, then the MoE block with the residual.
    ``router_ids``: optional expert ids ``[B, k]`` to use instead of the
    oracle's own top-k (top-k is discontinuous, so two paths that differ by
    rounding can pick different near-tied experts and then diverge); the
    weights are still the oracle's own probabilities of those experts,
    renormalised.  ``L`` may carry ``window`` (sliding-window attention over
    the last ``window`` positions, model.py:784-786) and ``use_rope`` (False
    on NoPE layers).  Returns ``(h_out, (own ids, probs))``."""
    nq, nkv, d = c["heads"], c["kv_heads"], c["head_dim"]
    rot, eps = c["rotary_dim"], c["eps"]
    bsz = h.shape[0]
    qkv = bf(ok.ternary_gemv(h, L["qkv"], L["qkv_alpha"], rms_weight=L["input_ln"], rms_eps=eps))
    attn = np.zeros((bsz, nq * d))
    for b in range(bsz):
        pos = min(int(cache["seqlen"][b]), cache["k"][i].shape[2] - 1)
        attn[b] = bf(attend_row(qkv[b], L, c, cache["k"][i][b], cache["v"][i][b], pos))
    o = bf(ok.ternary_gemv(attn, L["o"], L["o_alpha"]))
    s_full = h + o
    res = bf(s_full)
    mlp_in = bf(ok.rms_norm(s_full, L["post_ln"], eps))
    moe = L["moe"]
    rid, rw, probs = ok.router_topk(mlp_in, moe["gate_weight"], c["top_k"])
    use_ids, use_w = rid, rw
    if router_ids is not None:
        use_ids = np.asarray(router_ids).reshape(rid.shape)
        top = np.take_along_axis(probs.reshape(bsz, -1), use_ids.reshape(bsz, -1), axis=1)
        use_w = (top / (top.sum(axis=1, keepdims=True) + 1e-20)).astype(np.float32)
    y, _ = ok.moe_experts(mlp_in, use_ids, use_w, moe["up_gate_packed"], moe["up_gate_alpha"],
                          moe["down_packed"], moe["down_alpha"], residual=res)
    return bf(y), (rid, probs)


def final_logits(m: dict, h):
    """Final RMSNorm and the RTN4 lm_head (``model.py:876-886``), bf16 logits."""
    c = m["cfg"]
    hn = bf(ok.rms_norm(h, m["final_norm"], c["eps"]))
    packed, sc, bs = m["lm_head"]
    logits = np.empty((hn.shape[0], packed.shape[0]))
    for r0 in range(0, packed.shape[0], 16384):  # dense float64 rows in chunks
        r1 = min(packed.shape[0], r0 + 16384)
        logits[:, r0:r1] = ok.rtn4_gemv(hn, packed[r0:r1], sc[r0:r1], bs[r0:r1], group_size=c["rtn_group"])
    return bf(logits)


def decoder_step(m: dict, cache: dict, ids, *, router_ids=None):
    """One greedy decode step.

    ``m``: cfg (dict), layers (list of dicts of NumPy weights), embed / lm_head
    (packed, scales, biases), final_norm, cos, sin.  ``cache``: ``k``/``v``
    lists of float arrays ``[B, n_kv, max_len, D]`` (updated in place) and
    ``seqlen`` ``[B]``.  ``router_ids``: optional per-layer expert ids, as in
    ``decoder_layer``.  Returns ``(logits [B, V] float64 after bf16 rounding,
    per-layer (ids, probs))``.
    """
    c = dict(m["cfg"], cos=m["cos"], sin=m["sin"])
    ids = np.asarray(ids).reshape(-1)
    h = bf(ok.rtn4_embedding(ids, *m["embed"], group_size=c["rtn_group"]))
    routing = []
    for i, L in enumerate(m["layers"]):
        h, r = decoder_layer(L, c, h, cache, i, router_ids=None if router_ids is None else router_ids[i])
        routing.append(r)
    cache["seqlen"] = np.asarray(cache["seqlen"]) + 1
    return final_logits(m, h), routing
