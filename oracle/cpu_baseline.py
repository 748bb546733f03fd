"""The reference's CPU path, float32, timed as the CPU baseline (test
infrastructure only: the product never imports it).

Every ternary product is the reference's CPU oracle pattern: NumPy
``unpack_2bit`` -> ``(code - 1) * alpha`` in float32 ->
``torch.nn.functional.linear(x.float(), w_hat)`` (reference
tests/test_ternary_gemv.py:24-25,83-86), the unpack part of every call.  The
MoE layer composes the router chain of tests/test_model.py:226-229
(``linear -> softmax -> topk -> / (sum + 1e-20)``) with the selected experts'
SwiGLU and down projections (tests/test_model.py:230-241); for batches it
unpacks each selected expert once and runs its tokens together.  The RTN4
head dequantises ``q * scale + bias`` per group (tests/test_rtn4.py:33-50).
The decoder token follows model.py:368-414, 477-506, 848-886 with QK-norm,
rotate-half RoPE on the first ``rotary_dim`` dims and GQA over the cache.
Pinned against the float64 oracle in tests/test_oracle_cpu_baseline.py.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from .kernels import MLP_CLAMP
from .pack import unpack_2bit, unpack_4bit


def dequant_ternary(packed, alpha) -> torch.Tensor:
    """``(code - 1) * alpha[n]`` as a float32 ``[N, K]`` tensor."""
    w = unpack_2bit(np.asarray(packed)).astype(np.float32) - 1.0
    return torch.from_numpy(w * np.asarray(alpha, np.float32)[:, None])


def ternary_gemv(x, packed, alpha) -> torch.Tensor:
    return F.linear(torch.as_tensor(x).float(), dequant_ternary(packed, alpha))


def router(x, gate_weight, top_k, bias=None):
    logits = F.linear(torch.as_tensor(x).float(), torch.as_tensor(gate_weight).float())
    if bias is not None:
        logits = logits + torch.as_tensor(bias).float()
    p = torch.softmax(logits, dim=-1)
    scores, ids = torch.topk(p, top_k, dim=-1)
    return ids, scores / (scores.sum(dim=-1, keepdim=True) + 1e-20)


def moe_layer(x, gate_weight, up_gate_packed, up_gate_alpha, down_packed, down_alpha, top_k,
              bias=None, residual=None) -> torch.Tensor:
    """One MoE FFN layer on ``x [T, H]`` in float32; returns ``[T, H]``."""
    x = torch.as_tensor(x).float()
    ids, wts = router(x, gate_weight, top_k, bias)
    y = torch.zeros_like(x) if residual is None else torch.as_tensor(residual).float().clone()
    inter = np.shape(up_gate_packed)[1] // 2
    for e in torch.unique(ids).tolist():
        tok, slot = torch.nonzero(ids == e, as_tuple=True)
        ug = F.linear(x[tok], dequant_ternary(up_gate_packed[e], up_gate_alpha[e]))
        up = ug[:, :inter].clamp(-MLP_CLAMP, MLP_CLAMP)
        gate = ug[:, inter:].clamp(max=MLP_CLAMP)
        h = F.silu(gate) * up
        out = F.linear(h, dequant_ternary(down_packed[e], down_alpha[e]))
        y.index_add_(0, tok, out * wts[tok, slot][:, None])
    return y


def rtn4_dequant(packed, scales, biases, group_size) -> torch.Tensor:
    q = unpack_4bit(np.asarray(packed)).astype(np.float32)
    n, k = q.shape
    g = q.reshape(n, k // group_size, group_size)
    w = g * np.asarray(scales, np.float32)[..., None] + np.asarray(biases, np.float32)[..., None]
    return torch.from_numpy(w.reshape(n, k))


def rtn4_gemv(x, packed, scales, biases, group_size, chunk_rows: int = 16384) -> torch.Tensor:
    x = torch.as_tensor(x).float()
    out = []
    for r0 in range(0, np.shape(packed)[0], chunk_rows):
        r1 = min(np.shape(packed)[0], r0 + chunk_rows)
        out.append(F.linear(x, rtn4_dequant(packed[r0:r1], scales[r0:r1], biases[r0:r1], group_size)))
    return torch.cat(out, dim=-1)


def rms_norm(x, w, eps):
    x = torch.as_tensor(x).float()
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * torch.as_tensor(w).float()


def _norm_rope(v, w, cos, sin, rot, eps, use_rope):
    v = rms_norm(v, w, eps)
    if use_rope and rot:
        half = rot // 2
        lo, hi = v[..., :half].clone(), v[..., half:rot].clone()
        v = v.clone()
        v[..., :half] = lo * cos[:half] - hi * sin[:half]
        v[..., half:rot] = hi * cos[half:rot] + lo * sin[half:rot]
    return v


def decoder_token(m: dict, cache: dict, token: int) -> torch.Tensor:
    """One decode step at batch 1; ``m`` and ``cache`` as for
    ``oracle.decoder.decoder_step`` (cache rows updated in place).  Returns
    float32 logits ``[V]``."""
    c = m["cfg"]
    nq, nkv, d, rot, eps = c["heads"], c["kv_heads"], c["head_dim"], c["rotary_dim"], c["eps"]
    emb_p, emb_s, emb_b = m["embed"]
    h = rtn4_dequant(emb_p[token:token + 1], emb_s[token:token + 1], emb_b[token:token + 1], c["rtn_group"])[0]
    pos = int(cache["seqlen"][0])
    cos = torch.as_tensor(m["cos"][pos]).float()
    sin = torch.as_tensor(m["sin"][pos]).float()
    for i, L in enumerate(m["layers"]):
        qkv = ternary_gemv(rms_norm(h, L["input_ln"], eps), L["qkv"], L["qkv_alpha"])
        use_rope = L.get("use_rope", True)
        q = _norm_rope(qkv[:nq * d].reshape(nq, d), L["q_norm"], cos, sin, rot, eps, use_rope)
        k = _norm_rope(qkv[nq * d:(nq + nkv) * d].reshape(nkv, d), L["k_norm"], cos, sin, rot, eps, use_rope)
        v = qkv[(nq + nkv) * d:].reshape(nkv, d)
        kc, vc = cache["k"][i], cache["v"][i]
        kc[0, :, pos] = k.numpy()
        vc[0, :, pos] = v.numpy()
        start = max(0, pos + 1 - L["window"]) if L.get("window") else 0
        K = torch.as_tensor(kc[0, :, start:pos + 1]).float()  # [nkv, L, d]
        V = torch.as_tensor(vc[0, :, start:pos + 1]).float()
        qg = q.reshape(nkv, nq // nkv, d)
        att = torch.softmax(qg @ K.transpose(1, 2) * d ** -0.5, dim=-1) @ V
        o = ternary_gemv(att.reshape(-1), L["o"], L["o_alpha"])
        s = h + o
        mo = L["moe"]
        h = moe_layer(rms_norm(s, L["post_ln"], eps)[None], mo["gate_weight"], mo["up_gate_packed"],
                      mo["up_gate_alpha"], mo["down_packed"], mo["down_alpha"], c["top_k"], residual=s[None])[0]
    cache["seqlen"] = np.asarray(cache["seqlen"]) + 1
    return rtn4_gemv(rms_norm(h, m["final_norm"], eps)[None], *m["lm_head"], c["rtn_group"])[0]
