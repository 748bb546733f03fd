"""Closed forms of the hot-path kernels, float64 (test infrastructure only).

Every function takes NumPy arrays holding the exact values the device sees
(bf16 inputs are passed as their float32 widening) and returns float64 unless
an integer result is asked for.  Rounding to bf16 happens only where the
reference stores an intermediate in ``x.dtype`` (``bf16_round``).

Reference call sites restated here (paths under ``src/maple_run/``):

* ``ternary_gemv``          kernels/ternary_gemv.py:101-153 (B=1), :193-258 (B>1)
* ``router_topk``           kernels/router.py:39-126
* ``dispatch``              no reference code: stable counting sort of
                            (token, slot) pairs by expert id
* ``ternary_expert_gemv``   kernels/ternary_expert.py:80-122, :177-204
* ``ternary_expert_swiglu`` kernels/ternary_expert.py:263-319
* ``ternary_expert_down_sum`` kernels/ternary_expert.py:355-400
* ``moe_reduce_add``        kernels/fused_norm.py:59-96
* ``moe_block``             model.py:465-474
* ``rtn4_gemv``             kernels/rtn4.py:108-167, :197-282
* ``rtn4_embedding``        kernels/rtn4.py:27-47
* ``rms_norm`` / ``add_rms_norm``  kernels/fused_norm.py:10-56
"""

from __future__ import annotations

import numpy as np

from .pack import dequantize_rtn, ternary_values, unpack_2bit, unpack_4bit

MLP_CLAMP = 7.0  # ternary_expert.py:237, model.py:35


def bf16_round(a) -> np.ndarray:
    """Round to the nearest bfloat16 (ties to even), returned as float32.

    bf16 is the upper half of an IEEE float32; adding ``0x7FFF`` plus the
    lowest kept bit before truncating implements round-to-nearest-even.
    """
    f = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    out = u.astype(np.uint32).view(np.float32).reshape(f.shape)
    return np.where(np.isnan(f), f, out)


def _rows(x: np.ndarray, k: int) -> np.ndarray:
    return np.asarray(x, dtype=np.float64).reshape(-1, k)


def ternary_dense(packed: np.ndarray, alpha: np.ndarray, packed_kn: bool = False) -> np.ndarray:
    """Dequantised ``alpha[n] * (code[n, k] - 1)`` as a dense float64 matrix."""
    p = np.asarray(packed)
    if packed_kn:
        p = np.swapaxes(p, -1, -2)
    t = ternary_values(p)
    return t * np.asarray(alpha, dtype=np.float64)[..., None]


def ternary_gemv(x, packed, alpha, *, rms_weight=None, rms_eps=1e-6, packed_kn=False):
    """``y = alpha * (T @ x_hat)``; with ``rms_weight`` the input is RMS-normed.

    The reference folds RMSNorm into the GEMV as
    ``acc * rsqrt(sum(x^2)/K + eps)`` with ``x_hat = x * w_rms``
    (``ternary_gemv.py:110-146``), which equals ``T @ rms_norm(x)``.
    """
    w = ternary_dense(packed, alpha, packed_kn)
    n, k = w.shape
    xr = _rows(x, k)
    if rms_weight is not None:
        rstd = 1.0 / np.sqrt((xr * xr).mean(axis=1, keepdims=True) + rms_eps)
        xr = xr * rstd * np.asarray(rms_weight, np.float64).reshape(1, k)
    y = xr @ w.T
    return y.reshape(*np.shape(x)[:-1], n)


def router_topk(x, gate_weight, top_k, bias=None):
    """Softmax router with top-k and renormalisation (``router.py:39-126``).

    ``p = softmax(x @ W^T [+ bias])`` over all experts; the top-k are taken in
    descending probability, ties to the lowest expert index (Triton
    ``argmax`` semantics, ``router.py:115-121``); weights are
    ``p_j / (sum p_top + 1e-20)``.  ``bias`` is an optional additive
    logit bias for skewed-routing workloads; ``None`` is the reference.

    Returns ``(ids int32 [..., k], weights float32 [..., k], probs float64
    [..., E])`` -- ``probs`` lets a test measure how close a decision was.
    """
    g = np.asarray(gate_weight, np.float64)
    e, k = g.shape
    xr = _rows(x, k)
    logits = xr @ g.T
    if bias is not None:
        logits = logits + np.asarray(bias, np.float64)[None, :]
    logits = logits - logits.max(axis=1, keepdims=True)
    p = np.exp(logits)
    p = p / p.sum(axis=1, keepdims=True)
    order = np.argsort(-p, axis=1, kind="stable")[:, :top_k]
    top = np.take_along_axis(p, order, axis=1)
    wts = top / (top.sum(axis=1, keepdims=True) + 1e-20)
    lead = np.shape(x)[:-1]
    return (
        order.astype(np.int32).reshape(*lead, top_k),
        wts.astype(np.float32).reshape(*lead, top_k),
        p.reshape(*lead, e),
    )


def dispatch(expert_ids, n_experts):
    """Per-expert lists of (token, slot) pairs.

    Pair ``p = token * k + slot``.  ``pair_ids`` is the stable sort of pairs by
    expert id, so each expert's list is ascending in token; ``offsets`` is the
    exclusive scan of ``counts``; ``inverse[p]`` is where pair ``p`` landed.
    """
    flat = np.asarray(expert_ids).reshape(-1).astype(np.int64)
    if flat.size and (flat.min() < 0 or flat.max() >= n_experts):
        raise ValueError("expert id out of range")
    counts = np.bincount(flat, minlength=n_experts).astype(np.int32)
    offsets = np.zeros(n_experts + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    pair_ids = np.argsort(flat, kind="stable").astype(np.int32)
    inverse = np.empty_like(pair_ids)
    inverse[pair_ids] = np.arange(flat.size, dtype=np.int32)
    return counts, offsets, pair_ids, inverse


def _slot_inputs(x, k_in, id_shape):
    """Per-slot activation rows (``ternary_expert.py:177-204``)."""
    xs = np.asarray(x, np.float64)
    if xs.shape[:-1] == tuple(id_shape):
        return xs.reshape(-1, k_in)
    if xs.shape[:-1] == tuple(id_shape[:-1]):
        topk = id_shape[-1]
        return np.repeat(xs.reshape(-1, k_in), topk, axis=0)
    raise ValueError(f"x shape {xs.shape} incompatible with expert_ids {tuple(id_shape)}")


def ternary_expert_gemv(x, packed, alpha, expert_ids, *, packed_kn=False):
    """``y[s] = alpha_e * (T_e @ x_s)`` for every slot ``s`` with ``e = ids[s]``."""
    ids = np.asarray(expert_ids)
    flat = ids.reshape(-1)
    p, a = np.asarray(packed), np.asarray(alpha)
    n = p.shape[2] if packed_kn else p.shape[1]
    k = (p.shape[1] if packed_kn else p.shape[2]) * 16
    xs = _slot_inputs(x, k, ids.shape)
    y = np.zeros((flat.size, n))
    for e in np.unique(flat):  # one dense expert at a time keeps memory small
        rows = np.nonzero(flat == e)[0]
        y[rows] = xs[rows] @ ternary_dense(p[e], a[e], packed_kn).T
    return y.reshape(*ids.shape, n)


def swiglu_act(up, gate):
    """``clamp(up, -7, 7) * g * sigmoid(g)`` with ``g = min(gate, 7)``
    (``ternary_expert.py:314-318``)."""
    up = np.clip(up, -MLP_CLAMP, MLP_CLAMP)
    gate = np.minimum(gate, MLP_CLAMP)
    return up * gate / (1.0 + np.exp(-gate))


def ternary_expert_swiglu(x, packed, alpha, expert_ids, *, packed_kn=False):
    """Fused up+gate GEMV and SwiGLU; packed rows are ``[up; gate]``."""
    both = ternary_expert_gemv(x, packed, alpha, expert_ids, packed_kn=packed_kn)
    n = both.shape[-1] // 2
    return swiglu_act(both[..., :n], both[..., n:])


def ternary_expert_down_sum(x, packed, alpha, expert_ids, topk_weight, residual=None,
                            *, packed_kn=False):
    """``y[t] = sum_j w[t,j] * alpha_e (T_e @ x[t,j]) (+ residual)`` in one
    precision, no intermediate rounding (``ternary_expert.py:364-399``)."""
    ids = np.asarray(expert_ids)
    per_slot = ternary_expert_gemv(x, packed, alpha, ids, packed_kn=packed_kn)
    wts = np.asarray(topk_weight, np.float64)
    y = (per_slot * wts[..., None]).sum(axis=-2)
    if residual is not None:
        y = y + np.asarray(residual, np.float64).reshape(y.shape)
    return y


def moe_reduce_add(expert_out, topk_weight, residual=None):
    """``y = sum_j w_j * expert_out_j (+ residual)`` (``fused_norm.py:83-96``)."""
    eo = np.asarray(expert_out, np.float64)
    y = (eo * np.asarray(topk_weight, np.float64)[..., None]).sum(axis=-2)
    if residual is not None:
        y = y + np.asarray(residual, np.float64).reshape(y.shape)
    return y


def moe_block(x, gate_weight, up_gate_packed, up_gate_alpha, down_packed, down_alpha,
              top_k, residual=None, *, router_bias=None, round_bf16=True):
    """The MoE FFN of ``model.py:465-474``: router -> SwiGLU -> down -> combine.

    With ``round_bf16`` the intermediates are rounded where the reference
    stores them in ``x.dtype`` (bf16): the SwiGLU output ``h`` and the per-slot
    down outputs (``ternary_expert.py:208,441``).  Returns
    ``(y, ids, weights, probs)``.
    """
    ids, wts, probs = router_topk(x, gate_weight, top_k, bias=router_bias)
    h = ternary_expert_swiglu(x, up_gate_packed, up_gate_alpha, ids)
    if round_bf16:
        h = bf16_round(h).astype(np.float64)
    eo = ternary_expert_gemv(h, down_packed, down_alpha, ids)
    if round_bf16:
        eo = bf16_round(eo).astype(np.float64)
    y = moe_reduce_add(eo, wts, residual)
    return y, ids, wts, probs


def rtn4_dense(packed, scales, biases, group_size, packed_kn=False):
    """Dequantised ``q * s_g + b_g`` in float64 from the stored scales/biases."""
    p, s, b = np.asarray(packed), np.asarray(scales), np.asarray(biases)
    if packed_kn:
        p, s, b = p.T, s.T, b.T
    q = unpack_4bit(p).astype(np.float64)
    n, k = q.shape
    g = q.reshape(n, k // group_size, group_size)
    rec = g * np.asarray(s, np.float64)[..., None] + np.asarray(b, np.float64)[..., None]
    return rec.reshape(n, k)


def rtn4_gemv(x, packed, scales, biases, group_size=64, *, packed_kn=False):
    """``y = sum_g sum_{k in g} (q*s_g + b_g) x_k`` (``rtn4.py:108-167``)."""
    w = rtn4_dense(packed, scales, biases, group_size, packed_kn)
    n, k = w.shape
    y = _rows(x, k) @ w.T
    return y.reshape(*np.shape(x)[:-1], n)


def rtn4_embedding(input_ids, packed, scales, biases, group_size=64):
    """Dequantised rows of the 4-bit table for ``input_ids`` (``rtn4.py:27-47``)."""
    ids = np.asarray(input_ids).astype(np.int64)
    p = np.asarray(packed)[ids.reshape(-1)]
    s = np.asarray(scales, np.float32)[ids.reshape(-1)]
    b = np.asarray(biases, np.float32)[ids.reshape(-1)]
    rows = dequantize_rtn(p, s, b, group_size)
    return rows.reshape(*ids.shape, rows.shape[-1])


def rms_norm(x, weight, eps=1e-6):
    """``x * rsqrt(mean(x^2) + eps) * w`` over the last axis (``fused_norm.py:10-28``)."""
    xf = np.asarray(x, np.float64)
    rstd = 1.0 / np.sqrt((xf * xf).mean(axis=-1, keepdims=True) + eps)
    return xf * rstd * np.asarray(weight, np.float64)


def add_rms_norm(x, y, weight, eps=1e-6):
    """``s = x + y``; returns ``(s, rms_norm(s))`` (``fused_norm.py:31-56``)."""
    s = np.asarray(x, np.float64) + np.asarray(y, np.float64)
    return s, rms_norm(s, weight, eps)


def moe_layer_cpu_fp32(x, gate_weight, up_gate_packed, up_gate_alpha, down_packed, down_alpha, top_k):
    """The reference's CPU oracle path for one MoE layer, float32 throughout:
    router ``linear -> softmax -> topk -> renorm`` (``tests/test_model.py:225-229``),
    then for every selected expert NumPy ``unpack_2bit`` -> ``(code - 1) * alpha``
    -> matmul (``tests/test_ternary_gemv.py:24-25,83-86``; the loop of
    ``tests/test_model.py:230-241``).  The unpack is part of every call.
    Used as the CPU baseline; returns ``[T, H]`` float32.
    """
    x = np.asarray(x, np.float32).reshape(-1, np.shape(gate_weight)[1])
    logits = x @ np.asarray(gate_weight, np.float32).T
    logits -= logits.max(axis=1, keepdims=True)
    p = np.exp(logits)
    p /= p.sum(axis=1, keepdims=True)
    ids = np.argsort(-p, axis=1, kind="stable")[:, :top_k]
    top = np.take_along_axis(p, ids, axis=1)
    wts = top / (top.sum(axis=1, keepdims=True) + np.float32(1e-20))
    inter = np.shape(up_gate_packed)[1] // 2
    y = np.zeros_like(x)
    for t in range(x.shape[0]):
        for j in range(top_k):
            e = int(ids[t, j])
            wug = (unpack_2bit(up_gate_packed[e]).astype(np.float32) - 1.0) * np.asarray(up_gate_alpha[e], np.float32)[:, None]
            ug = wug @ x[t]
            up = np.clip(ug[:inter], -MLP_CLAMP, MLP_CLAMP)
            gate = np.minimum(ug[inter:], MLP_CLAMP)
            h = up * gate / (1.0 + np.exp(-gate))
            wd = (unpack_2bit(down_packed[e]).astype(np.float32) - 1.0) * np.asarray(down_alpha[e], np.float32)[:, None]
            y[t] += wts[t, j] * (wd @ h)
    return y


def moe_experts(x, ids, wts, up_gate_packed, up_gate_alpha, down_packed, down_alpha,
                residual=None, *, round_bf16=True):
    """Expert half of ``model.py:468-473`` for a given routing: SwiGLU, per-slot
    down projection and the weighted combine, with the reference's bf16
    rounding of ``h`` and of each slot's down output.  Returns ``(y, h)``."""
    h = ternary_expert_swiglu(x, up_gate_packed, up_gate_alpha, ids)
    if round_bf16:
        h = bf16_round(h).astype(np.float64)
    eo = ternary_expert_gemv(h, down_packed, down_alpha, ids)
    if round_bf16:
        eo = bf16_round(eo).astype(np.float64)
    return moe_reduce_add(eo, wts, residual), h
