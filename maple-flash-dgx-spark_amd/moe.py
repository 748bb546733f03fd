"""The MoE FFN block on the HIP kernels (reference ``src/maple_run/model.py:448-474``).

``MapleSparseMoeBlock`` keeps the reference composition and call signature:
router -> up+gate SwiGLU -> down -> top-k combine (+ residual), with no host
sync and no per-expert Python loop.  Three execution plans, chosen by the
token count and the shape alone (never by routing, which stays on the
device):

* one token, shapes built into ``ma_moe_fused`` (``plan="fused"``): router,
  SwiGLU, down and combine (optionally with the add + RMSNorm ahead of the
  block) in one persistent launch; 12.0 us per layer at hidden 2048 / 64
  experts / top-8 against 14.2 us for the per-slot chain.  Rounding points
  match the reference (bf16 h, bf16 per-slot output, float32 combine).
* other decode (``tokens < GROUPED_MIN_TOKENS``, ``plan="per_slot"``):
  per-slot kernels, as the reference does -- fused SwiGLU, then the down
  projection and the combine in one launch
  (``ternary_expert_down_sum(..., round_slots=True)``), with the reference's
  rounding points: each slot's down output rounded to bf16 before the
  float32 combine, the residual added last (``model.py:470-473``).
* batched decode / prefill: dispatch the (token, slot) pairs into per-expert
  lists and run grouped MFMA GEMMs (``ma_moe_grouped``), so each selected
  expert's weights are read once per tile of its tokens instead of once per
  pair.  Rounding points match the reference (bf16 h, bf16 per-slot output,
  float32 combine).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib, workspace
from .kernels.dispatch import moe_dispatch
from .kernels.router import router_topk
from .kernels.ternary_expert import ternary_expert_down_sum, ternary_expert_swiglu
from .synthetic import MoELayer

GROUPED_MIN_TOKENS = 4

_RESIDENT: dict[tuple, bool] = {}


def fused_resident(layer: MoELayer, top_k: int, device) -> bool:
    """True if every workgroup of the one-launch layer fits on ``device`` at
    once (its grid barrier needs that; not so on a partitioned GPU, say).
    Queried once per device and shape."""
    idx = torch.device(device).index
    idx = torch.cuda.current_device() if idx is None else idx
    key = (idx, layer.n_experts, layer.hidden, layer.inter, top_k)
    ok = _RESIDENT.get(key)
    if ok is None:
        needed, capacity = ctypes.c_int64(0), ctypes.c_int64(0)
        with torch.cuda.device(idx):
            _lib.call("ma_moe_fused_resident", layer.n_experts, layer.hidden, layer.inter, top_k,
                      ctypes.byref(needed), ctypes.byref(capacity))
        ok = _RESIDENT[key] = capacity.value >= needed.value
    return ok


def fused_supported(layer: MoELayer, top_k: int, x: torch.Tensor) -> bool:
    """True if ``ma_moe_fused`` is built for this layer's shape and dtypes and
    its grid fits on ``x``'s device at once."""
    if x.dtype != torch.bfloat16 or layer.gate_weight.dtype != torch.bfloat16:
        return False
    if layer.up_gate_alpha.dtype != layer.down_alpha.dtype or \
            layer.up_gate_alpha.dtype not in (torch.bfloat16, torch.float32):
        return False
    if int(_lib.load().ma_moe_fused_workspace_bytes(layer.n_experts, layer.hidden, layer.inter,
                                                    top_k)) == 0:
        return False
    return fused_resident(layer, top_k, x.device)


def fused_form(layer: MoELayer, top_k: int) -> int:
    """The form ``ma_moe_fused`` runs for this layer on the current device:
    1 the XCD split (each XCD one top-k slot), 0 the one-barrier grid, -1 not
    built."""
    return int(_lib.load().ma_moe_fused_form(layer.n_experts, layer.hidden, layer.inter, top_k))


LAYOUT_WORD = 4  # uint32 word of the one-launch workspace set by the XCD form's layout check


def _layout_check(workspaces, idx: int):
    """check_timeouts hook: if the XCD-split form found its workgroups not
    spread over the XCDs as it assumes (and aborted the call), turn the
    XCD-split forms off on the device so that later calls take the
    one-barrier / cross-XCD forms."""
    if not workspaces:
        return None
    words = torch.stack([ws.view(torch.int32)[LAYOUT_WORD] for ws in workspaces]).cpu()
    if not bool((words != 0).any()):
        return None
    _lib.call("ma_xcd_forms_disable", idx, 1)
    return (f"the XCD-split MoE launch found its workgroups not spread over the XCDs of device {idx} "
            "as probed; the XCD-split forms are now off on that device")


workspace.on_timeout("moe_fused", _layout_check)


def moe_fused_timed_out(device: torch.device | int = 0) -> bool:
    """True if a one-launch MoE call on ``device`` timed out waiting for another
    workgroup since its workspace was zeroed (the kernel records it instead of
    hanging).  Syncs."""
    return "moe_fused" in workspace.timed_out_kinds(device)


def moe_fused(x: torch.Tensor, layer: MoELayer, top_k: int, residual: torch.Tensor | None = None,
              *, add: torch.Tensor | None = None, norm_weight: torch.Tensor | None = None,
              eps: float = 1e-6, next_linear: tuple | None = None, o_linear: tuple | None = None,
              prefetch: torch.Tensor | None = None):
    """One token through the whole MoE layer in one launch.

    Plain: ``y = x_res + sum_j w_j down_j(swiglu_j(x))`` with ``x_res =
    residual`` (or none).  With ``add``/``norm_weight`` (the decoder's
    post-attention add + RMSNorm, ``fused_norm.py:128-161``): ``s = x + add``,
    the block runs on ``rms_norm(s) * norm_weight`` and adds ``bf16(s)``.
    Returns ``(y [1, H], ids int32 [1, k], weights float32 [1, k])``.

    ``next_linear = (packed [N, H/16] uint32, alpha [N], rms_weight float32
    [H], rms_eps)``: the same launch also computes the next layer's input
    projection ``ternary_gemv(y, packed, alpha, rms_weight=..., rms_eps=...)``
    (the same bits) and returns it as a fourth output ``[1, N]``.

    ``o_linear = (attn [1, H] bf16, packed [H, H/16] uint32, alpha [H])`` in
    place of ``add``: the launch computes ``add = ternary_gemv(attn, packed,
    alpha)`` itself (the attention's output projection, the same bits as the
    separate GEMV; alpha of the experts' row_alpha dtype); needs the XCD-split
    form (``fused_form(layer, top_k) == 1``).

    ``prefetch``: a contiguous device tensor (16-byte aligned) that the launch
    reads ahead into the caches for a later kernel -- the next MoE layer's
    router weight, say (routing-independent bytes); no effect on the results.
    """
    hidden = x.shape[-1]
    xf = x.reshape(1, hidden).contiguous()
    ad = None if add is None else add.reshape(1, hidden).contiguous()
    if o_linear is not None:
        if ad is not None:
            raise ValueError("moe_fused: add and o_linear are exclusive")
        o_in, o_w, o_a = o_linear
        o_in = o_in.reshape(1, hidden).contiguous()
        if o_in.dtype != torch.bfloat16 or o_w.dtype != torch.uint32 or tuple(o_w.shape) != (hidden, hidden // 16):
            raise TypeError("o_linear must be (bf16 [1, H], uint32 [H, H/16], alpha [H])")
        if o_a.dtype != layer.up_gate_alpha.dtype:
            raise TypeError("o_linear alpha must have the experts' row_alpha dtype")
        o_a = o_a.contiguous()
    if (ad is not None or o_linear is not None) and norm_weight is None:
        raise ValueError("moe_fused: add needs norm_weight")
    pf_bytes = 0
    if prefetch is not None:
        if not prefetch.is_contiguous() or prefetch.device != x.device:
            raise ValueError("moe_fused: prefetch must be a contiguous tensor on x's device")
        pf_bytes = prefetch.numel() * prefetch.element_size()
    res = (None if residual is None or ad is not None or o_linear is not None
           else residual.reshape(1, hidden).contiguous())
    nbytes = int(_lib.load().ma_moe_fused_workspace_bytes(layer.n_experts, hidden, layer.inter, top_k))
    if nbytes == 0:
        raise ValueError(f"moe_fused: shape (hidden {hidden}, inter {layer.inter}, top_k {top_k}) "
                         "is not built into the one-launch kernel")
    # zero-filled once: workgroups hand data to each other through it, tagged
    # with call counters the kernel keeps there
    ws = workspace.get("moe_fused", x.device, nbytes, (hidden, layer.inter, top_k))
    y = torch.empty(1, hidden, device=x.device, dtype=torch.bfloat16)
    ids = torch.empty(1, top_k, device=x.device, dtype=torch.int32)
    wts = torch.empty(1, top_k, device=x.device, dtype=torch.float32)
    nw = None if norm_weight is None else norm_weight.reshape(-1).contiguous()
    bias = None if layer.router_bias is None else layer.router_bias.float().contiguous()
    alpha_dt = _lib.dtype_code(layer.up_gate_alpha, "row_alpha")
    if _lib.dtype_code(layer.down_alpha, "row_alpha") != alpha_dt:
        raise TypeError("up_gate and down row_alpha must share a dtype")
    nx_w = nx_a = nx_r = nx_out = None
    nx_eps, nx_rows = 0.0, 0
    if next_linear is not None:
        nx_w, nx_a, nx_r, nx_eps = next_linear
        if nx_w.dtype != torch.uint32:
            raise TypeError("next_linear packed weight must be torch.uint32")
        if nx_w.shape[1] * 16 != hidden or nx_r.numel() != hidden or nx_r.dtype != torch.float32:
            raise ValueError("next_linear must be ([N, hidden/16] uint32, alpha [N], float32 rms [hidden], eps)")
        nx_rows = int(nx_w.shape[0])
        nx_a, nx_r = nx_a.contiguous(), nx_r.contiguous()
        if nx_a.dtype != layer.up_gate_alpha.dtype:
            raise TypeError("next_linear alpha must have the experts' row_alpha dtype")
        nx_out = torch.empty(1, nx_rows, device=x.device, dtype=torch.bfloat16)
    if o_linear is not None:
        _lib.call(
            "ma_moe_fused_o",
            _lib.ptr(xf), _lib.ptr(o_in), _lib.ptr(o_w), _lib.ptr(o_a), _lib.ptr(nw),
            _lib.dtype_code(nw, "norm_weight"), float(eps),
            _lib.ptr(layer.gate_weight), _lib.ptr(bias), layer.n_experts, hidden, layer.inter, top_k,
            _lib.ptr(layer.up_gate_packed), _lib.ptr(layer.up_gate_alpha), _lib.ptr(layer.down_packed),
            _lib.ptr(layer.down_alpha), alpha_dt, _lib.ptr(y), _lib.ptr(ids), _lib.ptr(wts), _lib.ptr(ws),
            ws.numel(), _lib.ptr(nx_w), _lib.ptr(nx_a),
            _lib.dtype_code(nx_a, "row_alpha") if nx_a is not None else 0, _lib.ptr(nx_r),
            float(nx_eps), nx_rows, _lib.ptr(nx_out), _lib.ptr(prefetch), pf_bytes, _lib.stream_of(x),
        )
        return (y, ids, wts, nx_out) if next_linear is not None else (y, ids, wts)
    _lib.call(
        "ma_moe_fused",
        _lib.ptr(xf), _lib.ptr(ad), _lib.ptr(nw),
        _lib.dtype_code(nw, "norm_weight") if nw is not None else 0, float(eps), _lib.ptr(res),
        _lib.ptr(layer.gate_weight), _lib.ptr(bias), layer.n_experts, hidden, layer.inter, top_k,
        _lib.ptr(layer.up_gate_packed), _lib.ptr(layer.up_gate_alpha), _lib.ptr(layer.down_packed),
        _lib.ptr(layer.down_alpha), alpha_dt, _lib.ptr(y), _lib.ptr(ids), _lib.ptr(wts), _lib.ptr(ws),
        ws.numel(), _lib.ptr(nx_w), _lib.ptr(nx_a),
        _lib.dtype_code(nx_a, "row_alpha") if nx_a is not None else 0, _lib.ptr(nx_r),
        float(nx_eps), nx_rows, _lib.ptr(nx_out), _lib.ptr(prefetch), pf_bytes, _lib.stream_of(x),
    )
    if next_linear is not None:
        return y, ids, wts, nx_out
    return y, ids, wts


ROUTE_MAX_TOKENS = 1024


def route_supported(layer: MoELayer, top_k: int, x: torch.Tensor) -> bool:
    """True if ``ma_moe_route`` takes these sizes and dtypes."""
    tokens, hidden = x.reshape(-1, x.shape[-1]).shape
    return (x.dtype == torch.bfloat16 and layer.gate_weight.dtype == torch.bfloat16
            and 1 <= tokens <= ROUTE_MAX_TOKENS and hidden % 8 == 0 and hidden <= 4096
            and layer.n_experts <= 256 and 1 <= top_k <= layer.n_experts)


def route_timed_out(device: torch.device | int = 0) -> bool:
    """True if a routing launch on ``device`` timed out waiting for another
    workgroup since its workspace was zeroed.  Syncs."""
    return "moe_route" in workspace.timed_out_kinds(device)


def moe_route(x: torch.Tensor, layer: MoELayer, top_k: int, norm_weight: torch.Tensor,
              eps: float, add: torch.Tensor | None = None, *, pairs: bool = False):
    """Residual add + RMSNorm + router + dispatch in one launch for ``x [T, H]``.

    Returns ``(h, xn, ids, weights, dispatch)``: ``h = x + add`` (``x`` itself
    when ``add`` is None), ``xn = rms_norm(h) * norm_weight``, the router's
    int32 ids / float32 weights ``[T, top_k]`` and the :class:`Dispatch` lists.
    Equal, bit for bit, to add_rms_norm + router_topk + moe_dispatch.  With
    ``pairs``, a sixth item ``(xn_pairs, xn_corr)``: xn in the x' pair form the
    grouped experts read, and each token's correction."""
    from .kernels.dispatch import Dispatch
    tokens, hidden = x.shape
    dev = x.device
    nbytes = int(_lib.load().ma_moe_route_workspace_bytes(ROUTE_MAX_TOKENS, layer.n_experts))
    # zero-filled once; each launch leaves its ticket counter and tags cleared
    ws = workspace.get("moe_route", dev, nbytes, (layer.n_experts,))
    xc = x.contiguous()
    ac = None if add is None else add.reshape(tokens, hidden).contiguous()
    h = torch.empty_like(xc) if ac is not None else xc
    xn = torch.empty_like(xc)
    ids = torch.empty(tokens, top_k, device=dev, dtype=torch.int32)
    wts = torch.empty(tokens, top_k, device=dev, dtype=torch.float32)
    n_exp = layer.n_experts
    counts = torch.empty(n_exp, device=dev, dtype=torch.int32)
    offsets = torch.empty(n_exp + 1, device=dev, dtype=torch.int32)
    pair_ids = torch.empty(tokens * top_k, device=dev, dtype=torch.int32)
    inverse = torch.empty(tokens * top_k, device=dev, dtype=torch.int32)
    nwc = norm_weight.contiguous()
    xp = torch.empty(tokens, hidden // 2, device=dev, dtype=torch.uint32) if pairs else None
    xcorr = torch.empty(tokens, device=dev, dtype=torch.float32) if pairs else None
    _lib.call(
        "ma_moe_route",
        _lib.ptr(xc), _lib.ptr(ac), tokens, hidden, _lib.ptr(nwc), _lib.dtype_code(nwc, "norm_weight"),
        float(eps), _lib.ptr(layer.gate_weight), _lib.ptr(layer.router_bias), n_exp, int(top_k),
        _lib.ptr(h) if ac is not None else None, _lib.ptr(xn), _lib.ptr(xp), _lib.ptr(xcorr),
        _lib.ptr(ids), _lib.ptr(wts),
        _lib.ptr(counts), _lib.ptr(offsets), _lib.ptr(pair_ids), _lib.ptr(inverse),
        _lib.ptr(ws), ws.numel(), _lib.stream_of(xc),
    )
    d = Dispatch(counts, offsets, pair_ids, inverse)
    if pairs:
        return h, xn, ids, wts, d, (xp, xcorr)
    return h, xn, ids, wts, d


@dataclass
class PendingCombine:
    """A grouped MoE layer whose top-k combine has not run yet: ``y[t] =
    sum_j weights[t, j] * slot_out[inverse[t, j]] + residual[t]``.  The next
    RMS-folded GEMM runs it (``kernels.ternary_gemv.ternary_gemv_combine``);
    ``workspace`` keeps ``slot_out``'s storage alive."""
    slot_out: torch.Tensor   # bf16 [T * k, H], inside workspace
    inverse: torch.Tensor    # int32 [T * k]
    weights: torch.Tensor    # float32 [T * k]
    residual: torch.Tensor | None
    top_k: int
    tokens: int
    hidden: int
    workspace: torch.Tensor


def moe_grouped(x: torch.Tensor, layer: MoELayer, ids: torch.Tensor, wts: torch.Tensor,
                residual: torch.Tensor | None = None, *, return_h: bool = False, dispatch=None,
                x_pairs=None, combine: bool = True):
    """Dispatch + grouped MFMA SwiGLU/down + combine for ``x [T, H]`` (bf16).

    ``dispatch``: the lists for ``ids`` if already built (``moe_route``);
    ``x_pairs``: ``(xn_pairs, xn_corr)`` of ``x`` from ``moe_route(pairs=True)``
    or ``router_topk(..., pairs=True)``.
    Returns ``y [T, H]`` (bf16), and with ``return_h`` also ``h [T, k, I]``;
    with ``combine=False`` a ``PendingCombine`` in place of ``y``.
    """
    tokens, hidden = x.shape
    top_k = int(ids.shape[-1])
    inter = layer.inter
    d = dispatch if dispatch is not None else moe_dispatch(ids, layer.n_experts)
    n_pairs = tokens * top_k
    nbytes = int(_lib.load().ma_grouped_workspace_bytes(n_pairs, inter, hidden))
    ws = torch.empty(nbytes, device=x.device, dtype=torch.uint8)
    y = torch.empty(tokens, hidden, device=x.device, dtype=torch.bfloat16) if combine else None
    h = torch.empty(n_pairs, inter, device=x.device, dtype=torch.bfloat16) if return_h else None
    res = None if residual is None else residual.reshape(tokens, hidden).contiguous()
    xc = x.contiguous()
    w = wts.reshape(-1).float().contiguous()
    alpha_dt = _lib.dtype_code(layer.up_gate_alpha, "row_alpha")
    if _lib.dtype_code(layer.down_alpha, "row_alpha") != alpha_dt:
        raise TypeError("up_gate and down row_alpha must share a dtype")
    _lib.call(
        "ma_moe_grouped",
        _lib.ptr(xc), xc.stride(0), _lib.ptr(x_pairs[0] if x_pairs else None),
        _lib.ptr(x_pairs[1] if x_pairs else None), tokens, top_k,
        _lib.ptr(layer.up_gate_packed), _lib.ptr(layer.up_gate_alpha),
        _lib.ptr(layer.down_packed), _lib.ptr(layer.down_alpha), alpha_dt,
        layer.n_experts, hidden, inter,
        _lib.ptr(d.offsets), _lib.ptr(d.pair_ids), _lib.ptr(d.inverse), _lib.ptr(w),
        _lib.ptr(res), _lib.dtype_code(res, "residual") if res is not None else 0,
        _lib.ptr(h), inter, _lib.ptr(y), _lib.ptr(ws), ws.numel(), _lib.stream_of(x),
    )
    if not combine:
        # the per-pair down outputs sit after the pair-format h in the workspace
        off = (n_pairs * inter * 2 + 255) // 256 * 256
        slot_out = ws[off:off + n_pairs * hidden * 2].view(torch.bfloat16).view(n_pairs, hidden)
        y = PendingCombine(slot_out, d.inverse, w, res, top_k, tokens, hidden, ws)
    if return_h:
        return y, h.reshape(tokens, top_k, inter)
    return y


def choose_plan(tokens: int, fused_ok: bool, grouped_ok: bool) -> str:
    """The execution plan of ``moe_block`` for ``tokens`` tokens: "fused" (one
    token, where ``ma_moe_fused`` is built for the shape and its grid fits on
    the device at once), "grouped" (from GROUPED_MIN_TOKENS tokens, where the
    grouped MFMA kernels take the shape), else "per_slot" -- the multi-launch
    kernels, which need no co-resident workgroups."""
    if tokens == 1 and fused_ok:
        return "fused"
    if tokens >= GROUPED_MIN_TOKENS and grouped_ok:
        return "grouped"
    return "per_slot"


def grouped_supported(layer: MoELayer, x: torch.Tensor) -> bool:
    """True if the grouped MFMA kernels take this layer's shape and ``x``."""
    return x.dtype == torch.bfloat16 and layer.hidden % 256 == 0 and layer.inter % 256 == 0


def moe_block(x: torch.Tensor, layer: MoELayer, top_k: int, residual: torch.Tensor | None = None,
              *, plan: str = "auto", prefetch: torch.Tensor | None = None):
    """One MoE layer on ``x [..., H]``; returns ``(y, ids, weights)``.

    ``plan``: "auto" (``choose_plan``), or "per_slot" / "grouped" / "fused"
    to force one.  ``prefetch``: bytes the one-launch plan reads ahead into
    the caches (``moe_fused``); the other plans ignore it."""
    hidden = x.shape[-1]
    xf = x.reshape(-1, hidden)
    if plan == "auto":
        tokens = xf.shape[0]
        plan = choose_plan(tokens, tokens == 1 and fused_supported(layer, top_k, xf),
                           grouped_supported(layer, xf))
    if plan == "fused":
        y, ids, wts = moe_fused(xf, layer, top_k, residual, prefetch=prefetch)
        return y.reshape(x.shape), ids, wts
    res = None if residual is None else residual.reshape(-1, hidden)
    if plan == "grouped" and xf.shape[0] * top_k > 16 * layer.n_experts and hidden % 16 == 0:
        # the grouped kernels' prefill form: the top-k launch also writes x'
        ids, wts, xp = router_topk(xf, layer.gate_weight, top_k, bias=layer.router_bias, pairs=True)
        y = moe_grouped(xf, layer, ids, wts, res, x_pairs=xp)
        return y.reshape(x.shape), ids, wts
    ids, wts = router_topk(xf, layer.gate_weight, top_k, bias=layer.router_bias)
    if plan == "grouped":
        y = moe_grouped(xf, layer, ids, wts, res)
    else:
        h = ternary_expert_swiglu(xf, layer.up_gate_packed, layer.up_gate_alpha, ids)
        y = ternary_expert_down_sum(h, layer.down_packed, layer.down_alpha, ids, wts, residual=res,
                                    round_slots=True)
    return y.reshape(x.shape), ids, wts


def moe_layer(hidden: torch.Tensor, layer: MoELayer, top_k: int, norm_weight: torch.Tensor,
              eps: float, add: torch.Tensor | None = None, defer_combine: bool = False):
    """Post-attention half of a decoder layer for ``hidden [T, H]``:
    ``h = hidden + add``, ``y = h + MoE(rms_norm(h) * norm_weight)``.
    Returns ``(y, ids)``.  From GROUPED_MIN_TOKENS tokens the add, norm, router
    and dispatch are one launch (``moe_route``) ahead of the grouped experts;
    there, ``defer_combine`` returns a ``PendingCombine`` in place of ``y``."""
    from .kernels.fused_norm import add_rms_norm, rms_norm
    tokens = hidden.shape[0]
    if (tokens >= GROUPED_MIN_TOKENS and route_supported(layer, top_k, hidden)
            and hidden.shape[-1] % 256 == 0 and layer.inter % 256 == 0):
        h, xn, ids, wts, d, xp = moe_route(hidden, layer, top_k, norm_weight, eps, add=add,
                                           pairs=True)
        return moe_grouped(xn, layer, ids, wts, h, dispatch=d, x_pairs=xp, combine=not defer_combine), ids
    if add is not None:
        h, xn = add_rms_norm(hidden, add, norm_weight, eps)
    else:
        h, xn = hidden, rms_norm(hidden, norm_weight, eps)
    y, ids, _ = moe_block(xn, layer, top_k, residual=h)
    return y, ids


class MapleSparseMoeBlock:
    """Top-k softmax router + fused packed SwitchGLU (``model.py:448-474``)."""

    def __init__(self, gate_weight, up_gate, down, top_k: int, moe_intermediate: int,
                 router_bias: torch.Tensor | None = None):
        self.gate_weight = gate_weight
        self.up_gate = up_gate
        self.down = down
        self.top_k = top_k
        self.moe_intermediate = moe_intermediate
        self.router_bias = router_bias

    def _layer(self) -> MoELayer:
        return MoELayer(self.gate_weight, self.up_gate.packed_weight, self.up_gate.row_alpha,
                        self.down.packed_weight, self.down.row_alpha, self.router_bias)

    def __call__(self, hidden_states: torch.Tensor, residual: torch.Tensor | None = None):
        y, _, _ = moe_block(hidden_states, self._layer(), self.top_k, residual)
        return y
