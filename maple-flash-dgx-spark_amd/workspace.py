"""Device workspaces of the kernels whose workgroups hand data to each other,
and the check of their timeout words.

The single-launch router, the routing launch, the one-launch MoE layer and the
decode attention keep cross-workgroup state in a zero-filled workspace: tagged
values, call counters, barrier counters and flags that each call leaves ready
for the next, so the workspace is zeroed once and never again.  Two calls on
one workspace must therefore not overlap.  Workspaces here are keyed by
(kind, device, stream, shape): calls issued on different streams use different
workspaces, and calls on one stream are ordered by it.
A HIP graph keeps the workspace of the stream it was captured on; replay it
in that stream's order relative to eager calls made on the capture stream.
(The attention workspace belongs to its KV cache, ``gqa_workspace``.)
The pool also holds per-call scratch that a kernel rewrites on every call (the
RTN4 GEMM's operands); it carries no timeout word and is never zeroed here.

A workspace that has to grow is replaced by a larger one (at least twice the
size, so the replaced ones add up to less than the current one), and the one
it replaces is retired, not freed: a graph captured while it was current
still writes into it on every replay, and stream handles are reused (torch
hands them out from a fixed pool), so a later capture or eager call on the
same handle at a larger size must not hand that memory back to the caching
allocator.  Retired workspaces stay in the timeout check.

Persistent launches (the one-launch MoE layer, the routing launch, the
single-launch router and the decode attention) assume that their whole grid
is resident at once, checked against the whole device.  Two of them must not
overlap on one GPU, even on different streams: their grids could then not all
fit, and the waits would run out (wrong values, reported by the timeout
check).  Issue them from one stream per device, or order the streams.

Every wait in those kernels is bounded (about 0.2 s; in the XCD-split
one-launch MoE layer 200 us after the launch's start); a wait that runs out
sets the workspace's timeout word and the kernel finishes with wrong values
instead of hanging.  The XCD-split layer also checks, in a call that ran out,
whether its workgroups were spread over the XCDs as it assumes; if not, the
timeout check turns the XCD-split forms off on that device (the hook the
MoE module registers with ``on_timeout``).  ``check_timeouts`` reads every timeout word of a device
in one copy (a host synchronisation) and raises ``RuntimeError`` if any is
set, after zeroing the workspaces again so that later calls start clean.
The decode loop (``generate.py``) calls it where it already synchronises.
"""

from __future__ import annotations

import weakref

import torch

# uint32 index of the timeout word in each kind of workspace
TIMEOUT_WORD = {
    "router": 1,      # ma_router_topk's single-launch decode router
    "moe_fused": 2,   # ma_moe_fused
    "moe_route": 64,  # ma_moe_route
    "attention": 2,   # ma_decode_attn_fused / ma_decode_gqa_attn (sync area, line 0)
}

# kind -> fn(workspaces of that kind on the device, device index) -> note or
# None: run by check_timeouts on a timed-out kind before the re-zeroing
# (the MoE layer's checks its layout word there)
_ON_TIMEOUT: dict = {}

_POOL: dict[tuple, torch.Tensor] = {}
# (key, tensor) of workspaces replaced by larger ones; kept until the process ends
_RETIRED: list[tuple[tuple, torch.Tensor]] = []
_ATTENTION: "weakref.WeakValueDictionary[int, torch.Tensor]" = weakref.WeakValueDictionary()


def _device_index(device) -> int:
    device = torch.device(device)
    return device.index if device.index is not None else torch.cuda.current_device()


def get(kind: str, device, nbytes: int, key: tuple = (), *, min_bytes: int = 0) -> torch.Tensor:
    """The zero-filled workspace of ``kind`` for ``key`` on ``device`` and its
    current stream (created, or grown, on first need; a grown workspace
    retires the one it replaces instead of freeing it)."""
    idx = _device_index(device)
    stream = torch.cuda.current_stream(idx).cuda_stream
    k = (kind, idx, stream) + tuple(key)
    ws = _POOL.get(k)
    if ws is None or ws.numel() < nbytes:
        size = max(int(nbytes), int(min_bytes))
        if ws is not None:
            size = max(size, 2 * ws.numel())
            _RETIRED.append((k, ws))
        ws = _alloc(size, idx)
        _POOL[k] = ws
    return ws


def _alloc(nbytes: int, idx: int) -> torch.Tensor:
    return torch.zeros(nbytes, device=torch.device("cuda", idx), dtype=torch.uint8)


def register_attention(ws: torch.Tensor) -> torch.Tensor:
    """Track an attention workspace (one per KV cache) for ``check_timeouts``."""
    _ATTENTION[id(ws)] = ws
    return ws


def _all(idx: int) -> list[tuple[str, torch.Tensor]]:
    """The workspaces on device ``idx`` that carry a timeout word (per-call
    scratch kept in the pool, such as the RTN4 GEMM's operands, has none)."""
    out = [(k[0], ws) for k, ws in list(_POOL.items()) + _RETIRED if k[1] == idx and k[0] in TIMEOUT_WORD]
    out += [("attention", ws) for ws in list(_ATTENTION.values()) if ws.device.index == idx]
    return out


def timed_out_kinds(device=None) -> list[str]:
    """Kinds of workspace on ``device`` whose timeout word is set.  One small
    device gather and one copy to the host (synchronises)."""
    idx = _device_index(device if device is not None else torch.cuda.current_device())
    wss = _all(idx)
    if not wss:
        return []
    words = torch.stack([ws.view(torch.int32)[TIMEOUT_WORD[kind]] for kind, ws in wss]).cpu()
    return sorted({kind for (kind, _), w in zip(wss, words.tolist()) if w != 0})


def check_timeouts(device=None) -> None:
    """Raise ``RuntimeError`` if any cross-workgroup wait on ``device`` timed
    out since the workspaces were zeroed; zero them again first."""
    kinds = timed_out_kinds(device)
    if kinds:
        idx = _device_index(device if device is not None else torch.cuda.current_device())
        notes = []
        for kind in kinds:
            hook = _ON_TIMEOUT.get(kind)
            if hook is not None:
                note = hook([ws for k, ws in _all(idx) if k == kind], idx)
                if note:
                    notes.append(note)
        for _, ws in _all(idx):
            ws.zero_()
        raise RuntimeError(
            "a cross-workgroup wait timed out in " + ", ".join(kinds)
            + "; the results of the calls since the last check are invalid "
            "(workspaces have been zeroed again)" + "".join("; " + n for n in notes))


def on_timeout(kind: str, fn) -> None:
    """Register ``fn(workspaces, device_index) -> note | None``, run by
    ``check_timeouts`` when ``kind`` timed out, before the re-zeroing."""
    _ON_TIMEOUT[kind] = fn
