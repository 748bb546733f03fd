"""Choice of the persistent kernels and the timeout check (CPU; no kernel runs).

The one-launch MoE layer's workgroups meet at a grid barrier, so it runs only
where its whole grid is resident at once.  With the device's capacity
stubbed below the grid (a partitioned GPU, say), ``fused_supported`` is false
and ``moe_block``'s plan falls back to the multi-launch per-slot kernels; the
decoder takes the same query.  ``check_timeouts`` raises once a timeout word
is set and zeroes the workspaces again.
"""

from __future__ import annotations

import pytest
import torch

from maple_amd import moe, synthetic, workspace


def _layer(hidden=2048, experts=64, inter=768):
    kw = hidden // 16
    return synthetic.MoELayer(
        torch.zeros(experts, hidden, dtype=torch.bfloat16),
        torch.zeros(experts, 2 * inter, kw, dtype=torch.int32).view(torch.uint32),
        torch.zeros(experts, 2 * inter, dtype=torch.bfloat16),
        torch.zeros(experts, hidden, inter // 16, dtype=torch.int32).view(torch.uint32),
        torch.zeros(experts, hidden, dtype=torch.bfloat16))


class _StubLib:
    """Stands in for the library's residency query with a given capacity."""

    def __init__(self, real, capacity):
        self.real, self.capacity = real, capacity

    def __getattr__(self, name):
        return getattr(self.real, name)

    def ma_moe_fused_resident(self, e, h, i, k, needed, capacity):
        needed._obj.value = 256 if h == 2048 else 32
        capacity._obj.value = self.capacity
        return 0


class _NullCtx:
    def __enter__(self):
        return self

    def __exit__(self, *a):
        return False


@pytest.mark.parametrize("capacity, expect", [(512, "fused"), (256, "fused"), (255, "per_slot"),
                                              (32, "per_slot")])
def test_fused_plan_needs_the_whole_grid_resident(monkeypatch, capacity, expect):
    stub = _StubLib(moe._lib.load(), capacity)
    monkeypatch.setattr(moe._lib, "load", lambda: stub)
    monkeypatch.setattr(moe, "_RESIDENT", {})
    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)
    monkeypatch.setattr(torch.cuda, "device", lambda idx: _NullCtx())
    layer = _layer()
    x = torch.zeros(1, 2048, dtype=torch.bfloat16)
    ok = moe.fused_supported(layer, 8, x)
    assert ok == (capacity >= 256)
    assert moe.choose_plan(1, ok, True) == expect


def test_plan_by_token_count():
    assert moe.choose_plan(1, True, True) == "fused"
    assert moe.choose_plan(2, True, True) == "per_slot"
    assert moe.choose_plan(moe.GROUPED_MIN_TOKENS, True, True) == "grouped"
    assert moe.choose_plan(64, True, False) == "per_slot"
    assert moe.choose_plan(1, False, True) == "per_slot"


def test_fused_supported_rejects_unbuilt_shapes_and_dtypes():
    x = torch.zeros(1, 2048, dtype=torch.bfloat16)
    assert not moe.fused_supported(_layer(inter=640), 8, x)  # shape not built: no device query
    assert not moe.fused_supported(_layer(), 8, x.float())


def test_check_timeouts_raises_and_rezeroes(monkeypatch):
    """The timeout words are read from every workspace of the device; a set
    word raises RuntimeError and the workspaces are zeroed again."""
    a = torch.zeros(1024, dtype=torch.uint8)
    b = torch.zeros(1024, dtype=torch.uint8)
    b[300] = 7  # state a kernel left (a tag), not a timeout
    pool = {("moe_fused", 0, 1, 2048): a, ("moe_route", 0, 1, 64): b}
    monkeypatch.setattr(workspace, "_POOL", pool)
    monkeypatch.setattr(workspace, "_ATTENTION", {})
    monkeypatch.setattr(workspace, "_device_index", lambda d: 0)
    assert workspace.timed_out_kinds(0) == []
    workspace.check_timeouts(0)  # nothing set: no error
    a.view(torch.int32)[workspace.TIMEOUT_WORD["moe_fused"]] = 1
    assert workspace.timed_out_kinds(0) == ["moe_fused"]
    with pytest.raises(RuntimeError, match="moe_fused"):
        workspace.check_timeouts(0)
    assert int(a.count_nonzero()) == 0 and int(b.count_nonzero()) == 0
    workspace.check_timeouts(0)


def test_check_timeouts_skips_pooled_scratch(monkeypatch):
    """Per-call scratch kept in the pool (the RTN4 GEMM's operands) has no
    timeout word: its contents are never read as one and are left alone."""
    a = torch.zeros(1024, dtype=torch.uint8)
    s = torch.full((1024,), 255, dtype=torch.uint8)
    pool = {("moe_fused", 0, 1, 2048): a, ("rtn4", 0, 1, 256, 64): s}
    monkeypatch.setattr(workspace, "_POOL", pool)
    monkeypatch.setattr(workspace, "_ATTENTION", {})
    monkeypatch.setattr(workspace, "_device_index", lambda d: 0)
    assert workspace.timed_out_kinds(0) == []
    a.view(torch.int32)[workspace.TIMEOUT_WORD["moe_fused"]] = 1
    with pytest.raises(RuntimeError, match="moe_fused"):
        workspace.check_timeouts(0)
    assert int(a.count_nonzero()) == 0 and bool((s == 255).all())


class _Stream:
    cuda_stream = 7  # one reused stream handle


def test_grown_workspace_is_retired_not_freed(monkeypatch):
    """A graph captured against a workspace keeps writing into it on every
    replay; a later call on the same (reused) stream handle that needs more
    room gets a new, larger tensor while the old one stays referenced (and
    in the timeout check)."""
    monkeypatch.setattr(workspace, "_POOL", {})
    monkeypatch.setattr(workspace, "_RETIRED", [])
    monkeypatch.setattr(workspace, "_ATTENTION", {})
    monkeypatch.setattr(workspace, "_device_index", lambda d: 0)
    monkeypatch.setattr(torch.cuda, "current_stream", lambda idx=None: _Stream())
    monkeypatch.setattr(workspace, "_alloc", lambda n, idx: torch.zeros(n, dtype=torch.uint8))
    first = workspace.get("router", 0, 4096)
    assert workspace.get("router", 0, 1000) is first  # fits: same tensor
    grown = workspace.get("router", 0, 5000)
    assert grown is not first and grown.numel() >= 2 * first.numel()
    assert any(t is first for _, t in workspace._RETIRED)
    # the retired workspace is still read by the timeout check
    first.view(torch.int32)[workspace.TIMEOUT_WORD["router"]] = 1
    assert workspace.timed_out_kinds(0) == ["router"]
    with pytest.raises(RuntimeError, match="router"):
        workspace.check_timeouts(0)
    assert int(first.count_nonzero()) == 0
    # growth is geometric, so retired bytes stay below the current size
    for n in range(5001, 40000, 3001):
        workspace.get("router", 0, n)
    cur = workspace._POOL[("router", 0, 7)].numel()
    assert sum(t.numel() for _, t in workspace._RETIRED) < cur


class _DisableRecorder:
    """Stands in for the library: records ma_xcd_forms_disable calls."""

    def __init__(self, real):
        self.real, self.calls = real, []

    def __getattr__(self, name):
        return getattr(self.real, name)

    def ma_xcd_forms_disable(self, device, disable):
        self.calls.append((device, disable))
        return 0


@pytest.mark.parametrize("layout_bad", [False, True])
def test_layout_check_turns_the_xcd_forms_off(monkeypatch, layout_bad):
    """A timed-out one-launch workspace whose layout word is set (the XCD
    form found two workgroups with one number on an XCD and aborted the
    call) makes check_timeouts turn the XCD-split forms off on that device
    and say so; a plain timeout leaves them on."""
    stub = _DisableRecorder(moe._lib.load())
    monkeypatch.setattr(moe._lib, "load", lambda: stub)
    a = torch.zeros(4096, dtype=torch.uint8)
    a.view(torch.int32)[workspace.TIMEOUT_WORD["moe_fused"]] = 1
    if layout_bad:
        a.view(torch.int32)[moe.LAYOUT_WORD] = 1
    monkeypatch.setattr(workspace, "_POOL", {("moe_fused", 0, 1, 2048): a})
    monkeypatch.setattr(workspace, "_RETIRED", [])
    monkeypatch.setattr(workspace, "_ATTENTION", {})
    monkeypatch.setattr(workspace, "_device_index", lambda d: 0)
    with pytest.raises(RuntimeError, match="XCD-split forms are now off" if layout_bad else "moe_fused") as ei:
        workspace.check_timeouts(0)
    assert stub.calls == ([(0, 1)] if layout_bad else [])
    assert layout_bad or "XCD-split" not in str(ei.value)
    assert int(a.count_nonzero()) == 0  # zeroed again
