"""Host logic of the decode-graph runner (CPU): settings, buckets, slots."""

from __future__ import annotations

import pytest
import torch

from maple_amd.decode_graph import (BucketedDecodeGraphs, Sampling, can_fuse_sampler, decode_buckets,
                                    is_greedy)
from maple_amd.model import KVCache


def test_greedy_and_fusable_settings():
    assert is_greedy(0.0, 20) and is_greedy(-1.0, 0) and is_greedy(0.7, 1)
    assert not is_greedy(0.7, 20)
    assert can_fuse_sampler(1.0, 0.95, 20)
    assert not can_fuse_sampler(0.0, 0.95, 20)
    assert not can_fuse_sampler(1.0, 0.95, 1)
    assert not can_fuse_sampler(1.0, 0.95, 0)
    assert not can_fuse_sampler(1.0, 0.95, 65)
    assert not can_fuse_sampler(1.0, 0.0, 20)
    Sampling().check()
    Sampling(temperature=0.8, top_p=0.9, top_k=40).check()
    for bad in (Sampling(temperature=0.8, top_k=0), Sampling(temperature=0.8, top_k=65),
                Sampling(temperature=0.8, top_p=1.5, top_k=8)):
        with pytest.raises(ValueError):
            bad.check()


def test_decode_buckets():
    assert decode_buckets(1) == (1,)
    assert decode_buckets(5) == (1, 2, 4, 5)
    assert decode_buckets(32) == (1, 2, 4, 8, 16, 32)
    assert decode_buckets(48) == (1, 2, 4, 8, 16, 32, 48)
    for n in range(1, 300):
        w = decode_buckets(n)
        assert w[-1] == n
        for live in range(1, n + 1):  # always a width within 2x of the live rows
            fit = min(x for x in w if x >= live)
            assert fit < 2 * live or fit == 1


def _cache(rows=4, max_len=16):
    k = [torch.zeros(rows, 2, max_len, 8) for _ in range(2)]
    v = [torch.zeros(rows, 2, max_len, 8) for _ in range(2)]
    return KVCache(k, v, torch.full((rows,), 5, dtype=torch.int64), max_len)


def test_slot_map_and_swaps():
    c = _cache()
    assert c.row_map.tolist() == [0, 1, 2, 3] and not c.remap
    sl, rm = c.slot_rows(4)
    assert rm is None and sl.data_ptr() == c.seqlen.data_ptr()
    sl, rm = c.slot_rows(2)
    assert rm.tolist() == [0, 1] and sl.numel() == 2
    with pytest.raises(ValueError):
        c.slot_rows(5)
    with pytest.raises(RuntimeError):
        c.swap_slots(0, 3)
    c.remap = True
    c.seqlen[3] = 9
    c.swap_slots(0, 3)
    assert c.row_map.tolist() == [3, 1, 2, 0] and c.seqlen.tolist() == [9, 5, 5, 5]
    assert c.slot_rows(4)[1].tolist() == [3, 1, 2, 0]
    c.reset_slot(0)
    assert c.seqlen.tolist() == [0, 5, 5, 5]


def test_snapshot_restores_the_span_it_saved():
    c = _cache()
    c.seqlen.copy_(torch.tensor([3, 5, 4, 6]))
    for t in c.k + c.v:
        t.normal_()
    ref = [t.clone() for t in c.k + c.v]
    snap = c.snapshot(steps=2)
    assert snap["span"] == (3, 9)
    for t in c.k + c.v:
        t[:, :, 3:9] = 7.0
    c.seqlen.add_(2)
    c.remap = True
    c.row_map.copy_(torch.tensor([1, 0, 2, 3]))
    c.restore(snap)
    assert c.seqlen.tolist() == [3, 5, 4, 6] and c.row_map.tolist() == [0, 1, 2, 3] and not c.remap
    for a, b in zip(c.k + c.v, ref):
        assert torch.equal(a, b)
    full = c.snapshot()
    assert full["span"] == (0, 16)


def test_bucketed_graphs_need_the_slot_map():
    with pytest.raises(ValueError, match="remap"):
        BucketedDecodeGraphs(None, _cache(), widths=(1, 2))
