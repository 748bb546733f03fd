"""Decode-graph runner on the GPU (maple_amd.decode_graph): the equality gate
keeps a graph whose replays choose the eager ids, rejects one that diverges
or fails to capture, restores the cache either way; graph and eager decoding
give the same ids, greedy and sampled; bucketed graphs replay at the
narrowest width and follow the slot map.  Reference behaviour:
src/maple_run/generate.py:168-373, 687-816."""

from __future__ import annotations

import pytest
import torch

from maple_amd.decode_graph import (BucketedDecodeGraphs, Sampling, decode_buckets, generate,
                                    try_decode_graph)
from maple_amd.kernels.greedy import greedy_argmax
from maple_amd.model import DecoderConfig, SyntheticDecoder

pytestmark = pytest.mark.gpu

SMALL = DecoderConfig(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64, experts=8, inter=256,
                      top_k=2, vocab=1024, rtn_group=128, lm_scale=(0.01, 0.02))


def _setup(dev, batch, seed=3, prefill=20):
    model = SyntheticDecoder(SMALL, dev, seed=seed, max_len=128)
    cache = model.make_cache(batch, prefill_len=prefill, seed=1)
    first = torch.arange(batch, device=dev, dtype=torch.int64) * 37 + 5
    return model, cache, first


def _state(cache):
    return cache.seqlen.clone(), [t.clone() for t in cache.k], [t.clone() for t in cache.v]


def _same_state(cache, st):
    return (torch.equal(cache.seqlen, st[0]) and all(torch.equal(a, b) for a, b in zip(cache.k, st[1]))
            and all(torch.equal(a, b) for a, b in zip(cache.v, st[2])))


@pytest.mark.parametrize("batch", [1, 3, 20])
def test_gate_keeps_the_graph_and_restores_the_cache(dev, batch):
    model, cache, first = _setup(dev, batch)
    st = _state(cache)
    logs = []
    g = try_decode_graph(model, cache, first, log=logs.append)
    assert g is not None, logs
    assert "matches eager" in logs[-1]
    assert _same_state(cache, st)


@pytest.mark.parametrize("batch", [1, 3, 20])
def test_graph_and_eager_generate_the_same_ids(dev, batch):
    model, c1, first = _setup(dev, batch)
    _, c2, _ = _setup(dev, batch)
    a = generate(model, c1, first, 12, use_graph=True)
    b = generate(model, c2, first, 12, use_graph=False)
    assert a.used_graph and not b.used_graph
    assert a.token_ids == b.token_ids
    assert torch.equal(c1.seqlen, c2.seqlen) and int(c1.seqlen[0]) == 20 + 12
    for x, y in zip(c1.k + c1.v, c2.k + c2.v):
        assert torch.equal(x, y)


def test_sampled_generate_is_seeded_and_graph_equals_eager(dev):
    model, c1, first = _setup(dev, 4)
    _, c2, _ = _setup(dev, 4)
    _, c3, _ = _setup(dev, 4)
    mk = lambda: Sampling(temperature=0.9, top_p=0.9, top_k=20,  # noqa: E731
                          generator=torch.Generator(device=dev).manual_seed(11))
    a = generate(model, c1, first, 10, mk(), use_graph=True)
    b = generate(model, c2, first, 10, mk(), use_graph=False)
    c = generate(model, c3, first, 10, Sampling(temperature=0.9, top_p=0.9, top_k=20,
                                               generator=torch.Generator(device=dev).manual_seed(12)),
                 use_graph=False)
    assert a.used_graph
    assert a.token_ids == b.token_ids
    assert a.token_ids != c.token_ids  # another seed draws other ids


def test_stop_ids_cut_rows(dev):
    model, cache, first = _setup(dev, 2)
    free = generate(model, cache, first, 16, use_graph=False)
    stop = free.token_ids[0][5]
    model, cache, first = _setup(dev, 2)
    r = generate(model, cache, first, 16, stop_ids=[stop], check_every=4)
    assert r.token_ids[0] == free.token_ids[0][:free.token_ids[0].index(stop) + 1]
    assert r.finish_reasons[0] == "stop"


class _HostCounterModel:
    """Adds a one-hot logit bias chosen by a host-side counter: eager steps
    move it, a graph replays the bias baked in at capture, so the ids differ."""

    def __init__(self, inner):
        self.inner, self.cfg, self.n = inner, inner.cfg, 0

    def forward(self, ids, cache):
        logits = self.inner.forward(ids, cache)
        self.n += 1
        bias = torch.zeros(self.cfg.vocab, device=logits.device, dtype=logits.dtype)
        bias.narrow(0, (self.n * 7) % self.cfg.vocab, 1).fill_(100.0)  # a fill kernel: capturable
        return logits + bias


class _NoCaptureModel(_HostCounterModel):
    """Raises inside capture, as a step that needs the host would."""

    def forward(self, ids, cache):
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("this step reads a value on the host")
        return self.inner.forward(ids, cache)


def test_gate_rejects_a_diverging_graph(dev):
    model, cache, first = _setup(dev, 2)
    st = _state(cache)
    logs = []
    assert try_decode_graph(_HostCounterModel(model), cache, first, log=logs.append) is None
    assert "diverged" in logs[-1]
    assert _same_state(cache, st)
    r = generate(_HostCounterModel(model), cache, first, 4, log=logs.append)
    assert not r.used_graph and len(r.token_ids[0]) == 4


def test_gate_survives_a_failed_capture(dev):
    model, cache, first = _setup(dev, 1)
    st = _state(cache)
    logs = []
    assert try_decode_graph(_NoCaptureModel(model), cache, first, log=logs.append) is None
    assert "capture failed" in logs[-1]
    assert _same_state(cache, st)
    torch.cuda.synchronize()


def test_bucketed_graphs_replay_at_the_narrowest_width(dev):
    batch = 5
    model, cache, first = _setup(dev, batch)
    cache.remap = True
    st = _state(cache)
    widths = decode_buckets(batch)
    bg = BucketedDecodeGraphs(model, cache, widths=widths, log=lambda m: None)
    assert bg.widths == (1, 2, 4, 5) and _same_state(cache, st)
    # live = 3 replays the width-4 graph: slots 0-2 match an eager width-4 step with the same padding
    _, ref_cache, _ = _setup(dev, batch)
    ref_cache.remap = True
    ids = bg.replay(first[:3])
    torch.cuda.synchronize()
    padded = torch.cat([first[:3], torch.zeros(1, device=dev, dtype=torch.int64)])
    want = greedy_argmax(model.forward(padded, ref_cache))[:3]
    assert bg.width_for(3) == 4
    assert torch.equal(ids, want)
    assert cache.seqlen.tolist() == [21, 21, 21, 21, 20]
    # a swap moves slot 0's sequence to row 4; the replay reads row 4's K/V
    cache.restore({"seqlen": st[0], "row_map": torch.arange(batch, device=dev), "remap": True,
                   "span": (0, cache.max_len), "k": st[1], "v": st[2]})
    ref_cache.restore({"seqlen": st[0], "row_map": torch.arange(batch, device=dev), "remap": True,
                       "span": (0, cache.max_len), "k": st[1], "v": st[2]})
    cache.swap_slots(0, 4)
    ref_cache.swap_slots(0, 4)
    lg = bg.replay_logits(first[:2]).clone()
    want = model.forward(first[:2], ref_cache)
    assert torch.equal(lg, want)
    assert cache.row_map.tolist() == [4, 1, 2, 3, 0]
