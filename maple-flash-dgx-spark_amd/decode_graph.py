"""Whole-step decode graphs with an eager-equality gate, and the decode loop.

Mirrors the decode drivers of reference ``src/maple_run/generate.py``:

* ``is_greedy`` / ``can_fuse_sampler`` (:64-76);
* ``capture_decode_graph`` (``_capture_decode_graph`` :168-227): warm-up on a
  side stream, then one HIP graph of the whole step -- embedding, every
  layer, the head and the token choice (greedy argmax, or the fused sampler
  reading its uniforms from a buffer) -- which also feeds the chosen ids back
  as the next step's input;
* ``try_decode_graph`` (``_try_decode_graph`` :284-373): snapshot the cache,
  capture, decode ``GRAPH_CHECK_TOKENS`` steps eagerly and the same steps by
  replay from the same cache state and random-number state, keep the graph
  only if the ids agree, else log why and return None (decode stays eager);
* ``decode_buckets`` / ``BucketedDecodeGraphs`` (:687-816): one graph per
  batch width over shared input buffers, replayed at the narrowest width
  that holds the live rows (live sequences kept in the low slots through the
  cache's slot map);
* ``generate``: the decode loop of ``run_generate`` (:1107-1281) without
  tokenizer and chat handling: graph when it validates, eager otherwise, ids
  gathered on the device, one host synchronisation at the end (or every
  ``check_every`` steps when stop ids are given), and the persistent kernels'
  timeout words checked there.

Sampling randomness stays with the caller's generator: each step draws one
uniform per row with ``torch.rand(rows, generator=...)`` on the device, eager
and replay alike, so a seeded run is reproducible and the equality gate
compares like with like.  Settings the fused sampler does not cover
(``top_k`` of 0 or above 64 while sampling) raise ``ValueError``.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Callable

import torch

from . import workspace
from .kernels.greedy import greedy_argmax
from .kernels.sampler import MAX_TOP_K, batched_sampler_workspace, fused_sample_batched

GRAPH_WARMUP = 3
GRAPH_CHECK_TOKENS = 8
DECODE_BUCKETS = (1, 2, 4, 8, 16, 32, 64, 128, 256)


def _log_print(msg: str) -> None:
    print(msg, flush=True)


def is_greedy(temperature: float, top_k: int) -> bool:
    """True when the next token is the argmax."""
    return temperature <= 0.0 or top_k == 1


def can_fuse_sampler(temperature: float, top_p: float, top_k: int) -> bool:
    """Whether the fused sampler covers these settings."""
    return not is_greedy(temperature, top_k) and 0 < top_k <= MAX_TOP_K and 0.0 < top_p <= 1.0


@dataclass
class Sampling:
    """Token choice of a decode run: greedy, or the fused top-k / temperature
    / nucleus draw with one uniform per row from ``generator``."""

    temperature: float = 0.0
    top_p: float = 1.0
    top_k: int = 0
    generator: torch.Generator | None = None

    @property
    def greedy(self) -> bool:
        return is_greedy(self.temperature, self.top_k)

    def check(self) -> None:
        if not self.greedy and not can_fuse_sampler(self.temperature, self.top_p, self.top_k):
            raise ValueError(
                f"sampling needs 0 < top_k <= {MAX_TOP_K} and 0 < top_p <= 1 (got top_k={self.top_k}, "
                f"top_p={self.top_p}); greedy decoding needs temperature <= 0 or top_k == 1.")

    def draw(self, rows: int, device) -> torch.Tensor:
        return torch.rand(rows, device=device, generator=self.generator)


def _rng_snapshot(device: torch.device, generator: torch.Generator | None):
    idx = device.index if device.index is not None else torch.cuda.current_device()
    default = torch.cuda.default_generators[idx].get_state()
    return default, (generator.get_state() if generator is not None else None)


def _rng_restore(device: torch.device, snap, generator: torch.Generator | None) -> None:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    torch.cuda.default_generators[idx].set_state(snap[0])
    if generator is not None and snap[1] is not None:
        generator.set_state(snap[1])


@dataclass
class DecodeGraph:
    """A captured decode step: write ``token_ids`` (and ``uniform`` when
    sampling), replay, read ``next_id``; the replay has already copied
    ``next_id`` into ``token_ids`` for the following step."""

    graph: torch.cuda.CUDAGraph
    token_ids: torch.Tensor
    logits: torch.Tensor
    next_id: torch.Tensor
    uniform: torch.Tensor | None = None
    feed: bool = True
    # Buffers the replay reads or writes that were allocated outside the
    # graph's own memory pool: held here so they outlive the capture.
    workspace: torch.Tensor | None = None

    def step(self, sampling: Sampling) -> torch.Tensor:
        if self.uniform is not None:
            self.uniform.copy_(sampling.draw(self.uniform.numel(), self.uniform.device))
        self.graph.replay()
        return self.next_id


def _choose(logits: torch.Tensor, sampling: Sampling, out: torch.Tensor, uniform: torch.Tensor | None,
            ws) -> torch.Tensor:
    if sampling.greedy:
        return greedy_argmax(logits, out=out)
    nxt = fused_sample_batched(logits, uniform, temperature=sampling.temperature, top_p=sampling.top_p,
                               top_k=sampling.top_k, workspace=(ws, out))
    return nxt


def capture_decode_graph(model, cache, token_ids: torch.Tensor, sampling: Sampling,
                         feed: bool = True) -> DecodeGraph:
    """Capture one whole decode step over slots ``[0, len(token_ids))``.
    Runs ``GRAPH_WARMUP`` eager steps first (they advance the cache: restore
    it afterwards)."""
    sampling.check()
    dev = token_ids.device
    rows = int(token_ids.numel())
    next_id = torch.zeros(rows, device=dev, dtype=torch.int64)
    uniform = ws = None
    if not sampling.greedy:
        uniform = torch.zeros(rows, device=dev, dtype=torch.float32)
        ws = batched_sampler_workspace(model.cfg.vocab, sampling.top_k, rows, dev)[0]

    def body():
        logits = model.forward(token_ids, cache)
        _choose(logits, sampling, next_id, uniform, ws)
        if feed:
            token_ids.copy_(next_id)
        return logits

    stream = torch.cuda.Stream(device=dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    saved = token_ids.clone()
    with torch.cuda.stream(stream):
        for _ in range(GRAPH_WARMUP):
            token_ids.copy_(saved)
            body()
        token_ids.copy_(saved)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            logits = body()
    torch.cuda.current_stream(dev).wait_stream(stream)
    token_ids.copy_(saved)
    return DecodeGraph(graph=graph, token_ids=token_ids, logits=logits, next_id=next_id, uniform=uniform,
                       feed=feed, workspace=ws)


def _eager_ids(model, cache, first: torch.Tensor, n: int, sampling: Sampling) -> list:
    ids, tok = [], first.clone()
    out = torch.empty_like(tok)
    ws = None
    if not sampling.greedy:
        ws = batched_sampler_workspace(model.cfg.vocab, sampling.top_k, int(tok.numel()), tok.device)[0]
    for _ in range(n):
        u = None if sampling.greedy else sampling.draw(int(tok.numel()), tok.device)
        logits = model.forward(tok, cache)
        _choose(logits, sampling, out, u, ws)
        tok.copy_(out)
        ids.append(out.clone())
    return torch.stack(ids).cpu().tolist()


def _graph_ids(g: DecodeGraph, first: torch.Tensor, n: int, sampling: Sampling) -> list:
    g.token_ids.copy_(first)
    ids = []
    for _ in range(n):
        ids.append(g.step(sampling).clone())
        if not g.feed:
            g.token_ids.copy_(g.next_id)
    return torch.stack(ids).cpu().tolist()


def try_decode_graph(model, cache, first_ids: torch.Tensor, sampling: Sampling | None = None, *,
                     n_check: int = GRAPH_CHECK_TOKENS,
                     log: Callable[[str], None] = _log_print) -> DecodeGraph | None:
    """Capture the decode step and keep it only if ``n_check`` replayed steps
    choose the same ids as ``n_check`` eager steps from the same cache and
    random state.  The cache and the random state are restored either way."""
    sampling = sampling or Sampling()
    sampling.check()
    dev = first_ids.device
    first = first_ids.reshape(-1).to(torch.int64)
    snap = cache.snapshot(steps=max(GRAPH_WARMUP, n_check) + 1)
    token_ids = first.clone()
    try:
        captured = capture_decode_graph(model, cache, token_ids, sampling)
    except Exception as exc:  # capture is an optimisation: eager decode still works
        cache.restore(snap)
        log(f"HIP graph capture failed ({exc}); using eager decode")
        return None
    cache.restore(snap)
    rng = _rng_snapshot(dev, sampling.generator)
    eager = _eager_ids(model, cache, first, n_check, sampling)
    cache.restore(snap)
    _rng_restore(dev, rng, sampling.generator)
    replay = _graph_ids(captured, first, n_check, sampling)
    cache.restore(snap)
    _rng_restore(dev, rng, sampling.generator)
    workspace.check_timeouts(dev)
    if eager != replay:
        log(f"HIP graph replay diverged (eager {eager[:4]} vs graph {replay[:4]}); using eager decode")
        return None
    log("HIP graph decode: replay matches eager ids")
    captured.token_ids.copy_(first)
    return captured


def decode_buckets(max_batch: int, buckets=DECODE_BUCKETS) -> tuple:
    """Graph widths for a cache of ``max_batch`` slots: the bucket sizes below
    it plus ``max_batch`` itself, so a shrinking batch always has a graph
    within 2x of its live width."""
    widths = [w for w in buckets if w < max_batch]
    widths.append(int(max_batch))
    return tuple(sorted(set(widths)))


class BucketedDecodeGraphs:
    """One captured decode step per width over shared token / uniform
    buffers, replayed at the narrowest width holding the live rows.  Rows
    past the live count are padding: they decode into the slots above the
    live ones, so the caller keeps live sequences in the low slots
    (``KVCache.swap_slots``), which needs ``cache.remap``."""

    def __init__(self, model, cache, *, widths: tuple, sampling: Sampling | None = None,
                 log: Callable[[str], None] = _log_print):
        if not cache.remap:
            raise ValueError("BucketedDecodeGraphs needs cache.remap enabled.")
        self.sampling = sampling or Sampling()
        self.sampling.check()
        dev = cache.seqlen.device
        self.widths = tuple(sorted(int(w) for w in widths))
        self.max_width = self.widths[-1]
        if self.max_width > cache.rows:
            raise ValueError(f"widest graph {self.max_width} exceeds the cache's {cache.rows} slots.")
        self.token_ids = torch.zeros(self.max_width, device=dev, dtype=torch.int64)
        self.graphs: dict = {}
        snap = cache.snapshot(steps=GRAPH_WARMUP + 1)
        try:
            for w in self.widths:
                g = capture_decode_graph(model, cache, self.token_ids[:w], self.sampling, feed=False)
                cache.restore(snap)
                self.graphs[w] = g
        finally:
            cache.restore(snap)
        log(f"Bucketed decode graphs: widths {list(self.widths)}"
            + (" greedy" if self.sampling.greedy else " with the fused sampler"))

    def width_for(self, live: int) -> int:
        for w in self.widths:
            if w >= live:
                return w
        raise ValueError(f"live batch {live} exceeds widest graph {self.max_width}.")

    def _run(self, tokens: torch.Tensor, uniform: torch.Tensor | None) -> tuple:
        live = int(tokens.numel())
        w = self.width_for(live)
        self.token_ids[:live].copy_(tokens.reshape(-1))
        if live < w:
            self.token_ids[live:w].zero_()
        g = self.graphs[w]
        if g.uniform is not None:
            g.uniform.copy_(self.sampling.draw(w, g.uniform.device) if uniform is None
                            else torch.cat([uniform.reshape(-1)[:live].float(),
                                            g.uniform.new_zeros(w - live)]))
        g.graph.replay()
        return g, live

    def replay(self, tokens: torch.Tensor, uniform: torch.Tensor | None = None) -> torch.Tensor:
        """Step ``tokens [live]``; returns the next ids ``[live]``."""
        g, live = self._run(tokens, uniform)
        return g.next_id[:live]

    def replay_logits(self, tokens: torch.Tensor) -> torch.Tensor:
        """Step ``tokens [live]``; returns the logits ``[live, vocab]``."""
        g, live = self._run(tokens, None)
        return g.logits[:live]


@dataclass
class GenerateResult:
    """Ids per row (cut after the first stop id), why each row ended and
    the decode timing."""

    token_ids: list
    finish_reasons: list
    steps: int
    decode_s: float
    used_graph: bool
    log: list = field(default_factory=list)

    @property
    def tokens_per_s(self) -> float:
        return sum(len(r) for r in self.token_ids) / self.decode_s if self.decode_s > 0 else 0.0


def generate(model, cache, first_ids: torch.Tensor, max_new_tokens: int, sampling: Sampling | None = None,
             *, use_graph: bool = True, stop_ids=(), check_every: int = 8,
             log: Callable[[str], None] | None = None) -> GenerateResult:
    """Decode ``max_new_tokens`` ids per row from ``first_ids [rows]`` (each
    row's last prompt token, its K/V not yet cached) over cache slots
    ``[0, rows)``: replay a validated graph, else eager steps."""
    sampling = sampling or Sampling()
    sampling.check()
    msgs: list = []
    say = log or msgs.append
    dev = first_ids.device
    first = first_ids.reshape(-1).to(torch.int64)
    rows = int(first.numel())
    stops = set(int(s) for s in stop_ids)
    g = try_decode_graph(model, cache, first, sampling, log=say) if use_graph else None
    out = torch.empty(max_new_tokens, rows, device=dev, dtype=torch.int64)
    tok = first.clone()
    ch = torch.empty_like(tok)
    ws = None
    if g is None and not sampling.greedy:
        ws = batched_sampler_workspace(model.cfg.vocab, sampling.top_k, rows, dev)[0]
    if g is not None:
        g.token_ids.copy_(first)
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    steps = 0
    for i in range(max_new_tokens):
        if g is not None:
            out[i].copy_(g.step(sampling))
        else:
            u = None if sampling.greedy else sampling.draw(rows, dev)
            logits = model.forward(tok, cache)
            _choose(logits, sampling, ch, u, ws)
            tok.copy_(ch)
            out[i].copy_(ch)
        steps = i + 1
        if stops and (steps % check_every == 0 or steps == max_new_tokens):
            done = torch.isin(out[:steps], torch.tensor(sorted(stops), device=dev)).any(dim=0)
            if bool(done.all()):
                break
    torch.cuda.synchronize(dev)
    decode_s = time.perf_counter() - t0
    workspace.check_timeouts(dev)
    ids = out[:steps].t().cpu().tolist()
    token_ids, reasons = [], []
    for r in ids:
        cut = next((j for j, t in enumerate(r) if t in stops), None)
        if cut is None:
            token_ids.append(r)
            reasons.append("length")
        else:
            token_ids.append(r[:cut + 1])
            reasons.append("stop")
    return GenerateResult(token_ids, reasons, steps, decode_s, g is not None, msgs)
