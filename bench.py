"""Benchmark: packed-ternary MoE FFN layer, decode batch 1, on one MI355X.

Workload: one synthetic MoE FFN layer (hidden 2048, 64 experts, SwiGLU
intermediate 768, top-8 routing) at decode batch 1, run through the HIP
one-launch MoE kernel (router top-k, up+gate SwiGLU, down projections and the
weighted combine in one persistent launch; the three-launch per-slot chain is
timed beside it).  ``--layers`` distinct layers (default 96: 7.3 GB of packed
weights, of which the 8 selected experts per layer are 0.91 GB, 3.6 times the
256 MB Infinity Cache) are chained -- each layer's output is the next
layer's input, as in a decoder -- and captured in one HIP graph replayed in a
cycle, so every layer's weights come from HBM.

Each layer's launch also reads the next layer's router rows ahead into the
caches while its workgroups wait for h (``prefetch``: routing-independent
bytes, fetched once and counted once, in the layer that uses them), as a
decoder's MoE launch can for the next MoE layer.

A step is one graph replay: ``--layers`` dependent MoE-layer decodes, each on
its own cold layer.  ``value`` is the whole-layer algorithmic HBM throughput:
(selected experts' packed codes + scales, the router weight, x in and y out)
per layer, times layers and steps, over the timed time.

``roofline`` covers the dominant kernel, which is the whole layer here
(``k_moe_xcd``, the form of ``ma_moe_fused`` that splits the layer by XCD, or
``k_moe_fused`` where that form does not apply -- ``ma_moe_fused_form`` says
which ran): algorithmic bytes per launch over its average launch
period, timed with HIP events on the stream it runs on over the graph of
back-to-back launches (the period includes the dispatch gap between dependent
kernels, so it is an upper bound on the kernel's own duration).  ``traffic``
is read from the rocprofv3 counter summary under profiles/ when present.

``cpu_baseline`` times the reference's CPU path (NumPy unpack -> dequantise
-> float32 ``torch.nn.functional.linear``, oracle/cpu_baseline.py) for the same
layer on this host's cores; ``extra.cpu_configs`` times the other
configurations the same way (bounded samples, each stated).

    python bench.py [--steps 20] [--warmup 3] [--layers 96] [--no-cpu]
                    [--no-decoder] [--no-extra]
    python bench.py --counters-pass moe_bs1|prefill|decode32   # for rocprofv3 --pmc
    python bench.py --decode-batch 32 # only the full decoder at one batch size
    python bench.py --timeline        # the one-launch MoE layer's phase stamps
    python bench.py --timeline-decoder  # the same with the add + norm and the next QKV projection
    python bench.py --gemv | --preview # config 1 alone | Maple-Preview shapes alone
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "decode tok/s (bs1, bs32); packed-ternary MoE layer HBM GB/s vs 8 TB/s peak"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0
HIDDEN, EXPERTS, INTER, TOPK = 2048, 64, 768, 8
ZIPF_FIXTURE = ROOT / "tests" / "golden" / "zipf_bias_e64.json"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def layer_bytes() -> dict:
    codes = (2 * INTER * HIDDEN + HIDDEN * INTER) // 4
    alpha = (2 * INTER + HIDDEN) * 2
    expert = codes + alpha
    router = EXPERTS * HIDDEN * 2
    act = HIDDEN * 2 * 2
    return {"expert": expert, "selected": TOPK * expert, "layer": TOPK * expert + router + act}


def zipf_fixture() -> dict:
    """Router bias for Zipf(1.1)-skewed top-8 routing over 64 experts and the
    expert load it is fitted to (tests/golden/make_zipf_bias.py)."""
    return json.loads(ZIPF_FIXTURE.read_text())


def load_report(ids, fixture: dict) -> dict:
    """Achieved expert load of a routing against the fixture's target."""
    import numpy as np

    c = np.bincount(np.asarray(ids).reshape(-1), minlength=EXPERTS).astype(np.float64)
    share = c / c.sum()
    target = np.asarray(fixture["target_share"])
    top = np.sort(share)[::-1]
    return {"tv_distance_to_target": round(0.5 * float(np.abs(share - target).sum()), 4),
            "top_shares": [round(float(v), 4) for v in top[:4]], "experts_hit": int((c > 0).sum())}


def graph_of(fn):
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def read_traffic(kernel: str):
    """HBM bytes per launch from profiles/<kernel>_traffic.txt, if measured."""
    p = ROOT / "profiles" / f"{kernel}_traffic.txt"
    if not p.exists():
        return None
    m = re.search(r"hbm_bytes_per_launch:\s*([0-9.eE+]+)", p.read_text())
    return float(m.group(1)) if m else None


def time_graph(g, steps: int, warmup: int) -> float:
    """Seconds per replay of graph ``g`` (HIP events on the current stream)."""
    import torch

    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(True), torch.cuda.Event(True)
    e0.record()
    for _ in range(steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / steps


def gemv_config1(dev, steps: int) -> dict:
    """Config 1: one packed ternary GEMV, 1536 x 2048, batch 1, bf16 x and
    row scales; 1024 distinct cold weight copies (0.8 GB) called back to
    back in one HIP graph, so each call reads its codes from HBM."""
    import torch  # noqa: F401

    from maple_amd import synthetic
    from maple_amd.kernels import ternary_gemv

    n, k, reps = 1536, 2048, 1024
    base = synthetic.ternary_packed((8, n, k), 77, dev)
    ws = [base[i % 8].clone() for i in range(reps)]
    alpha = synthetic.uniform_bf16((n,), 0.01, 0.05, 78, dev)
    xg = synthetic.randn_bf16((1, k), 79, dev)
    g = graph_of(lambda: [ternary_gemv(xg, ws[i], alpha) for i in range(reps)])
    t = time_graph(g, steps, 1) / reps
    nbytes = n * k // 4 + n * 2 + k * 2 + n * 2
    return {"us_per_call": round(t * 1e6, 3), "GB/s": round(nbytes / t / 1e9, 1), "bytes_per_call": nbytes,
            "calls_per_replay": reps}


def extra_workloads(layers, dev, steps: int) -> dict:
    """The other configurations: one GEMV, Zipf-routed batches, a prefill chunk."""
    import torch

    from maple_amd import synthetic
    from maple_amd.kernels import router_topk
    from maple_amd.moe import moe_block

    out = {}
    # The dispatch floor of one dependent launch in a graph (a 1-element fill).
    one = torch.zeros(1, device=dev)
    g = graph_of(lambda: [one.add_(1.0) for _ in range(256)])
    out["launch_floor_us"] = round(time_graph(g, 5, 2) / 256 * 1e6, 3)
    out["gemv_1536x2048_bs1"] = gemv_config1(dev, 3)
    # Zipf(1.1)-routed MoE layers at 32 and 128 tokens.
    fx = zipf_fixture()
    bias = torch.tensor(fx["bias"], dtype=torch.float32, device=dev)
    zl = [synthetic.MoELayer(l.gate_weight, l.up_gate_packed, l.up_gate_alpha, l.down_packed,
                             l.down_alpha, bias) for l in layers]
    for tokens in (32, 128):
        x = synthetic.randn_bf16((tokens, HIDDEN), 1000 + tokens, dev)
        touched, all_ids = 0, []
        for l in zl:
            ids, _ = router_topk(x, l.gate_weight, TOPK, bias=l.router_bias)
            touched += int(torch.unique(ids).numel())
            all_ids.append(ids.cpu())
        nbytes = touched * layer_bytes()["expert"] + len(zl) * (EXPERTS * HIDDEN * 2 + tokens * HIDDEN * 4)
        g = graph_of(lambda: [moe_block(x, l, TOPK) for l in zl])
        t = time_graph(g, max(steps // 2, 3), 2)
        out[f"moe_layer_zipf_T{tokens}"] = {
            "us_per_layer": round(t * 1e6 / len(zl), 2), "GB/s": round(nbytes / t / 1e9, 1),
            "experts_touched_per_layer": round(touched / len(zl), 1),
            "tokens_per_s": round(tokens * len(zl) / t, 0),
            "expert_load": load_report(torch.cat(all_ids).numpy(), fx)}
        del g
    # Prefill chunk: 2048 tokens through one MoE layer (grouped MFMA path).
    tokens = 2048
    x = synthetic.randn_bf16((tokens, HIDDEN), 2048, dev)
    pl = zl[:4]
    ids, _ = router_topk(x, pl[0].gate_weight, TOPK, bias=bias)
    g = graph_of(lambda: [moe_block(x, l, TOPK) for l in pl])
    t = time_graph(g, 5, 2) / len(pl)
    flops = tokens * TOPK * (3 * 2 * INTER * HIDDEN)
    out["moe_prefill_T2048"] = {"us_per_layer": round(t * 1e6, 1), "TFLOP/s": round(flops / t / 1e12, 1),
                                "mfma_frac_of_2500": round(flops / t / 1e12 / MFMA_PEAK_TFLOPS, 4),
                                "expert_load": load_report(ids.cpu().numpy(), fx)}
    return out


def maple_preview_config():
    """Maple-Preview's decoder shapes (the reference's published model,
    docs/HANDOFF.md:279-299): 24 layers, hidden 2048, 16/4 heads of 128 at
    half rotary, 256 experts top-8 with intermediate 512, RTN4 head and
    embeddings in groups of 64 over 151936 tokens, three sliding-window (512)
    layers to every full-attention layer, no RoPE on the full layers.
    Random-init weights of those shapes (no checkpoint here)."""
    from maple_amd.model import DecoderConfig

    return DecoderConfig(hidden=2048, layers=24, heads=16, kv_heads=4, head_dim=128, experts=256, inter=512,
                         top_k=8, vocab=151936, rtn_group=64,
                         layer_types=(("sliding_attention",) * 3 + ("full_attention",)) * 6,
                         sliding_window=512, nope_on_global=True)


def decoder_tokens_per_s(dev, batch: int, steps: int, warmup: int, flash: bool = False, cfg=None,
                         prefill: int = 4096, sampled: bool = False) -> dict:
    """Decode of the full synthetic decoder (by default config 4: 24 layers,
    hidden 2048, 32/4 heads of 64, 64 experts top-8, RTN4 lm_head over 151936
    tokens; ``cfg`` for other shapes) at ``batch`` rows over a ``prefill``-token
    KV cache, one HIP graph replay per step (the whole step captured by the
    decode-graph runner, which first checks 8 replayed steps against 8 eager
    ones).  Each replay appends one position per row and feeds the chosen ids
    to the next step.  Greedy, or with ``sampled`` the reference's benchmark
    sampling (temperature 1.0, top-p 0.95, top-k 20: the fused sampler inside
    the graph, one uniform per row drawn before each replay).  ``flash``: the
    lm_head through a FlashHead (4748 clusters of 32 tokens, 512 probed, one
    forced token; synthetic clusters)."""
    import torch

    from maple_amd import workspace
    from maple_amd.decode_graph import Sampling, try_decode_graph
    from maple_amd.model import DecoderConfig, SyntheticDecoder

    cfg = cfg or DecoderConfig()
    model = SyntheticDecoder(cfg, dev, seed=0, max_len=prefill + steps + warmup + 64)
    cache = model.make_cache(batch, prefill_len=prefill, seed=0)
    if flash:
        from maple_amd.synthetic import flash_head_for

        model.flash_head = flash_head_for(model.lm_head, 4748, 512, 9, dev, force=(151643,))
    gen = torch.Generator(device=dev).manual_seed(batch)
    ids = torch.randint(0, cfg.vocab, (batch,), device=dev, generator=gen)
    mode = (Sampling(temperature=1.0, top_p=0.95, top_k=20, generator=torch.Generator(device=dev).manual_seed(7))
            if sampled else Sampling())
    g = try_decode_graph(model, cache, ids, mode, log=log)
    if g is None:
        raise RuntimeError("the decode graph did not validate against eager decoding")
    for _ in range(warmup):
        g.step(mode)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(True), torch.cuda.Event(True)
    e0.record()
    for _ in range(steps):
        g.step(mode)
    e1.record()
    torch.cuda.synchronize()
    workspace.check_timeouts(dev)
    t = e0.elapsed_time(e1) * 1e-3 / steps
    nbytes = model.decode_bytes(batch, prefill + warmup + steps // 2)
    if flash:
        fh, c = model.flash_head, cfg
        row = lambda grp: c.hidden // 2 + 2 * (c.hidden // grp) * 2  # noqa: E731  codes + scales + biases
        nbytes += (fh.n_clusters * row(64) + (fh.n_probes * fh.cluster_size + fh.n_force) * row(c.rtn_group)
                   - c.vocab * row(c.rtn_group))
    out = {"tokens_per_s": round(batch / t, 1), "ms_per_step": round(t * 1e3, 4),
           "kv_len": prefill, "algorithmic_GB/s": round(nbytes / t / 1e9, 1),
           "hbm_frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4),
           "bytes_per_step": int(nbytes), "sampling": "T1.0 top-p 0.95 top-k 20" if sampled else "greedy"}
    del g, cache, model
    torch.cuda.empty_cache()
    return out


def preview_decode(dev, steps: int, warmup: int) -> dict:
    """Maple-Preview shapes at the reference's published setting (bs1,
    sampled, exact head and FlashHead; a 512-token context, inside the
    reference's 256-700-token haiku runs), greedy bs1 and bs32 beside it.
    The reference's numbers come from a GB10 (~368 tok/s sampled with the
    exact head, 417 MB/token; ~487 tok/s with its FlashHead): context only."""
    cfg = maple_preview_config()
    out = {}
    for key, kw in (("bs1_sampled", dict(batch=1, sampled=True)),
                    ("bs1_sampled_flash_head", dict(batch=1, sampled=True, flash=True)),
                    ("bs1_greedy", dict(batch=1)),
                    ("bs32_greedy", dict(batch=32))):
        log(f"timing Maple-Preview shapes: {key} ...")
        out[key] = decoder_tokens_per_s(dev, kw.pop("batch"), steps, warmup, cfg=cfg, prefill=512, **kw)
        log(json.dumps(out[key]))
    out["reference_gb10_context"] = {"bs1_sampled_tok_s": 368, "bs1_sampled_flash_head_tok_s": 487,
                                     "packed_MB_per_token": 417, "source": "docs/HANDOFF.md:279-299"}
    return out


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _median_time(fn, warmup: int, runs: int, budget_s: float) -> tuple[float, int]:
    import numpy as np

    for _ in range(warmup):
        fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < runs or (time.perf_counter() < t_end and len(times) < 200):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def _np_layer(seed: int):
    import numpy as np

    from oracle import pack

    rng = np.random.default_rng(seed)
    return dict(
        gate=(rng.standard_normal((EXPERTS, HIDDEN)) * 0.02).astype(np.float32),
        ug=pack.pack_2bit(rng.integers(0, 3, (EXPERTS, 2 * INTER, HIDDEN), dtype=np.uint32)),
        ua=rng.uniform(0.01, 0.05, (EXPERTS, 2 * INTER)).astype(np.float32),
        dn=pack.pack_2bit(rng.integers(0, 3, (EXPERTS, HIDDEN, INTER), dtype=np.uint32)),
        da=rng.uniform(0.01, 0.05, (EXPERTS, HIDDEN)).astype(np.float32))


def cpu_baseline() -> dict:
    """Config 2 (one MoE layer, bs1) on the reference's CPU path: 3 warm-ups,
    median of >= 20 runs, the unpack in every call."""
    import numpy as np
    import torch

    from oracle import cpu_baseline as cb

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    L = _np_layer(0)
    xs = np.random.default_rng(1).standard_normal((64, 1, HIDDEN)).astype(np.float32)
    i = [0]

    def run():
        cb.moe_layer(xs[i[0] % 64], L["gate"], L["ug"], L["ua"], L["dn"], L["da"], TOPK)
        i[0] += 1

    med, n = _median_time(run, 3, 20, 10.0)
    return {
        "value": round(layer_bytes()["layer"] / med / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{n} MoE-layer decodes (bs1, H2048 E64 I768 top-8), median {med * 1e3:.1f} ms; "
                  f"NumPy unpack + float32 torch F.linear per selected expert (the reference's CPU "
                  f"oracle path), torch threads = {cores}, os.cpu_count() = {os.cpu_count()}, "
                  f"CPU {_cpu_model()}",
    }


def cpu_configs(decoder_seconds: bool = True) -> dict:
    """The other configurations on the same CPU path (bounded samples)."""
    import numpy as np
    import torch

    from oracle import cpu_baseline as cb
    from oracle import pack

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    out = {"cores": cores, "cpu": _cpu_model()}
    rng = np.random.default_rng(2)
    # config 1: one GEMV 1536 x 2048
    packed = pack.pack_2bit(rng.integers(0, 3, (1536, 2048), dtype=np.uint32))
    alpha = rng.uniform(0.01, 0.05, 1536).astype(np.float32)
    x = rng.standard_normal((1, 2048)).astype(np.float32)
    med, n = _median_time(lambda: cb.ternary_gemv(x, packed, alpha), 3, 20, 3.0)
    nbytes = 1536 * 2048 // 4 + 1536 * 2 + 2048 * 2 + 1536 * 2
    out["gemv_1536x2048_bs1"] = {"us_per_call": round(med * 1e6, 1), "GB/s": round(nbytes / med / 1e9, 3),
                                 "sample": f"median of {n}"}
    # configs 3 and 5: Zipf-routed layers
    L = _np_layer(3)
    bias = np.asarray(zipf_fixture()["bias"], np.float32)
    for tokens, warm, runs, budget in ((32, 3, 20, 8.0), (128, 3, 20, 10.0), (2048, 1, 3, 0.0)):
        xt = rng.standard_normal((tokens, HIDDEN)).astype(np.float32)
        med, n = _median_time(lambda: cb.moe_layer(xt, L["gate"], L["ug"], L["ua"], L["dn"], L["da"], TOPK,
                                                   bias=bias), warm, runs, budget)
        key = f"moe_layer_zipf_T{tokens}" if tokens < 2048 else "moe_prefill_T2048"
        out[key] = {"ms_per_layer": round(med * 1e3, 2), "tokens_per_s": round(tokens / med, 1),
                    "sample": f"median of {n} ({warm} warm-up)"}
        if tokens == 2048:
            out[key]["TFLOP/s"] = round(tokens * TOPK * 3 * 2 * INTER * HIDDEN / med / 1e12, 4)
    if decoder_seconds:
        out["decoder_bs1_token"] = cpu_decoder_token()
    return out


def cpu_decoder_token() -> dict:
    """One bs1 token of the full synthetic decoder (24 layers, 4096-token cache)
    on the CPU path: a single timed token after one warm-up layer pass."""
    import numpy as np
    import torch

    from oracle import cpu_baseline as cb
    from oracle import decoder as od
    from oracle import pack

    rng = np.random.default_rng(4)
    H, nq, nkv, d, vocab, grp = HIDDEN, 32, 4, 64, 151936, 128
    qkv_rows = (nq + 2 * nkv) * d
    ones = np.ones
    shared = _np_layer(5)  # the MoE weights are shared by the layers here (same work per layer)
    layers = []
    for i in range(24):
        layers.append(dict(
            qkv=pack.pack_2bit(rng.integers(0, 3, (qkv_rows, H), dtype=np.uint32)),
            qkv_alpha=rng.uniform(0.01, 0.05, qkv_rows).astype(np.float32),
            o=pack.pack_2bit(rng.integers(0, 3, (H, nq * d), dtype=np.uint32)),
            o_alpha=rng.uniform(0.01, 0.05, H).astype(np.float32),
            input_ln=ones(H, np.float32), post_ln=ones(H, np.float32), q_norm=ones(d, np.float32),
            k_norm=ones(d, np.float32),
            moe=dict(gate_weight=shared["gate"], up_gate_packed=shared["ug"], up_gate_alpha=shared["ua"],
                     down_packed=shared["dn"], down_alpha=shared["da"])))
    words = rng.integers(0, 2 ** 32, (vocab, H // 8), dtype=np.uint64).astype(np.uint32)
    sc = rng.uniform(0.003, 0.006, (vocab, H // grp)).astype(np.float32)
    table = (words, sc, (-7.5 * sc).astype(np.float32))
    cos, sin = od.rope_tables(4096 + 8, 32, 1e4)
    m = dict(cfg=dict(hidden=H, heads=nq, kv_heads=nkv, head_dim=d, rotary_dim=32, eps=1e-6, rtn_group=grp,
                      top_k=TOPK), layers=layers, embed=table, lm_head=table, final_norm=ones(H, np.float32),
             cos=cos, sin=sin)
    kv = lambda: rng.standard_normal((1, nkv, 4096 + 8, d), dtype=np.float32)  # noqa: E731
    cache = dict(k=[kv() for _ in range(24)], v=[kv() for _ in range(24)], seqlen=np.array([4096]))
    t0 = time.perf_counter()
    cb.decoder_token(m, cache, 12345)
    t = time.perf_counter() - t0
    return {"s_per_token": round(t, 3), "tokens_per_s": round(1.0 / t, 3),
            "sample": "1 token (24 layers over a 4096-position cache + the 151936-row RTN4 head), "
                      f"torch threads = {torch.get_num_threads()}"}


def counters_pass(dev, kind: str, n_layers: int) -> int:
    """Workloads for rocprofv3 --pmc passes (no device random numbers: torch's
    RNG kernels have faulted under the counter collector here).  Each runs its
    kernels, then a plain 256 MiB device copy four times to calibrate the
    counters against a known byte count.

    moe_bs1:  the one-launch MoE layer kernel over ``n_layers`` cold layers,
              twice; router rows set by fill kernels so that layer l selects 8
              distinct experts (8l + 56 .. 8l + 63 mod 64); expert weights left
              uninitialised (traffic does not depend on their values).
    prefill:  the 2048-token grouped MoE layer on 4 layers generated on the
              host (CPU random numbers) and copied over, with the Zipf bias.
    decode32: the batch-32 RTN4 lm_head GEMM (151936 x 2048, group 128) and the
              batch-32 fused decode attention over a 4096-position cache, on
              zero-filled tensors."""
    import torch

    from maple_amd import synthetic
    from maple_amd.moe import moe_block

    if kind == "moe_bs1":
        kw = HIDDEN // 16
        layers = []
        e = torch.arange(EXPERTS, device=dev, dtype=torch.float32)
        for l in range(n_layers):
            rank = torch.remainder(e - 8 * l, EXPERTS)  # logit of expert e with x = ones: rank / 64
            gate = (rank / (EXPERTS * HIDDEN))[:, None].expand(EXPERTS, HIDDEN).to(torch.bfloat16).contiguous()
            ug = torch.empty(EXPERTS, 2 * INTER, kw, device=dev, dtype=torch.int32).view(torch.uint32)
            ua = torch.empty(EXPERTS, 2 * INTER, device=dev, dtype=torch.bfloat16)
            dn = torch.empty(EXPERTS, HIDDEN, INTER // 16, device=dev, dtype=torch.int32).view(torch.uint32)
            da = torch.empty(EXPERTS, HIDDEN, device=dev, dtype=torch.bfloat16)
            layers.append(synthetic.MoELayer(gate, ug, ua, dn, da, None))
        x = torch.ones(1, HIDDEN, dtype=torch.bfloat16).to(dev)
        torch.cuda.synchronize()
        for _ in range(2):
            for l in range(n_layers):
                moe_block(x, layers[l], TOPK, plan="fused")
        info = {"moe_fused_launches": 2 * n_layers, "layer_bytes_per_launch": layer_bytes()["layer"]}
    elif kind == "prefill":
        fx = zipf_fixture()
        layers = []
        for i in range(4):
            c = synthetic.make_moe_layer(HIDDEN, EXPERTS, INTER, seed=200 + i, device="cpu")
            layers.append(synthetic.MoELayer(
                c.gate_weight.to(dev), c.up_gate_packed.view(torch.int32).to(dev).view(torch.uint32),
                c.up_gate_alpha.to(dev), c.down_packed.view(torch.int32).to(dev).view(torch.uint32),
                c.down_alpha.to(dev), torch.tensor(fx["bias"], dtype=torch.float32, device=dev)))
        x = synthetic.randn_bf16((2048, HIDDEN), 2048, "cpu").to(dev)
        torch.cuda.synchronize()
        for _ in range(2):
            for l in layers:
                moe_block(x, l, TOPK)
        info = {"prefill_layers": 8, "tokens": 2048, "flops_per_layer": 2048 * TOPK * 3 * 2 * INTER * HIDDEN}
    elif kind == "decode32":
        from maple_amd.kernels.decode_attn import decode_attention, gqa_workspace
        from maple_amd.kernels.rtn4 import rtn4_gemv

        vocab, batch, max_len = 151936, 32, 4096 + 64
        w = torch.zeros(vocab, HIDDEN // 8, device=dev, dtype=torch.int32).view(torch.uint32)
        sc = torch.zeros(vocab, HIDDEN // 128, device=dev, dtype=torch.bfloat16)
        xh = torch.zeros(batch, HIDDEN, device=dev, dtype=torch.bfloat16)
        kc = torch.zeros(batch, 4, max_len, 64, device=dev, dtype=torch.bfloat16)
        vc = torch.zeros_like(kc)
        qkv = torch.zeros(batch, (32 + 8) * 64, device=dev, dtype=torch.bfloat16)
        nw = torch.ones(64, device=dev)
        cos = torch.ones(max_len, 32, device=dev)
        sin = torch.zeros(max_len, 32, device=dev)
        seqlen = torch.full((batch,), 4096, device=dev, dtype=torch.int64)
        ws = gqa_workspace(batch, 4, max_len, dev, 64)
        torch.cuda.synchronize()
        for _ in range(4):
            rtn4_gemv(xh, w, sc, sc, group_size=128)
            decode_attention(qkv, nw, nw, cos, sin, kc, vc, seqlen, ws, num_heads=32, num_kv_heads=4,
                             head_dim=64, rotary_dim=32, scale=0.125)
        # the decoder's MoE layer at 32 tokens (routing launch, grouped SwiGLU and down)
        from maple_amd.moe import moe_layer

        layer = synthetic.make_moe_layer(HIDDEN, 64, INTER, seed=5, device=dev)
        xm = synthetic.randn_bf16((batch, HIDDEN), 6, dev)
        am = synthetic.randn_bf16((batch, HIDDEN), 7, dev)
        lnw = torch.ones(HIDDEN, device=dev)
        torch.cuda.synchronize()
        hit = 0
        for _ in range(4):
            _, ids = moe_layer(xm, layer, TOPK, lnw, 1e-6, add=am)
            hit = int(torch.unique(ids).numel())
        info = {"rtn4_launches": 4, "rtn4_bytes_per_launch": vocab * HIDDEN // 2 + 2 * vocab * 16 * 2,
                "attn_launches": 4, "attn_kv_bytes_per_launch": batch * 2 * 4 * 4097 * 64 * 2,
                "grouped_launches": 4, "experts_hit": hit,
                "swiglu_weight_bytes_per_launch": hit * (2 * INTER * HIDDEN // 4 + 2 * INTER * 2),
                "down_weight_bytes_per_launch": hit * (HIDDEN * INTER // 4 + HIDDEN * 2)}
    else:
        raise ValueError(f"unknown counters pass {kind}")
    torch.cuda.synchronize()
    a = torch.empty(128 << 20, device=dev, dtype=torch.bfloat16)
    b = torch.empty_like(a)
    for _ in range(4):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"counters_pass": kind, **info, "copy_bytes_read": a.numel() * 2,
                      "copy_bytes_written": a.numel() * 2}), flush=True)
    return 0


PHASES = ["start", "router logit out", "logits seen", "ranked", "weight loads issued", "h published",
          "h seen", "h staged", "down values out", "down values seen", "y out", "end"]
# with the add + RMSNorm in front and the next layer's QKV projection behind
NEXT_PHASES = ["next: y seen", "next: x' staged", "next: rows out"]


def timeline(dev, n_layers: int, reps: int, decoder_form: bool = False) -> int:
    """Per-phase timeline of the one-launch MoE layer: the library's stamped
    variant (libmaple_amd_stamps.so, ma_moe_phase_stamps) runs ``n_layers``
    chained cold layers in one graph; after each replay the stamps of the
    chain's last layer are read from the workspace.  Prints one JSON line:
    per phase the median / p90 / max over workgroups and replays of the time
    since the launch's first workgroup started (us), and the stamped build's
    period per layer (the stamps' own stores and waits lengthen it).

    ``decoder_form``: each layer as the bs1 decoder runs it -- the
    attention's projected output added to x and RMS-normed in front (a fixed
    bf16 vector, float32 norm weights), and the next layer's RMS-folded QKV
    projection (2560 x 2048 ternary rows, bf16 row scales) behind, from each
    XCD's own copy of y."""
    import ctypes

    import numpy as np
    import torch

    from maple_amd import _lib, synthetic, workspace
    from maple_amd.moe import fused_form, moe_block

    _lib.use_stamped_library()
    lib = _lib.load()
    off, words, wgs = ctypes.c_size_t(), ctypes.c_int(), ctypes.c_int()
    if lib.ma_moe_phase_stamps(ctypes.byref(off), ctypes.byref(words), ctypes.byref(wgs)) != 0:
        log("timeline: " + lib.ma_last_error().decode(errors="replace"))
        return 1
    layers = [synthetic.make_moe_layer(HIDDEN, EXPERTS, INTER, seed=i, device=dev) for i in range(n_layers)]
    if fused_form(layers[0], TOPK) != 1:
        log("timeline: the XCD-split form does not run on this device")
        return 1
    x = synthetic.randn_bf16((1, HIDDEN), 12345, dev)
    phases = PHASES + (NEXT_PHASES if decoder_form else [])
    if decoder_form:
        from maple_amd.moe import moe_fused

        o = synthetic.randn_bf16((1, HIDDEN), 54321, dev)
        norms = [(torch.rand(HIDDEN, generator=torch.Generator().manual_seed(i)) + 0.5).to(dev)
                 for i in range(n_layers)]
        qkv = [synthetic.ternary_linear(2560, HIDDEN, 1000 + i, dev) for i in range(n_layers)]

    def chain():
        h = x
        for i, layer in enumerate(layers):
            nxt = (i + 1) % n_layers
            if decoder_form:
                h = moe_fused(h, layer, TOPK, add=o, norm_weight=norms[i], eps=1e-6,
                              next_linear=(qkv[nxt][0], qkv[nxt][1], norms[nxt], 1e-6),
                              prefetch=layers[nxt].gate_weight)[0]
            else:
                h, _, _ = moe_block(h, layer, TOPK, plan="fused", prefetch=layers[nxt].gate_weight)

    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        chain()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        chain()
    ws = [w for k, w in workspace._POOL.items() if k[0] == "moe_fused" and k[2] == s.cuda_stream][-1]
    n0, nw, ng = off.value // 4, words.value, wgs.value
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    rows = []
    e0, e1 = torch.cuda.Event(True), torch.cuda.Event(True)
    elapsed = 0.0
    for _ in range(reps):
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        elapsed += e0.elapsed_time(e1) * 1e-3
        rows.append(ws.view(torch.int32)[n0:n0 + nw * ng].cpu().numpy().astype(np.int64).reshape(ng, nw))
    workspace.check_timeouts(dev)
    d = np.stack(rows) & 0xFFFFFFFF  # [reps, workgroups, words], 32-bit counter values
    t0 = d[:, :, 0].min(axis=1, keepdims=True)
    rel = ((d[:, :, :len(phases)] - t0[:, :, None]) & 0xFFFFFFFF) * 0.01  # 100 MHz ticks -> us
    out = {}
    router_wgs = np.arange(ng) < 64  # workgroups 0..7 of each XCD (i / 8 < 8)
    for i, name in enumerate(phases):
        v = rel[:, router_wgs, i] if i == 1 else rel[:, :, i]
        out[name] = {"median": round(float(np.median(v)), 2), "p90": round(float(np.percentile(v, 90)), 2),
                     "max": round(float(v.max()), 2)}
    xcds = sorted(set(int(v) for v in d[0, :, 15]))
    print(json.dumps({"timeline": "k_moe_xcd phase stamps, us from the launch's first workgroup",
                      "form": "decoder (add + norm, next QKV projection)" if decoder_form else "plain",
                      "layers_in_chain": n_layers, "replays": reps, "xcds_seen": xcds,
                      "stamped_us_per_layer": round(elapsed / reps / n_layers * 1e6, 3), "phases": out}),
          flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=96)
    ap.add_argument("--counters-pass", choices=("moe_bs1", "prefill", "decode32"), default=None,
                    help="only run one workload and a plain 256 MiB copy (for counters)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-decoder", action="store_true")
    ap.add_argument("--decode-batch", type=int, default=0,
                    help="only time the full decoder at this batch (for profiling runs)")
    ap.add_argument("--flash-head", action="store_true",
                    help="with --decode-batch 1: the lm_head through a FlashHead")
    ap.add_argument("--gemv", action="store_true",
                    help="only the config-1 GEMV (1024 cold 1536 x 2048 calls per graph replay)")
    ap.add_argument("--preview", action="store_true",
                    help="only the decoder at Maple-Preview shapes (bs1 sampled / greedy, bs32)")
    ap.add_argument("--timeline", action="store_true",
                    help="only the one-launch MoE layer's per-phase timeline (stamped library)")
    ap.add_argument("--timeline-decoder", action="store_true",
                    help="the same in the decoder's form (add + norm in front, next QKV projection behind)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: there is no multi-GPU path "
              "(run with --gpus 1).", file=sys.stderr)
        return 2

    import torch

    import __graft_entry__

    __graft_entry__.load_package()
    from maple_amd import synthetic, workspace
    from maple_amd.moe import moe_block

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    nb = layer_bytes()
    L = args.layers
    if args.counters_pass:
        return counters_pass(dev, args.counters_pass, L)
    if args.timeline or args.timeline_decoder:
        return timeline(dev, L, max(args.steps, 10), decoder_form=args.timeline_decoder)
    if args.gemv:
        print(json.dumps({"gemv_1536x2048_bs1": gemv_config1(dev, max(args.steps, 3))}), flush=True)
        return 0
    if args.preview:
        print(json.dumps({"decode": {"maple_preview": preview_decode(dev, max(args.steps, 10), args.warmup)}}),
              flush=True)
        return 0
    if args.decode_batch > 0:
        res = decoder_tokens_per_s(dev, args.decode_batch, max(args.steps, 10), args.warmup,
                                   flash=args.flash_head)
        print(json.dumps({"decode": {f"bs{args.decode_batch}": res}}), flush=True)
        return 0
    log(f"building {L} cold MoE layers ...")
    layers = [synthetic.make_moe_layer(HIDDEN, EXPERTS, INTER, seed=i, device=dev) for i in range(L)]
    x = synthetic.randn_bf16((1, HIDDEN), 12345, dev)
    torch.cuda.synchronize()

    def chain(plan):
        # each layer's launch reads the next layer's router rows ahead into
        # the caches (the one-launch plan; routing-independent bytes, counted
        # once, in the layer that uses them)
        h = x
        for i, layer in enumerate(layers):
            h, _, _ = moe_block(h, layer, TOPK, plan=plan, prefetch=layers[(i + 1) % L].gate_weight)

    # Whole-layer timing: L dependent layer decodes per graph replay (one launch each).
    g = graph_of(lambda: chain("fused"))
    for _ in range(args.warmup):
        g.replay()
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(True), torch.cuda.Event(True)
    t0 = time.perf_counter()
    e0.record(s)
    for _ in range(args.steps):
        g.replay()
    e1.record(s)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / args.steps
    value = nb["layer"] * L / (ms * 1e-3) / 1e9
    per_launch = ms * 1e-3 / L  # the whole layer is one launch of ma_moe_fused
    from maple_amd.moe import fused_form
    xcd_form = fused_form(layers[0], TOPK) == 1
    kname, tname = ("k_moe_xcd", "moe_xcd_bs1") if xcd_form else ("k_moe_fused", "moe_fused_bs1")
    achieved = nb["layer"] / per_launch / 1e9
    log(f"MoE layer bs1: {ms * 1e3 / L:.2f} us/layer, {value:.1f} GB/s (wall {wall:.3f} s)")
    del g
    # The three-launch chain (router, SwiGLU, down + combine) on the same layers.
    gc = graph_of(lambda: chain("per_slot"))
    per_slot = time_graph(gc, args.steps, args.warmup) / L
    del gc
    log(f"per-slot chain: {per_slot * 1e6:.2f} us/layer")
    try:
        workspace.check_timeouts(dev)
    except RuntimeError as exc:
        log(f"{exc}: results invalid")
        return 1
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "moe_ffn_layer_decode_bs1", "hidden": HIDDEN, "experts": EXPERTS,
                   "intermediate": INTER, "top_k": TOPK, "tokens": 1, "cold_layers": L,
                   "chained": True, "bytes_per_layer": nb["layer"],
                   "us_per_layer": round(ms * 1e3 / L, 3),
                   "per_slot_chain_us_per_layer": round(per_slot * 1e6, 3)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic(tname), "kernel": kname,
                     "bytes_per_launch": nb["layer"],
                     "us_per_launch": round(per_launch * 1e6, 3)},
        "cpu_baseline": None,
        "decode": None,
        "extra": None,
    }
    if not args.no_decoder:
        out["decode"] = {}
        for bsz in (1, 32):
            log(f"timing the full decoder at batch {bsz} ...")
            out["decode"][f"bs{bsz}"] = decoder_tokens_per_s(dev, bsz, max(args.steps, 10), args.warmup)
            log(json.dumps(out["decode"][f"bs{bsz}"]))
        log("timing the full decoder at batch 1 with the FlashHead ...")
        out["decode"]["bs1_flash_head"] = decoder_tokens_per_s(dev, 1, max(args.steps, 10), args.warmup, flash=True)
        log(json.dumps(out["decode"]["bs1_flash_head"]))
        out["decode"]["maple_preview"] = preview_decode(dev, max(args.steps, 10), args.warmup)
    if not args.no_extra:
        log("timing the other workloads ...")
        out["extra"] = extra_workloads(layers, dev, args.steps)
        log(json.dumps(out["extra"]))
    if not args.no_cpu:
        log("timing the CPU baseline ...")
        out["cpu_baseline"] = cpu_baseline()
        log(json.dumps(out["cpu_baseline"]))
        if not args.no_extra:
            log("timing the other configurations on the CPU ...")
            out["extra"] = out["extra"] or {}
            out["extra"]["cpu_configs"] = cpu_configs()
            log(json.dumps(out["extra"]["cpu_configs"]))
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
