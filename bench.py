"""Benchmark: packed-ternary MoE FFN layer, decode batch 1, on one MI355X.

Workload: one synthetic MoE FFN layer (hidden 2048, 64 experts, SwiGLU
intermediate 768, top-8 routing) at decode batch 1, run through the HIP
one-launch MoE kernel (router top-k, up+gate SwiGLU, down projections and the
weighted combine in one persistent launch; the three-launch per-slot chain is
timed beside it).  ``--layers`` distinct layers (default 96: 7.3 GB of packed
weights, of which the 8 selected experts per layer are 0.91 GB, 3.6 times the
256 MB Infinity Cache) are captured in one HIP graph and replayed in a cycle,
so every layer's weights come from HBM.

A step is one graph replay: ``--layers`` MoE-layer decodes, each on its own
cold layer.  ``value`` is the whole-layer algorithmic HBM throughput:
(selected experts' packed codes + scales, the router weight, x in and y out)
per layer, times layers and steps, over the timed wall time.

``roofline`` covers the dominant kernel, which is the whole layer here
(``k_moe_fused``): algorithmic bytes per launch over its average launch
period, timed with HIP events on the stream it runs on over the graph of
back-to-back launches on the cold layers (the period includes the dispatch
gap between dependent kernels, so it is an upper bound on the kernel's own
duration).  ``traffic`` is read from the rocprofv3 counter summary under
profiles/ when present.

``cpu_baseline`` times the CPU oracle path (NumPy unpack -> dequantise ->
float32 matmul over the 8 selected experts, the reference's own test
oracle) on a bounded sample of the same workload on this host's cores.

    python bench.py [--steps 20] [--warmup 3] [--layers 96] [--no-cpu]
                    [--no-decoder] [--no-extra]
    python bench.py --counters-pass   # MoE layer graph + a 256 MiB copy, for rocprofv3 --pmc
    python bench.py --decode-batch 32 # only the full decoder at one batch size
"""

from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "decode tok/s (bs1, bs32); packed-ternary MoE layer HBM GB/s vs 8 TB/s peak"
HBM_PEAK_GBS = 8000.0
HIDDEN, EXPERTS, INTER, TOPK = 2048, 64, 768, 8


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def layer_bytes() -> dict:
    codes = (2 * INTER * HIDDEN + HIDDEN * INTER) // 4
    alpha = (2 * INTER + HIDDEN) * 2
    expert = codes + alpha
    router = EXPERTS * HIDDEN * 2
    act = HIDDEN * 2 * 2
    return {"expert": expert, "selected": TOPK * expert, "layer": TOPK * expert + router + act}


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


def extra_workloads(layers, dev, steps: int) -> dict:
    """The other configurations: one GEMV, Zipf-routed batches, a prefill chunk."""
    import torch

    from maple_amd import synthetic
    from maple_amd.kernels import router_topk, ternary_gemv
    from maple_amd.moe import moe_block

    out = {}
    # Single packed ternary GEMV, 1536 x 2048, batch 1, 1024 distinct cold copies.
    n, k, reps = 1536, 2048, 1024
    base = synthetic.ternary_packed((8, n, k), 77, dev)
    ws = [base[i % 8].clone() for i in range(reps)]
    alpha = synthetic.uniform_bf16((n,), 0.01, 0.05, 78, dev)
    xg = synthetic.randn_bf16((1, k), 79, dev)
    g = graph_of(lambda: [ternary_gemv(xg, ws[i], alpha) for i in range(reps)])
    t = time_graph(g, 3, 1) / reps
    nbytes = n * k // 4 + n * 2 + k * 2 + n * 2
    out["gemv_1536x2048_bs1"] = {"us_per_call": round(t * 1e6, 3), "GB/s": round(nbytes / t / 1e9, 1)}
    del ws, base, g
    # Zipf(1.1)-routed MoE layers at 32 and 128 tokens.
    bias = synthetic.zipf_router_bias(EXPERTS, 1.1, 1.0, seed=3).to(dev)
    zl = [synthetic.MoELayer(l.gate_weight, l.up_gate_packed, l.up_gate_alpha, l.down_packed,
                             l.down_alpha, bias) for l in layers]
    for tokens in (32, 128):
        x = synthetic.randn_bf16((tokens, HIDDEN), 1000 + tokens, dev)
        touched = 0
        for l in zl:
            ids, _ = router_topk(x, l.gate_weight, TOPK, bias=l.router_bias)
            touched += int(torch.unique(ids).numel())
        nbytes = touched * layer_bytes()["expert"] + len(zl) * (EXPERTS * HIDDEN * 2 + tokens * HIDDEN * 4)
        g = graph_of(lambda: [moe_block(x, l, TOPK) for l in zl])
        t = time_graph(g, max(steps // 2, 3), 2)
        out[f"moe_layer_zipf_T{tokens}"] = {
            "us_per_layer": round(t * 1e6 / len(zl), 2), "GB/s": round(nbytes / t / 1e9, 1),
            "experts_touched_per_layer": round(touched / len(zl), 1),
            "tokens_per_s": round(tokens * len(zl) / t, 0)}
        del g
    # Prefill chunk: 2048 tokens through one MoE layer (grouped MFMA path).
    tokens = 2048
    x = synthetic.randn_bf16((tokens, HIDDEN), 2048, dev)
    pl = zl[:4]
    g = graph_of(lambda: [moe_block(x, l, TOPK) for l in pl])
    t = time_graph(g, 5, 2) / len(pl)
    flops = tokens * TOPK * (3 * 2 * INTER * HIDDEN)
    out["moe_prefill_T2048"] = {"us_per_layer": round(t * 1e6, 1), "TFLOP/s": round(flops / t / 1e12, 1),
                                "mfma_frac_of_2500": round(flops / t / 2.5e15, 4)}
    return out


def decoder_tokens_per_s(dev, batch: int, steps: int, warmup: int) -> dict:
    """Greedy decode of the full synthetic decoder (24 layers, hidden 2048,
    32/4 heads of 64, 64 experts top-8, RTN4 lm_head over 151936 tokens) at
    ``batch`` rows over a 4096-token KV cache, one HIP graph replay per step
    (the whole step captured).  Each replay appends one position per row."""
    import torch

    from maple_amd.model import DecoderConfig, SyntheticDecoder

    cfg = DecoderConfig()
    model = SyntheticDecoder(cfg, dev, seed=0, max_len=4096 + steps + warmup + 8)
    cache = model.make_cache(batch, prefill_len=4096, seed=0)
    gen = torch.Generator(device=dev).manual_seed(batch)
    ids = torch.randint(0, cfg.vocab, (batch,), device=dev, generator=gen)
    g = graph_of(lambda: model.greedy_step(ids, cache))
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(True), torch.cuda.Event(True)
    e0.record()
    for _ in range(steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) * 1e-3 / steps
    nbytes = model.decode_bytes(batch, 4096 + warmup + steps // 2)
    out = {"tokens_per_s": round(batch / t, 1), "ms_per_step": round(t * 1e3, 4),
           "kv_len": 4096, "algorithmic_GB/s": round(nbytes / t / 1e9, 1),
           "hbm_frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)}
    del g, cache, model
    torch.cuda.empty_cache()
    return out


def cpu_baseline(seconds: float = 12.0) -> dict:
    import numpy as np

    from oracle import kernels as ok
    from oracle import pack

    cores = len(os.sched_getaffinity(0))
    rng = np.random.default_rng(0)
    ug = pack.pack_2bit(rng.integers(0, 3, (EXPERTS, 2 * INTER, HIDDEN), dtype=np.uint32))
    ua = rng.uniform(0.01, 0.05, (EXPERTS, 2 * INTER)).astype(np.float32)
    dn = pack.pack_2bit(rng.integers(0, 3, (EXPERTS, HIDDEN, INTER), dtype=np.uint32))
    da = rng.uniform(0.01, 0.05, (EXPERTS, HIDDEN)).astype(np.float32)
    gw = (rng.standard_normal((EXPERTS, HIDDEN)) * 0.02).astype(np.float32)
    xs = rng.standard_normal((64, 1, HIDDEN)).astype(np.float32)
    for i in range(3):
        ok.moe_layer_cpu_fp32(xs[i], gw, ug, ua, dn, da, TOPK)
    times = []
    t_end = time.perf_counter() + seconds
    i = 0
    while len(times) < 20 or (time.perf_counter() < t_end and len(times) < 200):
        t0 = time.perf_counter()
        ok.moe_layer_cpu_fp32(xs[i % 64], gw, ug, ua, dn, da, TOPK)
        times.append(time.perf_counter() - t0)
        i += 1
    med = float(np.median(times))
    return {
        "value": round(layer_bytes()["layer"] / med / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{len(times)} MoE-layer decodes (bs1, H2048 E64 I768 top-8), median "
                  f"{med * 1e3:.1f} ms; NumPy unpack + float32 matmul per selected expert, "
                  f"BLAS threads = {cores}, os.cpu_count() = {os.cpu_count()}",
    }


def counters_pass(dev, n_layers: int) -> int:
    """Workload for rocprofv3 --pmc passes (FETCH_SIZE / WRITE_SIZE per
    dispatch): the one-launch MoE layer kernel over ``n_layers`` cold layers,
    twice, then a plain 256 MiB device copy four times to calibrate the
    counter against a known byte count.  Traffic does not depend on the weight
    values, so the expert weights are left uninitialised; the router rows are
    set (by fill kernels, no random numbers under the profiler) so that layer
    l selects 8 distinct experts, 8l + 56 .. 8l + 63 mod 64."""
    import torch

    from maple_amd import synthetic
    from maple_amd.moe import moe_block

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
    torch.cuda.synchronize()
    a = torch.empty(128 << 20, device=dev, dtype=torch.bfloat16)
    b = torch.empty_like(a)
    for _ in range(4):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"counters_pass": True, "moe_fused_launches": 2 * n_layers,
                      "layer_bytes_per_launch": layer_bytes()["layer"],
                      "copy_bytes_read": a.numel() * 2, "copy_bytes_written": a.numel() * 2}),
          flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=96)
    ap.add_argument("--counters-pass", action="store_true",
                    help="only run the MoE layer kernel and a plain 256 MiB copy (for counters)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-decoder", action="store_true")
    ap.add_argument("--decode-batch", type=int, default=0,
                    help="only time the full decoder at this batch (for profiling runs)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: there is no multi-GPU path "
              "(run with --gpus 1).", file=sys.stderr)
        return 2

    import torch

    import __graft_entry__

    __graft_entry__.load_package()
    from maple_amd import synthetic
    from maple_amd.moe import moe_block

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    nb = layer_bytes()
    L = args.layers
    if args.counters_pass:
        return counters_pass(dev, L)
    if args.decode_batch > 0:
        res = decoder_tokens_per_s(dev, args.decode_batch, max(args.steps, 10), args.warmup)
        print(json.dumps({"decode": {f"bs{args.decode_batch}": res}}), flush=True)
        return 0
    log(f"building {L} cold MoE layers ...")
    layers = [synthetic.make_moe_layer(HIDDEN, EXPERTS, INTER, seed=i, device=dev) for i in range(L)]
    x = synthetic.randn_bf16((1, HIDDEN), 12345, dev)
    torch.cuda.synchronize()

    # Whole-layer timing: L layer decodes per graph replay (one launch each).
    g = graph_of(lambda: [moe_block(x, layers[i], TOPK) for i in range(L)])
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
    per_launch = ms * 1e-3 / L  # the whole layer is one k_moe_fused launch
    achieved = nb["layer"] / per_launch / 1e9
    log(f"MoE layer bs1: {ms * 1e3 / L:.2f} us/layer, {value:.1f} GB/s (wall {wall:.3f} s)")
    del g
    from maple_amd.moe import moe_fused_timed_out

    # The three-launch chain (router, SwiGLU, down + combine) on the same layers.
    gc = graph_of(lambda: [moe_block(x, layers[i], TOPK, plan="per_slot") for i in range(L)])
    chain = time_graph(gc, args.steps, args.warmup) / L
    del gc
    log(f"per-slot chain: {chain * 1e6:.2f} us/layer")

    from maple_amd.kernels.router import router_wait_timed_out

    if router_wait_timed_out(dev) or moe_fused_timed_out(dev):
        log("a kernel reported a timed-out cross-workgroup wait: results invalid")
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
                   "bytes_per_layer": nb["layer"], "us_per_layer": round(ms * 1e3 / L, 3),
                   "per_slot_chain_us_per_layer": round(chain * 1e6, 3)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic("moe_fused_bs1"), "kernel": "k_moe_fused",
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
    if not args.no_extra:
        log("timing the other workloads ...")
        out["extra"] = extra_workloads(layers, dev, args.steps)
        log(json.dumps(out["extra"]))
    if not args.no_cpu:
        log("timing the CPU baseline ...")
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
