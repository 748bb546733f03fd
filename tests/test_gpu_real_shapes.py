"""Maple-Preview's shapes on the HIP kernels vs the CPU oracle (needs the GPU).

Shapes (reference docs/HANDOFF.md:190-199, model.py:750-832): hidden 2048,
16 query / 4 KV heads of 128 (partial rotary 0.5), 256 experts top-8 with
intermediate 512, the RTN4 head in groups of 64, layer_types 3 sliding
(window 512) : 1 full with NoPE on the full layers.

* the MoE layer at 1 token (the one-launch kernel, also with the add +
  RMSNorm in front and the next layer's 3072-row QKV projection in the same
  launch), 2-3 tokens (per-slot kernels), 8-32 tokens (routing launch +
  grouped experts) and a 2048-token prefill chunk (grouped MFMA GEMMs);
* the RTN4 lm_head over the full 151936-row vocabulary in groups of 64 at
  batch 1 and 32;
* a 4-layer decoder at these shapes written as a packed-ternary-v1
  checkpoint, loaded back, and decoded over a 600-position cache (past the
  sliding window) at batch 1, 3 and 20 against the oracle.
Tolerances as in the other parity tests.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from _helpers import assert_bf16_close, np_f, np_u32, tie_safe_rows
from maple_amd import synthetic
from maple_amd.kernels import rtn4_gemv, ternary_gemv
from maple_amd.model import DecoderConfig, SyntheticDecoder
from maple_amd.moe import fused_supported, moe_block, moe_fused, moe_fused_timed_out
from oracle import kernels as ok
from test_gpu_decoder import _to_np

pytestmark = pytest.mark.gpu

H, E, I, K = 2048, 256, 512, 8
Y_ATOL = 2.0 ** -7
MAPLE = DecoderConfig(hidden=2048, layers=4, heads=16, kv_heads=4, head_dim=128, experts=256, inter=512,
                      top_k=8, vocab=8192, rtn_group=64, lm_scale=(0.003, 0.006),
                      layer_types=("sliding_attention",) * 3 + ("full_attention",), sliding_window=512,
                      nope_on_global=True)


@pytest.fixture(scope="module")
def layer(dev):
    return synthetic.make_moe_layer(H, E, I, seed=21, device=dev)


def _oracle_y(x, L, ids, wts, residual=None):
    rid, rw, probs = ok.router_topk(x, np_f(L.gate_weight), K,
                                    bias=None if L.router_bias is None else np_f(L.router_bias))
    safe = tie_safe_rows(probs, K)
    assert safe.mean() > 0.98
    idn, wn = ids.cpu().numpy(), wts.cpu().numpy()
    np.testing.assert_array_equal(idn[safe], rid[safe])
    np.testing.assert_allclose(wn[safe], rw[safe], rtol=1e-4, atol=1e-6)
    y, _ = ok.moe_experts(x, idn, wn, np_u32(L.up_gate_packed), np_f(L.up_gate_alpha),
                          np_u32(L.down_packed), np_f(L.down_alpha), residual=residual)
    return y


def test_one_launch_layer_is_built_and_matches_the_oracle(dev, layer):
    x = synthetic.randn_bf16((1, H), 31, dev)
    assert fused_supported(layer, K, x)
    for step in range(3):
        x = synthetic.randn_bf16((1, H), 31 + step, dev)
        res = synthetic.randn_bf16((1, H), 41 + step, dev)
        y, ids, wts = moe_fused(x, layer, K, res)
        torch.cuda.synchronize()
        assert_bf16_close(np_f(y), _oracle_y(np_f(x), layer, ids, wts, np_f(res)), atol_frac=Y_ATOL,
                          what=f"E256 I512 fused step {step}")
    assert not moe_fused_timed_out(dev)


def test_one_launch_layer_add_norm_and_next_qkv(dev, layer):
    """add + RMSNorm in front, and the next layer's RMS-folded 3072 x 2048 QKV
    projection from y in the same launch (the bits of ternary_gemv on y)."""
    a = synthetic.randn_bf16((1, H), 51, dev)
    b = synthetic.randn_bf16((1, H), 52, dev)
    nw = (torch.rand(H, device=dev) + 0.5).float()
    qkv_w, qkv_a = synthetic.ternary_linear(3072, H, 53, dev)
    rms = torch.ones(H, device=dev)
    out = moe_fused(a, layer, K, add=b, norm_weight=nw, eps=1e-6, next_linear=(qkv_w, qkv_a, rms, 1e-6))
    torch.cuda.synchronize()
    y, ids, wts, nxt = out[0], out[1], out[2], out[3]
    s = np_f(a) + np_f(b)
    xn = s / np.sqrt(np.mean(s * s, axis=-1, keepdims=True) + 1e-6) * np_f(nw)
    xn = np_f(torch.from_numpy(xn).to(torch.bfloat16))
    res = np_f(torch.from_numpy(s).to(torch.bfloat16))
    assert_bf16_close(np_f(y), _oracle_y(xn, layer, ids, wts, res), atol_frac=Y_ATOL, what="add+norm")
    want = ternary_gemv(y, qkv_w, qkv_a, rms_weight=rms, rms_eps=1e-6)
    assert torch.equal(nxt, want)


@pytest.mark.parametrize("tokens", [2, 3, 8, 32])
def test_moe_block_decode_batches(dev, layer, tokens):
    x = synthetic.randn_bf16((tokens, H), 60 + tokens, dev)
    res = synthetic.randn_bf16((tokens, H), 70 + tokens, dev)
    y, ids, wts = moe_block(x, layer, K, residual=res)
    torch.cuda.synchronize()
    assert_bf16_close(np_f(y), _oracle_y(np_f(x), layer, ids, wts, np_f(res)), atol_frac=Y_ATOL,
                      what=f"E256 I512 T{tokens}")


def test_moe_block_prefill_chunk(dev, layer):
    tokens = 2048
    x = synthetic.randn_bf16((tokens, H), 99, dev)
    y, ids, wts = moe_block(x, layer, K)
    torch.cuda.synchronize()
    rows = np.r_[0:96, tokens - 32:tokens]  # the oracle on a subset of the chunk's tokens
    ref = _oracle_y(np_f(x)[rows], layer, ids[rows], wts[rows])
    assert_bf16_close(np_f(y)[rows], ref, atol_frac=Y_ATOL, what="E256 I512 T2048")
    y2, _, _ = moe_block(x, layer, K)
    assert torch.equal(y, y2)  # fixed-order sums: run to run the same bits


@pytest.mark.parametrize("batch", [1, 32])
def test_rtn4_head_full_vocab_group64(dev, batch):
    vocab = 151936
    w, sc, bs = synthetic.rtn4_table(vocab, H, 64, 81, dev, 0.003, 0.006)
    x = synthetic.randn_bf16((batch, H), 82, dev)
    y = rtn4_gemv(x, w, sc, bs, group_size=64)
    torch.cuda.synchronize()
    rows = np.r_[0:2048, vocab - 2048:vocab]
    wn = np_u32(w)[rows]
    ref = ok.rtn4_gemv(np_f(x), wn, np_f(sc)[rows], np_f(bs)[rows], group_size=64)
    assert_bf16_close(np_f(y)[:, rows], ref, what=f"rtn4 head g64 B{batch}")


@pytest.mark.timeout(600)
def test_maple_shaped_checkpoint_decodes_vs_oracle(dev, tmp_path, capsys):
    """Layer by layer (each device layer's output against the oracle's layer
    on the same device input, the device's routing and the device's cache
    rows): cosine >= 0.9999 per row, max error <= 1e-2 of the row's scale,
    the expert ids equal the oracle's own where the k-th and (k+1)-th
    probabilities are more than 1e-3 apart; the head's logits on the device's
    final hidden state meet the logits bar; ``forward`` gives the same logits
    bit for bit.  End to end (the oracle run on its own states) cosine >=
    0.999: four random layers amplify bf16 rounding (measured 0.99982 at
    batch 1)."""
    from maple_amd import checkpoint
    from oracle import decoder as od
    from test_gpu_decoder import _check_logits, _cos

    model = SyntheticDecoder(MAPLE, dev, seed=12, max_len=640)
    checkpoint.save_decoder(model, tmp_path)
    back = checkpoint.load_decoder(tmp_path, dev, max_len=640)
    assert dataclasses.asdict(back.cfg) == dataclasses.asdict(dataclasses.replace(MAPLE, lm_scale=back.cfg.lm_scale))
    assert back.layers[0].qkv.shape == (3072, 128) and back.layers[0].moe.up_gate_packed.shape == (256, 1024, 128)
    m = _to_np(back)
    oc = dict(m["cfg"], cos=m["cos"], sin=m["sin"])
    c = back.cfg
    for batch in (1, 3, 20):
        cache = back.make_cache(batch, prefill_len=600, seed=7)
        cache_fw = back.make_cache(batch, prefill_len=600, seed=7)
        ids = torch.arange(batch, device=dev) * 211 % c.vocab
        h = back.embed_tokens(ids)
        h_e2e = np_f(h)
        e2e_cache = dict(k=[np_f(k).astype(np.float32) for k in cache.k],
                         v=[np_f(v).astype(np.float32) for v in cache.v], seqlen=cache.seqlen.cpu().numpy().copy())
        for i in range(c.layers):
            cnp = dict(k=[None] * i + [np_f(cache.k[i]).astype(np.float32)],
                       v=[None] * i + [np_f(cache.v[i]).astype(np.float32)], seqlen=cache.seqlen.cpu().numpy().copy())
            routing = []
            out = back.layer_step(i, h, cache, routing)
            rid = routing[0].cpu().numpy()
            ref, (own, probs) = od.decoder_layer(m["layers"][i], oc, np_f(h), cnp, i, router_ids=rid)
            y = np_f(out)
            for b in range(batch):
                assert _cos(y[b], ref[b]) >= 0.9999, f"batch {batch} layer {i} row {b}: cosine {_cos(y[b], ref[b]):.6f}"
                assert np.abs(y[b] - ref[b]).max() <= 1e-2 * np.abs(ref[b]).max(), f"layer {i} row {b}: max err"
                p = np.sort(probs[b])[::-1]
                if p[c.top_k - 1] - p[c.top_k] > 1e-3:
                    np.testing.assert_array_equal(np.sort(rid[b]), np.sort(own[b]), err_msg=f"layer {i} row {b} ids")
            h_e2e, _ = od.decoder_layer(m["layers"][i], oc, h_e2e, e2e_cache, i, router_ids=rid)
            h = out
        cache.seqlen.add_(1)
        logits = back.head(h)
        torch.cuda.synchronize()
        _check_logits(logits, od.final_logits(m, np_f(h)), f"maple shapes batch {batch} head")
        ref_e2e = od.final_logits(m, h_e2e)
        for b in range(batch):
            cos = _cos(np_f(logits[b]), ref_e2e[b])
            assert cos >= 0.999, f"batch {batch} row {b}: end-to-end cosine {cos:.6f}"
        assert torch.equal(back.forward(ids, cache_fw), logits)
        assert torch.equal(cache_fw.seqlen, cache.seqlen)
        with capsys.disabled():
            print(f"  maple shapes batch {batch}: every layer matches the oracle", flush=True)
    assert not moe_fused_timed_out(dev)
