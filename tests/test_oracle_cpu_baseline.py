"""The CPU-baseline path (oracle/cpu_baseline.py, float32 torch) against the
float64 oracle (CPU).  Both restate the same reference functions; the baseline
carries no intermediate bf16 rounding, so it is compared with the oracle's
unrounded forms at float32 tolerance, and the decoder token by logits cosine.
"""

from __future__ import annotations

import numpy as np
import torch

from _helpers import tie_safe_rows
from oracle import cpu_baseline as cb
from oracle import decoder as od
from oracle import kernels as ok
from oracle import pack
from test_oracle_composition import _cache, _tiny_model


def _experts(rng, e_n, hid, inter):
    ug = pack.pack_2bit(rng.integers(0, 3, (e_n, 2 * inter, hid), dtype=np.uint32))
    ug_a = rng.uniform(0.01, 0.05, (e_n, 2 * inter)).astype(np.float32)
    dn = pack.pack_2bit(rng.integers(0, 3, (e_n, hid, inter), dtype=np.uint32))
    dn_a = rng.uniform(0.01, 0.05, (e_n, hid)).astype(np.float32)
    return ug, ug_a, dn, dn_a


def test_gemv_and_rtn4_match_the_oracle():
    rng = np.random.default_rng(30)
    packed = pack.pack_2bit(rng.integers(0, 3, (96, 256), dtype=np.uint32))
    alpha = rng.uniform(0.01, 0.05, 96).astype(np.float32)
    x = rng.standard_normal((3, 256)).astype(np.float32)
    np.testing.assert_allclose(cb.ternary_gemv(x, packed, alpha).numpy(), ok.ternary_gemv(x, packed, alpha),
                               rtol=1e-4, atol=1e-5)
    codes = rng.integers(0, 16, (40, 256), dtype=np.uint32)
    sc = rng.uniform(0.01, 0.03, (40, 4)).astype(np.float32)
    bs = rng.uniform(-0.2, 0.0, (40, 4)).astype(np.float32)
    np.testing.assert_allclose(cb.rtn4_gemv(x, pack.pack_4bit(codes), sc, bs, 64, chunk_rows=16).numpy(),
                               ok.rtn4_gemv(x, pack.pack_4bit(codes), sc, bs, group_size=64), rtol=1e-4, atol=1e-5)


def test_moe_layer_matches_the_oracle_block():
    rng = np.random.default_rng(31)
    e_n, hid, inter, k, t = 8, 128, 64, 3, 12
    gw = (rng.standard_normal((e_n, hid)) * 0.3).astype(np.float32)
    ug, ug_a, dn, dn_a = _experts(rng, e_n, hid, inter)
    x = rng.standard_normal((t, hid)).astype(np.float32)
    bias = rng.standard_normal(e_n).astype(np.float32)
    res = rng.standard_normal((t, hid)).astype(np.float32)
    ids, wts = cb.router(x, gw, k, bias)
    rid, rw, probs = ok.router_topk(x, gw, k, bias=bias)
    safe = tie_safe_rows(probs, k)
    np.testing.assert_array_equal(ids.numpy()[safe], rid[safe])
    np.testing.assert_allclose(wts.numpy(), rw, rtol=1e-5, atol=1e-7)
    y = cb.moe_layer(x, gw, ug, ug_a, dn, dn_a, k, bias=bias, residual=res).numpy()
    ref, _, _, _ = ok.moe_block(x, gw, ug, ug_a, dn, dn_a, k, residual=res, router_bias=bias, round_bf16=False)
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())


def test_decoder_token_matches_the_oracle_step():
    rng = np.random.default_rng(32)
    m = _tiny_model(rng, layers=2, zero_q_k=False, zero_o=False, zero_experts=False)
    for L in m["layers"]:
        L["moe"]["gate_weight"] = od.bf(np.random.default_rng(33).standard_normal(L["moe"]["gate_weight"].shape))
    cache = _cache(np.random.default_rng(34), m, 1, 9)
    cache32 = dict(k=[a.astype(np.float32) for a in cache["k"]], v=[a.astype(np.float32) for a in cache["v"]],
                   seqlen=cache["seqlen"].copy())
    ref, routing = od.decoder_step(m, cache, np.array([5]))
    got = cb.decoder_token(m, cache32, 5).numpy()
    cos = float(np.dot(got, ref[0]) / (np.linalg.norm(got) * np.linalg.norm(ref[0])))
    assert cos >= 0.999, cos
    np.testing.assert_array_equal(cache32["seqlen"], cache["seqlen"])
    # the K/V written at the old position agree (up to the oracle's bf16 stores)
    np.testing.assert_allclose(cache32["v"][1][0, :, 9], cache["v"][1][0, :, 9], rtol=2 ** -7, atol=1e-2)
    assert torch.is_tensor(cb.rms_norm(np.ones(4), np.ones(4), 1e-6))
