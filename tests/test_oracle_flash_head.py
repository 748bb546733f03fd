"""The FlashHead oracle (oracle/flash_head.py) against independent checks (CPU):
every cluster probed gives the exact head; with fewer probes a token's logit
is finite exactly when a brute-force ranking of the centroid scores (written
here from the dequantised centroid rows) puts its cluster among the best;
ties at the cut go to the lower cluster index; forced tokens always carry
their exact logit.  Reference behaviour: src/maple_run/flash_head.py:334-370
and tests/test_flash_head.py:88-112."""

from __future__ import annotations

import numpy as np

from oracle import flash_head as ofh
from oracle import kernels as ok
from oracle import pack
from oracle.decoder import bf

H, V, G = 128, 96, 64


def _head(rng, n=V):
    codes = rng.integers(0, 16, (n, H), dtype=np.uint32)
    sc = rng.uniform(0.01, 0.03, (n, H // G)).astype(np.float32)
    bs = rng.uniform(-0.2, 0.0, (n, H // G)).astype(np.float32)
    return pack.pack_4bit(codes), sc, bs


def _case(seed, n_clusters=12):
    rng = np.random.default_rng(seed)
    w, s, b = _head(rng)
    tm = rng.permutation(V).astype(np.int32).reshape(n_clusters, V // n_clusters)
    cw, cs, cb = pack.quantize_rtn(rng.standard_normal((n_clusters, H)).astype(np.float32), group_size=G)
    order = tm.reshape(-1)
    head = (w[order].reshape(n_clusters, V // n_clusters, -1), s[order].reshape(n_clusters, V // n_clusters, -1),
            b[order].reshape(n_clusters, V // n_clusters, -1))
    x = rng.standard_normal(H)
    return x, (w, s, b), (cw, cs, cb), head, tm


def test_all_probes_is_the_exact_head():
    x, full, cent, head, tm = _case(0)
    out, sel, _ = ofh.flash_head_logits(x, cent, head, tm, tm.shape[0], V)
    np.testing.assert_array_equal(sel, np.arange(tm.shape[0]))
    np.testing.assert_array_equal(out, bf(ok.rtn4_gemv(x[None], *full, group_size=G))[0])


def test_probed_set_matches_a_brute_force_ranking():
    for seed in range(1, 6):
        x, full, cent, head, tm = _case(seed)
        for n_probes in (1, 3, 7):
            out, sel, scores = ofh.flash_head_logits(x, cent, head, tm, n_probes, V)
            cw, cs, cb = cent
            dense = pack.dequantize_rtn(cw, cs, cb, group_size=G).astype(np.float64)
            sc = [float(bf(np.array([dense[c] @ x]))[0]) for c in range(tm.shape[0])]
            chosen = [c for c in range(tm.shape[0])
                      if sum(1 for d in range(tm.shape[0]) if sc[d] > sc[c] or (sc[d] == sc[c] and d < c)) < n_probes]
            assert list(sel) == chosen
            exact = bf(ok.rtn4_gemv(x[None], *full, group_size=G))[0]
            probed = set(tm[chosen].reshape(-1).tolist())
            for t in range(V):
                if t in probed:
                    assert out[t] == exact[t]
                else:
                    assert out[t] == -np.inf


def test_ties_at_the_cut_go_to_the_lower_cluster():
    x, full, cent, head, tm = _case(7)
    rng = np.random.default_rng(70)
    rows = rng.standard_normal((tm.shape[0], H)).astype(np.float32) * 0.1
    rows[[2, 5, 9]] = 10.0 * x  # three equal centroids, far ahead of the rest
    cent = pack.quantize_rtn(rows, group_size=G)
    _, sel, scores = ofh.flash_head_logits(x, cent, head, tm, 2, V)
    assert scores[2] == scores[5] == scores[9] and scores[2] > np.delete(scores, [2, 5, 9]).max()
    assert list(sel) == [2, 5]


def test_forced_tokens_keep_their_exact_logit():
    x, full, cent, head, tm = _case(8)
    w, s, b = full
    fid = np.array([tm[-1, 0], tm[-2, 3]])
    out, sel, _ = ofh.flash_head_logits(x, cent, head, tm, 1, V, force=(w[fid], s[fid], b[fid], fid))
    exact = bf(ok.rtn4_gemv(x[None], *full, group_size=G))[0]
    np.testing.assert_array_equal(out[fid], exact[fid])
    assert np.isfinite(out).sum() == tm.shape[1] + len(set(fid.tolist()) - set(tm[sel].reshape(-1).tolist()))
