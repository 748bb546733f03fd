"""FlashHead on the HIP kernels (maple_amd.flash_head, ``ma_flash_head``,
``ma_rtn4_indexed_gemv``) vs the exact head and the oracle (needs the GPU).

* ``rtn4_indexed_gemv`` gives ``rtn4_gemv``'s bits for the gathered rows, and
  the oracle's values within the bf16 bar;
* the centroid scores are ``rtn4_gemv``'s bits; the probed clusters are the
  oracle's selection on those scores exactly (ties at the lower index);
  every finite logit is the exact head's bits, every other one -inf, forced
  tokens always present;
* all clusters probed = the exact head (reference
  tests/test_flash_head.py:88-112); a decoder at batch > 1 keeps the exact
  head (:114-136); a checkpoint loaded without ``flash_head`` ignores the
  tensors (:138-155); graph replays equal eager calls;
* at the full size (151936 tokens in 4748 clusters of 32, 512 probes,
  hidden 2048, group 64) the same bits-and-selection checks.
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from _helpers import assert_bf16_close, np_f, np_u32
from maple_amd import synthetic
from maple_amd.flash_head import FlashHead
from maple_amd.kernels import rtn4_gemv, rtn4_indexed_gemv
from oracle import flash_head as ofh
from oracle import kernels as ok
from oracle import pack

pytestmark = pytest.mark.gpu


def _flash(dev, lm_head, n_clusters, n_probes, *, seed=0, force=(), group=64, from_means=True):
    """A FlashHead over ``lm_head`` with a random token permutation split into
    clusters and centroids quantised from the members' mean rows (or random
    rows), built the way ``build_flash_head`` permutes the head."""
    w, sc, bs = lm_head
    vocab, nwords = w.shape
    hidden = nwords * 8
    rng = np.random.default_rng(seed)
    tm = rng.permutation(vocab).astype(np.int32).reshape(n_clusters, vocab // n_clusters)
    if from_means:
        dense = pack.dequantize_rtn(np_u32(w), np_f(sc).astype(np.float32), np_f(bs).astype(np.float32), group)
        rows = dense[tm].mean(axis=1).astype(np.float32)
    else:
        rows = rng.standard_normal((n_clusters, hidden)).astype(np.float32)
    cw, cs, cb = pack.quantize_rtn(rows, group_size=64)
    order = torch.from_numpy(tm.reshape(-1).astype(np.int64)).to(dev)
    fid = torch.tensor(list(force), device=dev, dtype=torch.int64)
    fh = FlashHead(
        centroids_weight=torch.from_numpy(cw.view(np.int32)).to(dev).view(torch.uint32),
        centroids_scales=torch.from_numpy(cs).to(dev).to(torch.bfloat16),
        centroids_biases=torch.from_numpy(cb).to(dev).to(torch.bfloat16),
        token_map=torch.from_numpy(tm).to(dev),
        head_weight=w.view(torch.int32).index_select(0, order).view(torch.uint32).reshape(n_clusters, -1, nwords),
        head_scales=sc.index_select(0, order).reshape(n_clusters, vocab // n_clusters, -1),
        head_biases=bs.index_select(0, order).reshape(n_clusters, vocab // n_clusters, -1),
        force_ids=fid,
        force_weight=w.view(torch.int32).index_select(0, fid).view(torch.uint32) if len(force) else None,
        force_scales=sc.index_select(0, fid) if len(force) else None,
        force_biases=bs.index_select(0, fid) if len(force) else None,
        n_probes=n_probes, vocab_size=vocab, group_size=group, device=dev)
    return fh, tm, (cw, np_f(fh.centroids_scales), np_f(fh.centroids_biases))


def _check(fh, tm, cent, lm_head, x, n_probes, force=()):
    w, sc, bs = lm_head
    out = fh(x.reshape(1, 1, -1)).reshape(-1)
    exact = rtn4_gemv(x.reshape(1, -1), w, sc, bs, group_size=fh.group_size).reshape(-1)
    scores = rtn4_gemv(x.reshape(1, -1), fh.centroids_weight, fh.centroids_scales, fh.centroids_biases,
                       group_size=fh.centroid_group_size).reshape(-1)
    torch.cuda.synchronize()
    sel = ofh.select_clusters(np_f(scores), n_probes)
    np.testing.assert_array_equal(fh.cluster_ids.cpu().numpy(), sel)
    finite = torch.zeros_like(exact, dtype=torch.bool)
    finite[torch.from_numpy(tm[sel].reshape(-1).astype(np.int64)).to(x.device)] = True
    if len(force):
        finite[torch.tensor(list(force), device=x.device)] = True
    assert torch.equal(out[finite], exact[finite])
    assert bool(torch.isneginf(out[~finite].float()).all())
    # and the oracle on the same scores' ordering (values within the bf16 bar)
    ref, rsel, _ = ofh.flash_head_logits(np_f(x), cent, (np_u32(fh.head_weight), np_f(fh.head_scales),
                                                        np_f(fh.head_biases)), tm, n_probes, tm.size,
                                         head_group=fh.group_size)
    common = np.intersect1d(sel, rsel)
    assert len(common) >= n_probes - 2  # near-equal scores may sit on either side of the cut
    toks = tm[common].reshape(-1)
    assert_bf16_close(np_f(out)[toks], ref[toks], what="flash head probed logits")
    return out


def test_indexed_gemv_is_rtn4_gemv_on_the_gathered_rows(dev):
    vocab, hidden = 4096, 2048
    w, sc, bs = synthetic.rtn4_table(vocab, hidden, 64, 5, dev, 0.003, 0.006)
    head_w = w.reshape(128, 32, -1)
    ids = torch.tensor([5, 0, 127, 64, 5], device=dev, dtype=torch.int32)
    for batch in (1, 3):
        x = synthetic.randn_bf16((batch, hidden), 6 + batch, dev)
        y = rtn4_indexed_gemv(x, head_w, sc.reshape(128, 32, -1), bs.reshape(128, 32, -1), ids, group_size=64)
        full = rtn4_gemv(x, w, sc, bs, group_size=64) if batch < 5 else None
        rows = (ids.long()[:, None] * 32 + torch.arange(32, device=dev)[None, :]).reshape(-1)
        assert torch.equal(y, full[:, rows])
        ref = ok.rtn4_gemv(np_f(x), np_u32(w)[rows.cpu().numpy()], np_f(sc)[rows.cpu().numpy()],
                           np_f(bs)[rows.cpu().numpy()], group_size=64)
        assert_bf16_close(np_f(y), ref, what=f"indexed gemv B{batch}")


@pytest.mark.parametrize("n_probes", [1, 8, 32, 64])
def test_flash_head_small_vs_exact_and_oracle(dev, n_probes):
    vocab, hidden = 2048, 2048
    head = synthetic.rtn4_table(vocab, hidden, 64, 11, dev, 0.003, 0.006)
    fh, tm, cent = _flash(dev, head, 64, n_probes, seed=n_probes, force=(3, 2047))
    for i in range(3):
        x = synthetic.randn_bf16((1, hidden), 20 + i, dev)
        _check(fh, tm, cent, head, x, n_probes, force=(3, 2047))


def test_all_probes_is_the_exact_head(dev):
    vocab, hidden = 2048, 2048
    head = synthetic.rtn4_table(vocab, hidden, 64, 12, dev, 0.003, 0.006)
    fh, _, _ = _flash(dev, head, 64, 64, seed=1, from_means=False)
    x = synthetic.randn_bf16((1, hidden), 30, dev)
    out = fh(x)
    assert torch.equal(out.reshape(-1), rtn4_gemv(x, *head, group_size=64).reshape(-1))


def test_flash_head_graph_replays_match_eager(dev):
    vocab, hidden = 8192, 2048
    head = synthetic.rtn4_table(vocab, hidden, 64, 13, dev, 0.003, 0.006)
    fh, _, _ = _flash(dev, head, 256, 16, seed=2, force=(7,))
    x = synthetic.randn_bf16((1, hidden), 40, dev)
    out = torch.empty(vocab, device=dev, dtype=torch.bfloat16)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fh(x, out=out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fh(x, out=out)
    for i in range(3):
        x.copy_(synthetic.randn_bf16((1, hidden), 41 + i, dev))
        want = fh(x).reshape(-1).clone()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), i
        torch.zeros(1, device=dev).add_(1)


@pytest.mark.timeout(300)
def test_flash_head_at_full_size(dev):
    """151936 tokens in 4748 clusters of 32, 512 probes, hidden 2048, group 64,
    one forced token."""
    vocab, hidden, n_clusters, n_probes = 151936, 2048, 4748, 512
    head = synthetic.rtn4_table(vocab, hidden, 64, 14, dev, 0.003, 0.006)
    fh, tm, cent = _flash(dev, head, n_clusters, n_probes, seed=3, force=(151643,), from_means=False)
    x = synthetic.randn_bf16((1, hidden), 50, dev)
    w, sc, bs = head
    out = fh(x).reshape(-1)
    exact = rtn4_gemv(x, w, sc, bs, group_size=64).reshape(-1)
    scores = rtn4_gemv(x, fh.centroids_weight, fh.centroids_scales, fh.centroids_biases, group_size=64).reshape(-1)
    torch.cuda.synchronize()
    sel = ofh.select_clusters(np_f(scores), n_probes)
    np.testing.assert_array_equal(fh.cluster_ids.cpu().numpy(), sel)
    finite = torch.zeros(vocab, device=dev, dtype=torch.bool)
    finite[torch.from_numpy(tm[sel].reshape(-1).astype(np.int64)).to(dev)] = True
    finite[151643] = True
    assert int(finite.sum()) in (n_probes * 32, n_probes * 32 + 1)
    assert torch.equal(out[finite], exact[finite])
    assert bool(torch.isneginf(out[~finite].float()).all())


def test_checkpoint_flash_head_decode(dev, tmp_path):
    """A checkpoint with FlashHead tensors: loaded with ``flash_head`` the
    batch-1 logits are the exact head's on the probed tokens (all probed:
    everywhere) and -inf elsewhere; batch 2 keeps the exact head; loaded
    without it the tensors are ignored."""
    from safetensors.torch import save_file

    from maple_amd import checkpoint
    from maple_amd.model import DecoderConfig, SyntheticDecoder

    cfg = DecoderConfig(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64, experts=8, inter=256, top_k=2,
                        vocab=1024, rtn_group=64, lm_scale=(0.01, 0.02))
    model = SyntheticDecoder(cfg, dev, seed=3, max_len=64)
    checkpoint.save_decoder(model, tmp_path)
    _, tm, (cw, cs, cb) = _flash(dev, model.lm_head, 32, 32, seed=4)
    save_file({"lm_head_flash.token_map": torch.from_numpy(tm),
               "lm_head_flash.centroids.weight": torch.from_numpy(cw.view(np.int32)),
               "lm_head_flash.centroids.scales": torch.from_numpy(cs.astype(np.float32)),
               "lm_head_flash.centroids.biases": torch.from_numpy(cb.astype(np.float32))},
              str(tmp_path / "model-flashhead.safetensors"))
    conf = json.loads((tmp_path / "config.json").read_text())
    meta = {"n_clusters": 32, "cluster_size": 32, "n_probes": 32, "group_size": 64, "bits": 4,
            "head_group_size": 64, "head_bits": 4, "scaled_centroids": True, "force_tokens": []}
    conf["flash_head"] = meta
    conf["maple_run"]["flash_head"] = meta
    (tmp_path / "config.json").write_text(json.dumps(conf))
    exact = checkpoint.load_decoder(tmp_path, dev, max_len=64)
    assert exact.flash_head is None
    flash = checkpoint.load_decoder(tmp_path, dev, max_len=64, flash_head=True)
    assert flash.flash_head is not None and flash.flash_head.n_probes == 32
    ids = torch.tensor([17], device=dev)
    ce, cf = exact.make_cache(1, 9, seed=2), flash.make_cache(1, 9, seed=2)
    le, lf = exact.forward(ids, ce), flash.forward(ids, cf)
    assert bool(torch.isfinite(lf.float()).all()) and torch.equal(lf, le)
    ce2, cf2 = exact.make_cache(2, 9, seed=2), flash.make_cache(2, 9, seed=2)
    ids2 = torch.tensor([17, 400], device=dev)
    assert torch.equal(flash.forward(ids2, cf2), exact.forward(ids2, ce2))
    # fewer probes: finite exactly on the probed clusters, the exact bits there
    flash.flash_head = _flash(dev, flash.lm_head, 32, 4, seed=4)[0]
    cf3 = flash.make_cache(1, 9, seed=2)
    lf3 = flash.forward(ids, cf3).reshape(-1)
    fin = torch.isfinite(lf3.float())
    assert int(fin.sum()) == 4 * 32 and torch.equal(lf3[fin], le.reshape(-1)[fin])
