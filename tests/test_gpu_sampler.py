"""HIP fused sampler (kernels/sampler.py, ``ma_fused_sample``) against the
sampler oracle (oracle/sampler.py): the drawn id must equal the oracle's,
except where the oracle's ``u * total`` lies within 1e-5 (relative) of a CDF
step, where float32 summation order may put it on either side.  Cases follow
the reference's tests/test_fused_sampler.py."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import sampler as osm

pytestmark = pytest.mark.gpu

VOCAB = 151936


def _check_rows(logits: torch.Tensor, u: torch.Tensor, got: torch.Tensor, *, temperature, top_p, top_k):
    x = logits.float().cpu().numpy().reshape(-1, logits.shape[-1])
    uu = u.float().cpu().numpy().reshape(-1)
    g = got.cpu().numpy().reshape(-1)
    for b in range(x.shape[0]):
        want = osm.sample_row(x[b], float(uu[b]), temperature=temperature, top_p=top_p, top_k=top_k)
        if int(g[b]) != want:
            margin = osm.pick_margin(x[b], float(uu[b]), temperature=temperature, top_p=top_p, top_k=top_k)
            assert margin < 1e-5, (b, int(g[b]), want, margin)


@pytest.mark.parametrize("top_k", [2, 20, 64])
@pytest.mark.parametrize("top_p", [0.95, 1.0])
def test_fused_sample_inverts_the_same_cdf(dev, top_k, top_p):
    from maple_amd.kernels.sampler import fused_sample, sampler_workspace

    gen = torch.Generator().manual_seed(0)
    ws = sampler_workspace(VOCAB, top_k, dev)
    for trial in range(4):
        logits = (torch.randn(VOCAB, generator=gen) * 3.0).to(dev)
        for u_val in (0.0, 0.25, 0.5, 0.75, 0.999):
            u = torch.tensor(u_val, device=dev)
            got = fused_sample(logits, u, temperature=0.8, top_p=top_p, top_k=top_k, workspace=ws)
            _check_rows(logits, u, got, temperature=0.8, top_p=top_p, top_k=top_k)


def test_fused_sample_respects_the_nucleus(dev):
    from maple_amd.kernels.sampler import fused_sample

    logits = torch.full((VOCAB,), -20.0, device=dev)
    logits[7], logits[11], logits[13] = 10.0, 2.0, 1.0
    drawn = {int(fused_sample(logits, torch.tensor(i / 64.0, device=dev), temperature=1.0, top_p=0.9,
                              top_k=20)) for i in range(64)}
    assert drawn == {7}, drawn


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("top_k", [1, 20, 64])
@pytest.mark.parametrize("top_p", [0.3, 0.95, 1.0])
def test_batched_sampler_matches_oracle_and_per_row(dev, dtype, top_k, top_p):
    """bf16 logits tie often over 152k values: the lower index must win, as
    in the oracle; every row draws bit-exactly what it draws alone."""
    from maple_amd.kernels.sampler import fused_sample, fused_sample_batched

    gen = torch.Generator().manual_seed(4)
    bsz = 9
    logits = (torch.randn(bsz, VOCAB, generator=gen) * 4).to(dtype).to(dev)
    u = torch.rand(bsz, generator=gen).to(dev)
    got = fused_sample_batched(logits, u, temperature=0.8, top_p=top_p, top_k=top_k)
    want = torch.stack([fused_sample(logits[b].contiguous(), u[b], temperature=0.8, top_p=top_p, top_k=top_k)
                        for b in range(bsz)])
    assert torch.equal(got, want)
    _check_rows(logits, u, got, temperature=0.8, top_p=top_p, top_k=top_k)


@pytest.mark.parametrize("vocab", [64, 100, 4096, 4097, 12289])
def test_small_and_ragged_vocab(dev, vocab):
    from maple_amd.kernels.sampler import fused_sample_batched

    gen = torch.Generator().manual_seed(vocab)
    logits = torch.randn(3, vocab, generator=gen).to(dev)
    u = torch.tensor([0.05, 0.5, 0.95], device=dev)
    for k in sorted({1, min(vocab, 7), min(vocab, 64)}):
        got = fused_sample_batched(logits, u, temperature=1.3, top_p=0.9, top_k=k)
        _check_rows(logits, u, got, temperature=1.3, top_p=0.9, top_k=k)


def test_top1_equals_greedy_argmax(dev):
    from maple_amd.kernels.greedy import greedy_argmax
    from maple_amd.kernels.sampler import fused_sample_batched

    gen = torch.Generator().manual_seed(9)
    logits = (torch.randn(5, VOCAB, generator=gen) * 2).to(torch.bfloat16).to(dev)
    u = torch.rand(5, generator=gen).to(dev)
    got = fused_sample_batched(logits, u, temperature=1.0, top_p=1.0, top_k=1)
    assert torch.equal(got, greedy_argmax(logits))


def test_distribution_tracks_the_probabilities(dev):
    from maple_amd.kernels.sampler import fused_sample_batched

    gen = torch.Generator().manual_seed(2)
    row = torch.randn(VOCAB, generator=gen) * 2.0
    n = 4000
    logits = row.to(dev).expand(n, VOCAB).contiguous()
    u = ((torch.arange(n, dtype=torch.float32) + 0.5) / n).to(dev)
    got = fused_sample_batched(logits, u, temperature=1.0, top_p=0.95, top_k=20).cpu().numpy()
    vals, idx = torch.topk(row, 20)
    probs = torch.softmax(vals.double(), dim=-1)
    sp = torch.cumsum(probs, 0)
    keep = (sp - probs) <= 0.95
    probs = torch.where(keep, probs, torch.zeros_like(probs))
    probs = (probs / probs.sum()).numpy()
    freq = np.array([(got == int(j)).mean() for j in idx.numpy()])
    np.testing.assert_allclose(freq, probs, atol=2.0 / n + 1e-4)


def test_sampler_rejects_unsupported_settings(dev):
    from maple_amd.kernels.sampler import MAX_TOP_K, fused_sample

    logits = torch.randn(VOCAB, device=dev)
    u = torch.tensor(0.5, device=dev)
    for kw in (dict(temperature=1.0, top_p=0.95, top_k=0), dict(temperature=0.0, top_p=0.95, top_k=20),
               dict(temperature=1.0, top_p=0.95, top_k=MAX_TOP_K + 1), dict(temperature=1.0, top_p=0.0, top_k=5),
               dict(temperature=1.0, top_p=1.5, top_k=5)):
        with pytest.raises(ValueError):
            fused_sample(logits, u, **kw)
    with pytest.raises(ValueError):
        fused_sample(torch.randn(10, device=dev), u, temperature=1.0, top_p=1.0, top_k=11)


def test_sampler_graph_replay_matches_eager(dev):
    from maple_amd.kernels.sampler import batched_sampler_workspace, fused_sample_batched

    gen = torch.Generator().manual_seed(11)
    bsz = 4
    logits = (torch.randn(bsz, VOCAB, generator=gen) * 3).to(dev)
    u = torch.rand(bsz, generator=gen).to(dev)
    ws = batched_sampler_workspace(VOCAB, 20, bsz, dev)
    eager = fused_sample_batched(logits, u, temperature=0.7, top_p=0.9, top_k=20, workspace=ws).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fused_sample_batched(logits, u, temperature=0.7, top_p=0.9, top_k=20, workspace=ws)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fused_sample_batched(logits, u, temperature=0.7, top_p=0.9, top_k=20, workspace=ws)
    for i in range(3):
        u.copy_(torch.rand(bsz, generator=gen).to(dev))
        want = fused_sample_batched(logits, u, temperature=0.7, top_p=0.9, top_k=20).clone()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), i
    u.copy_(torch.zeros(bsz))
    g.replay()
    assert torch.equal(out, fused_sample_batched(logits, u, temperature=0.7, top_p=0.9, top_k=20))
    assert eager.shape == (bsz,)
