"""Device ternarisation (``ma_ternarize``) against the oracle (needs the GPU).

The reference converter's ``ternarize`` (``src/maple_run/pack.py:120-149``) in
NumPy float32: the packed codes must be bit-exact and the row scales the same
bits (float32), or the float32 scale rounded to the weight dtype (bfloat16,
float16, as ``astype`` does).  Rows of several K, stacked [E, N, K] weights,
zero rows, negative zeros and rows crowded at the threshold.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from maple_amd.pack import ternarize
from oracle import pack as opack

pytestmark = pytest.mark.gpu


def _weights(shape, seed, dtype, dev):
    g = torch.Generator().manual_seed(seed)
    scale = 10.0 ** (torch.rand(shape[:-1] + (1,), generator=g) * 4 - 2)
    w = torch.randn(shape, generator=g) * scale
    return w.to(dtype).to(dev)


def _check(w):
    packed, alpha = ternarize(w)
    torch.cuda.synchronize()
    wf = w.float().cpu().numpy()
    rp, ra = opack.ternarize(wf)  # float32 arithmetic, float32 alpha
    np.testing.assert_array_equal(packed.cpu().numpy(), rp)
    ra_t = torch.from_numpy(np.ascontiguousarray(ra)).to(w.dtype)
    assert torch.equal(alpha.cpu().view(torch.int16 if w.dtype != torch.float32 else torch.int32),
                       ra_t.view(torch.int16 if w.dtype != torch.float32 else torch.int32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(64, 128), (37, 768), (96, 2048), (2, 3, 640), (5, 8192)])
def test_ternarize_bits_vs_oracle(dev, dtype, shape):
    _check(_weights(shape, hash(shape) % 1000, dtype, dev))


def test_ternarize_edge_rows(dev):
    """All-zero rows (alpha 0, every code 1), negative zeros (code 1), rows
    whose values sit on and around the threshold, a single survivor."""
    k = 256
    rows = [np.zeros(k, np.float32), -np.zeros(k, np.float32)]
    r = np.full(k, 1.0, np.float32)  # mean 1, thr 0.7: all kept
    rows.append(r)
    r = np.linspace(0.0, 1.0, k, dtype=np.float32) * np.where(np.arange(k) % 2, -1, 1).astype(np.float32)
    rows.append(r)
    r = np.zeros(k, np.float32)
    r[17] = -3.0  # one survivor
    rows.append(r)
    base = np.float32(0.7) * np.float32(0.5)
    r = np.full(k, 0.5, np.float32)
    r[::2] = np.nextafter(np.float32(0.5), np.float32(1))  # mean a hair above 0.5
    r[1::4] = base  # exactly 0.7 * 0.5, just under the threshold
    rows.append(r)
    w = torch.from_numpy(np.stack(rows)).to(dev)
    _check(w)


def test_ternarize_rejects_bad_k(dev):
    with pytest.raises(ValueError, match="multiple of 128"):
        ternarize(torch.ones(4, 64, device=dev))
