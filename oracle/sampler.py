"""Fused top-k / temperature / nucleus sampling, float32 NumPy (test
infrastructure only: the product never imports it).

Restates the reference's two-launch sampler, ``src/maple_run/kernels/sampler.py``:

* ``_topk_partial_kernel`` / the merge in ``_sample_final_kernel`` (:24-53,
  :73-83): the top_k largest logits of a row, descending, equal values at the
  lower index first (repeated argmax takes the first maximum);
* ``_sample_final_kernel`` (:85-103): ``p = exp((v - v_max) / T)`` over those,
  normalised; the nucleus keeps a token while the mass before it is at most
  ``top_p``; ``u = uniform * (kept mass)``; the pick is the number of kept
  inclusive prefixes ``<= u``, capped at ``top_k - 1``.

Pinned in tests/test_oracle_sampler.py against the reference test's own chain
(``tests/test_fused_sampler.py:14-50``: ``torch.topk`` -> softmax ->
``generate._nucleus`` -> CDF inversion), its nucleus case (:53-67), a
brute-force distribution over a uniform grid, and argmax at ``top_k = 1``.
"""

from __future__ import annotations

import numpy as np


def topk_desc(row: np.ndarray, k: int) -> np.ndarray:
    """Indices of the ``k`` largest values, descending, ties at the lower index."""
    order = np.lexsort((np.arange(row.shape[0]), -row.astype(np.float64)))
    return order[:k]


def sample_row(row, u: float, *, temperature: float, top_p: float, top_k: int, detail: bool = False):
    """The id drawn from one row of float32 logits at uniform ``u``."""
    x = np.asarray(row, np.float32)
    idx = topk_desc(x, top_k)
    kv = x[idx]
    inv_t = np.float32(1.0 / float(temperature))
    p = np.exp((kv - kv[0]) * inv_t).astype(np.float32)
    p = (p / p.sum(dtype=np.float32)).astype(np.float32)
    cum = np.cumsum(p, dtype=np.float32)
    p = np.where(cum - p <= np.float32(top_p), p, np.float32(0)).astype(np.float32)
    total = p.sum(dtype=np.float32)
    cum = np.cumsum(p, dtype=np.float32)
    uu = np.float32(u) * total
    pick = min(int((cum <= uu).sum()), top_k - 1)
    if detail:
        return int(idx[pick]), dict(idx=idx, p=p, cum=cum, u=uu, pick=pick)
    return int(idx[pick])


def fused_sample(logits, uniform, *, temperature: float, top_p: float, top_k: int) -> np.ndarray:
    """One id per row of ``logits [B, V]`` (or a 1-D row) at ``uniform [B]``."""
    x = np.asarray(logits, np.float32)
    x2 = x.reshape(-1, x.shape[-1])
    u = np.asarray(uniform, np.float32).reshape(-1)
    out = np.array([sample_row(x2[b], float(u[b]), temperature=temperature, top_p=top_p, top_k=top_k)
                    for b in range(x2.shape[0])], np.int64)
    return out.reshape(x.shape[:-1])


def pick_margin(row, u: float, *, temperature: float, top_p: float, top_k: int) -> float:
    """Distance of ``u * total`` from the nearest kept CDF step, relative to the
    kept mass: a draw this close to a boundary may round either way."""
    _, d = sample_row(row, u, temperature=temperature, top_p=top_p, top_k=top_k, detail=True)
    kept = d["cum"][d["p"] > 0]
    total = float(d["cum"][-1]) if d["cum"].size else 1.0
    return float(np.min(np.abs(kept - d["u"]))) / max(total, 1e-30)
