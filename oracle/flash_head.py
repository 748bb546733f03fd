"""FlashHead logits, NumPy (test infrastructure only: the product never
imports it).

Restates reference ``src/maple_run/flash_head.py`` ``FlashHead.__call__``
(:334-370): centroid scores = the RTN4 GEMV of the centroid rows, stored bf16
(``rtn4_gemv`` returns ``x.dtype``); the ``n_probes`` best clusters
(``torch.topk``; equal scores taken at the lower cluster index here, an
order torch leaves unspecified); the probed clusters' head rows
(``rtn4_indexed_gemv``, bf16) and the forced tokens' rows written into a
row of -inf (``fill_`` + ``index_put_``).  ``head`` is the lm_head permuted
by ``token_map`` (``build_flash_head`` :395-420), so row ``c * S + m`` is
token ``token_map[c, m]``.

Pinned in tests/test_oracle_flash_head.py: with every cluster probed the row
equals the exact head's logits; with fewer, a token is finite exactly when
its cluster is among the best-scoring (brute force over the scores); ties at
the cut go to the lower index.
"""

from __future__ import annotations

import numpy as np

from . import kernels as ok
from .decoder import bf


def select_clusters(scores, n_probes: int) -> np.ndarray:
    """Indices of the ``n_probes`` largest scores (ties: lower index), ascending."""
    s = np.asarray(scores, np.float64)
    order = np.lexsort((np.arange(s.shape[0]), -s))
    return np.sort(order[:n_probes])


def flash_head_logits(hv, centroids, head, token_map, n_probes: int, vocab: int, *, force=None,
                      centroid_group: int = 64, head_group: int = 64):
    """``(logits [vocab] float64 with -inf, selected cluster ids, scores)`` for
    one hidden row ``hv [H]``; ``centroids`` / ``head`` are ``(packed,
    scales, biases)`` with head arrays shaped ``[C, S, ...]``; ``force`` is
    ``(packed, scales, biases, ids)`` or None."""
    x = np.asarray(hv, np.float64).reshape(1, -1)
    cw, cs, cb = centroids
    scores = bf(ok.rtn4_gemv(x, cw, cs, cb, group_size=centroid_group))[0]
    sel = select_clusters(scores, n_probes)
    hw, hs, hb = head
    tm = np.asarray(token_map)
    n_c, c_s = tm.shape
    rows = (sel[:, None] * c_s + np.arange(c_s)[None, :]).reshape(-1)
    flat = lambda a: np.asarray(a).reshape(n_c * c_s, -1)[rows]  # noqa: E731
    probe = bf(ok.rtn4_gemv(x, flat(hw), flat(hs), flat(hb), group_size=head_group))[0]
    out = np.full(vocab, -np.inf)
    out[tm.reshape(-1)[rows]] = probe
    if force is not None and len(force[3]):
        fw, fs, fb, fid = force
        out[np.asarray(fid)] = bf(ok.rtn4_gemv(x, fw, fs, fb, group_size=head_group))[0]
    return out, sel, scores
