"""The Zipf(1.1) router-bias fixture (tests/golden/zipf_bias_e64.json), CPU.

The target load is Zipf(1.1) over 64 expert ranks capped at 1/8 (a token's
8 experts are distinct, so no expert can take more than 1/8 of the pairs),
the excess spread in proportion over the other ranks.  The fitted bias, put
through the oracle's router on a synthetic layer (router rows ~ N(0, 0.02),
2048 tokens ~ N(0, 1)), gives an expert load within the sampling distance of
that target.
"""

from __future__ import annotations

import numpy as np

from _helpers import ZIPF, load_tv_distance
from oracle import kernels as ok


def test_target_is_capped_zipf():
    t = np.asarray(ZIPF["target_share"])
    rank = np.asarray(ZIPF["rank_of_expert"])
    assert sorted(rank.tolist()) == list(range(1, 65))
    by_rank = t[np.argsort(rank)]
    np.testing.assert_allclose(by_rank.sum(), 1.0, atol=1e-6)
    assert by_rank.max() <= 1 / 8 + 1e-7
    np.testing.assert_allclose(by_rank[:2], 1 / 8, atol=1e-7)  # Zipf gives rank 1 0.250, rank 2 0.117
    r = np.arange(3, 65, dtype=np.float64)
    ratio = by_rank[2:] / r ** -1.1  # uncapped ranks keep the Zipf(1.1) proportions
    np.testing.assert_allclose(ratio, ratio[0], rtol=2e-5)
    p = np.arange(1, 65, dtype=np.float64) ** -1.1
    assert abs(p[0] / p.sum() - 0.2505) < 1e-3


def test_fitted_bias_gives_target_load_through_the_oracle_router():
    rng = np.random.default_rng(21)
    gate = ok.bf16_round(rng.standard_normal((64, 2048)) * 0.02)
    x = ok.bf16_round(rng.standard_normal((2048, 2048)))
    ids, _, _ = ok.router_topk(x, gate, 8, bias=np.asarray(ZIPF["bias"], np.float32))
    assert load_tv_distance(ids) <= 0.04
    ids_u, _, _ = ok.router_topk(x, gate, 8)
    assert load_tv_distance(ids_u) > 0.3  # without the bias the load is far from the target
    share = np.bincount(ids.reshape(-1), minlength=64) / ids.size
    assert share.max() <= 1 / 8
