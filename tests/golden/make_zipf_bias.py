"""Write ``zipf_bias_e64.json``: the router bias of the skewed-routing workloads.

The skewed MoE workloads (64 experts, top-8, decode batches of 32 and 128
tokens and the 2048-token prefill chunk) ask for a router bias under which the
load of the experts follows a Zipf(s = 1.1) law over expert ranks.  A token
routes to 8 *distinct* experts, so no expert can take more than 1/8 of the
(token, slot) pairs; Zipf(1.1) over 64 ranks gives rank 1 a share of 0.250
and rank 2 one of 0.117.  The target is therefore the Zipf law capped at 1/8
with the excess spread over the uncapped ranks in proportion (water filling):
ranks 1 and 2 at 0.125, rank 3 at 0.0887, ..., rank 64 at 0.0031.

Expert e has rank ``perm[e] + 1`` for a seeded permutation.  The bias starts
as ``log p_rank`` (the one-parameter family ``gamma * log p``; the best
gamma reaches a total-variation distance of only about 0.09 from the target)
and is fitted per expert by the fixed-point iteration
``b_e += 0.5 * (log target_e - log achieved_e)`` on the router logits of
200,000 synthetic tokens (x ~ N(0, 1), router rows ~ N(0, 0.02) over hidden
2048, so a token's logits are close to iid N(0, 0.02^2 * 2048)).  The
achieved load of the fitted bias is measured again on 200,000 fresh tokens and
written with the fixture.

    python tests/golden/make_zipf_bias.py
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np

E, TOP_K, S, HIDDEN, ROUTER_STD = 64, 8, 1.1, 2048, 0.02
PERM_SEED, FIT_SEED, CHECK_SEED, TOKENS, ITERS = 3, 0, 1, 200_000, 80
OUT = Path(__file__).with_name("zipf_bias_e64.json")


def zipf_target(n_experts: int = E, s: float = S, top_k: int = TOP_K) -> np.ndarray:
    """Zipf(s) shares over ranks 1..n, capped at 1/top_k, the excess spread
    over the uncapped ranks in proportion."""
    p = np.arange(1, n_experts + 1, dtype=np.float64) ** -s
    p /= p.sum()
    capped = np.zeros(n_experts, bool)
    while True:
        t = np.where(capped, 1.0 / top_k, p / p[~capped].sum() * (1.0 - capped.sum() / top_k))
        over = t > 1.0 / top_k + 1e-15
        if not over.any():
            return t
        capped |= over


def loads(logits: np.ndarray, bias: np.ndarray, top_k: int = TOP_K) -> np.ndarray:
    """Share of the (token, slot) pairs routed to each expert."""
    top = np.argpartition(-(logits + bias), top_k, axis=1)[:, :top_k]
    c = np.bincount(top.ravel(), minlength=logits.shape[1]).astype(np.float64)
    return c / c.sum()


def main() -> None:
    sigma = ROUTER_STD * np.sqrt(HIDDEN)
    perm = np.random.default_rng(PERM_SEED).permutation(E)  # expert e has rank perm[e] + 1
    target_rank = zipf_target()
    target = target_rank[perm]
    p = np.arange(1, E + 1, dtype=np.float64) ** -S
    p /= p.sum()
    fit = np.random.default_rng(FIT_SEED).standard_normal((TOKENS, E)) * sigma
    tv = lambda a: 0.5 * float(np.abs(a - target).sum())  # noqa: E731
    gammas = np.round(np.arange(0.25, 2.01, 0.05), 2)
    gamma_tv = {float(g): tv(loads(fit, g * np.log(p[perm]))) for g in gammas}
    bias = np.log(p[perm])
    for _ in range(ITERS):
        a = loads(fit, bias)
        bias = bias + 0.5 * (np.log(target) - np.log(np.maximum(a, 1e-9)))
        bias -= bias.max()
    bias = bias.astype(np.float32)
    check = np.random.default_rng(CHECK_SEED).standard_normal((TOKENS, E)) * sigma
    achieved = loads(check, bias.astype(np.float64))
    best_g = min(gamma_tv, key=gamma_tv.get)
    fixture = {
        "what": "router bias (float32, one per expert) for Zipf(1.1)-skewed top-8 routing over 64 "
                "experts; written by make_zipf_bias.py",
        "n_experts": E, "top_k": TOP_K, "zipf_s": S, "hidden": HIDDEN, "router_std": ROUTER_STD,
        "rank_of_expert": (perm + 1).tolist(),
        "bias": [float(v) for v in bias],
        "target_share": [round(float(v), 7) for v in target],
        "achieved_share_fresh_tokens": [round(float(v), 7) for v in achieved],
        "tv_distance_fresh_tokens": round(tv(achieved), 6),
        "best_single_gamma": best_g, "best_single_gamma_tv": round(gamma_tv[best_g], 4),
        "tokens": TOKENS, "iterations": ITERS,
    }
    OUT.write_text("{\n" + ",\n".join(f" {json.dumps(k)}: {json.dumps(v)}" for k, v in fixture.items())
                   + "\n}\n")
    print(f"wrote {OUT}: TV {tv(achieved):.4f} (best single gamma {best_g}: {gamma_tv[best_g]:.4f})")


if __name__ == "__main__":
    main()
