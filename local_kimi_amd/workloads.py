"""Synthetic inputs of the benchmarked W4A16 MoE workloads (numpy, seeded).

Router logits with Zipf-skewed expert popularity: popularity
``p_i ~ 1 / rank_i ** s`` over a seeded permutation of the routed expert ids,
and ``logits = log p + Gumbel(0, 1)``. The top-k of such logits is a draw of k
distinct experts without replacement in proportion to ``p`` (the Gumbel top-k
construction), so routing still goes through the sigmoid top-k router while
per-expert token counts are uneven: many experts get 0 or 1 token, hot experts
get many.
"""

from __future__ import annotations

import numpy as np


def zipf_router_logits(rng: np.random.Generator, tokens: int, experts: int,
                       s: float = 1.1) -> np.ndarray:
    """float32 ``[tokens, experts]`` logits with Zipf(s) expert popularity."""
    ranks = np.empty(experts, dtype=np.float64)
    ranks[rng.permutation(experts)] = np.arange(1, experts + 1, dtype=np.float64)
    log_p = -s * np.log(ranks)
    log_p -= np.log(np.exp(log_p).sum())
    gumbel = -np.log(-np.log(rng.uniform(1e-12, 1.0, (tokens, experts))))
    return (log_p[None, :] + gumbel).astype(np.float32)


def normal_router_logits(rng: np.random.Generator, tokens: int, experts: int) -> np.ndarray:
    """float32 ``[tokens, experts]`` logits ~ N(0, 1) (uniform expert popularity)."""
    return rng.normal(0.0, 1.0, (tokens, experts)).astype(np.float32)
