"""Synthetic workloads of the benchmark configurations (no reference counterpart: the
reference's benchmarks load checkpoints; this build has random-init weights only).

``zipf_router`` skews a random router so expert popularity over a batch follows Zipf(s),
the routing distribution of the batch-64 skewed decode workload.
"""

from __future__ import annotations

import torch

BF16 = torch.bfloat16

ZIPF_S = 1.1
ZIPF_BETA = 0.43  # calibrated: Gaussian logit noise (std 0.02*sqrt(2048)) + this bias gives
                  # ~140 distinct experts over 64 tokens x top-8, as Zipf(1.1) sampling
                  # without replacement does (mean 140, 5-95%: 131-151; numpy, 200 reps)
ZIPF_MU = 8.0


def zipf_router(router: torch.Tensor, s: float = ZIPF_S, beta: float = ZIPF_BETA,
                mu: float = ZIPF_MU, seed: int = 0):
    """Router weight biased so expert popularity follows Zipf(s) (skewed decode routing).

    Tokens are x = N(0, 1) + mu * v for a fixed unit direction v; W_r[e] gains
    (beta * log(zipf_e) / mu) * v, so expert e's logit gains beta * log(zipf_e) on every
    token, on top of the N(0, 0.02^2 * H) spread of the random router. Expert ranks are a
    seeded permutation. Returns (W_r', v); build the tokens as x + mu * v."""
    experts, hidden = router.shape
    g = torch.Generator().manual_seed(seed + 1)
    v = torch.randn(hidden, generator=g)
    v = v / v.norm()
    ranks = torch.randperm(experts, generator=g).float() + 1.0
    logz = -s * torch.log(ranks)
    logz = logz - logz.mean()
    w = router.float() + (beta * logz / mu)[:, None] * v[None, :]
    return w.to(BF16), v
