"""Shared helpers of the tests: synthetic routings and tolerance metrics."""

from __future__ import annotations

import torch

BF16 = torch.bfloat16


def routing(n, e, k, mode, g):
    """(top_i int64, top_w bf16) as the reference tests build them
    (tests/test_moe_prefill.py:30-37): uniform, skewed (3 popular experts), sparse
    (only k experts), one (every pair on expert e//2)."""
    logits = torch.randn(n, e, generator=g)
    if mode == "skewed":
        logits[:, :3] += 6.0
    elif mode == "sparse":
        logits[:, k:] = -1e9
    w, idx = torch.topk(torch.softmax(logits, -1), k, dim=-1)
    w = (w / w.sum(-1, keepdim=True)).to(BF16)
    if mode == "one":
        idx = torch.full((n, k), e // 2, dtype=torch.long)
    return idx, w


def router_rows(n, E, seed):
    """Router logits with the cases that matter for ties (the row families of the
    reference's tests/test_fused_glue.py:73-84: peaked, coarse ties, all tied, flat, large)."""
    g = torch.Generator().manual_seed(seed)
    r = torch.randn(n, E, generator=g)
    k = n // 4
    r[:k] *= 4.0
    r[k : 2 * k] = torch.round(r[k : 2 * k] * 2) / 2
    r[2 * k : 2 * k + 8] = 0.5
    r[2 * k + 8 : 3 * k] *= 0.05
    r[3 * k :] = r[3 * k :] * 8 + 30
    return r.to(BF16)


def max_abs(a, b):
    return (a.float().cpu() - b.float().cpu()).abs().max().item()


def mean_rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return ((a - b).abs().mean() / b.abs().mean().clamp_min(1e-30)).item()


class knobs:
    """Run the body with the library's comparison switches (MOE_DECODE, MOE_MIXED, ...) set
    as given (None: unset). The library reads them once per process and again on
    moe_reload_tuning(), which this calls on entry and exit."""

    def __init__(self, **env):
        self.env = env

    def _reload(self):
        import __graft_entry__

        __graft_entry__.load_package()._lib.load().moe_reload_tuning()

    def __enter__(self):
        import os

        self.old = {k: os.environ.get(k) for k in self.env}
        for k, v in self.env.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
        self._reload()
        return self

    def __exit__(self, *exc):
        import os

        for k, v in self.old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
        self._reload()
