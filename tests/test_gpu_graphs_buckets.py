"""graphs.MoeGraphs: a step of B rows replays the smallest bucket >= B and gives the bits of
the eager call on those rows (padding rows repeat the last row; a row's output does not
depend on the others of its call), for the plain block with a residual and with the
post-attention add + RMSNorm in front; replays with new inputs are not stale; a later,
larger bucket leaves the earlier graphs working."""

from __future__ import annotations

import pytest
import torch

from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
H = 2048


@pytest.fixture(scope="module")
def mlp(dev):
    import __graft_entry__

    return __graft_entry__._mlp_from_weights(orc.make_weights(H, 256, 512, 512, seed=41), dev)


@pytest.mark.parametrize("with_norm", [False, True])
def test_bucket_replays_match_eager(pkg, dev, mlp, with_norm):
    g = torch.Generator().manual_seed(5 + with_norm)
    nw = (torch.randn(H, generator=g) * 0.1).to(BF16).to(dev)
    graphs = pkg.graphs.MoeGraphs(mlp, 8, H, dev, buckets=(1, 4, 8, 16),
                                  norm=(nw, 1e-6) if with_norm else None)
    for rows in (1, 3, 4, 7, 12, 2, 3):
        print(f"bucket replay rows={rows} norm={with_norm}", flush=True)
        x = torch.randn(rows, H, generator=g).to(BF16).to(dev)
        y = torch.randn(rows, H, generator=g).to(BF16).to(dev)
        got = graphs.run(x, y).clone()
        if with_norm:
            want = pkg.block.add_rms_moe(x, y, nw, 1e-6, mlp, 8, decode=True)
        else:
            want = pkg.block.moe(x, mlp, 8, decode=True, residual=y)
        torch.cuda.synchronize()
        assert graphs.bucket(rows) in graphs.graphs
        assert torch.equal(got, want), rows
    with pytest.raises(ValueError):
        graphs.bucket(17)
