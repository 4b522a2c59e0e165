"""The block under HIP graph capture (how the engine runs decode, engine/fast/model.py:1947-2093):
every regime — the three-launch decode path, the tiled decode path, fp8 experts with the bf16
shared expert on the auxiliary stream, the prefill tiles with the LDS-tiled router — is
captured once and replayed several times with eager calls in between; every replay must give
the eager call's bits."""

from __future__ import annotations

import pytest
import torch

from tests.helpers import BF16

pytestmark = pytest.mark.gpu


def _layer(dev, fp8, pkg):
    import __graft_entry__

    g = torch.Generator(device=dev).manual_seed(5)

    def rnd(*shape):
        return (torch.randn(*shape, generator=g, device=dev) * 0.02).to(BF16)

    H, E, I = 2048, 256, 512
    w = {"router": rnd(E, H), "gate_up": rnd(E, 2 * I, H), "down": rnd(E, H, I),
         "sh_gate": rnd(I, H), "sh_up": rnd(I, H), "sh_down": rnd(H, I), "sh_gate_w": rnd(1, H)}
    mlp = __graft_entry__._mlp_from_weights(w, dev)
    if fp8:
        q, s = pkg.fp8.quantize_rows(w["gate_up"])
        q2, s2 = pkg.fp8.quantize_rows(w["down"])
        mlp.experts.gate_up_proj, mlp.experts.gate_up_scale = q, s
        mlp.experts.down_proj, mlp.experts.down_scale = q2, s2
    return mlp


@pytest.mark.parametrize("T,fp8", [(1, False), (8, False), (32, True), (64, False), (1024, False)])
def test_block_graph_replays_match_eager(pkg, dev, T, fp8):
    print("graph", T, fp8, flush=True)
    mlp = _layer(dev, fp8, pkg)
    x = torch.randn(T, 2048, generator=torch.Generator().manual_seed(T)).to(BF16).to(dev)
    r = torch.randn(T, 2048, generator=torch.Generator().manual_seed(T + 1)).to(BF16).to(dev)
    eager = pkg.block.moe(x, mlp, 8, decode=T <= 64, residual=r)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        pkg.block.moe(x, mlp, 8, decode=T <= 64, residual=r)  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = pkg.block.moe(x, mlp, 8, decode=T <= 64, residual=r)
    for i in range(3):
        out.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        again = pkg.block.moe(x, mlp, 8, decode=T <= 64, residual=r)  # eager work between
        torch.cuda.synchronize()
        assert torch.equal(again, eager)
