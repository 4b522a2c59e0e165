"""Post-attention add + RMSNorm: the stand-alone kernel and the fused block entry point.

- ``ops.add_rms`` (k_add_rms): total = bf16(x + h) bit-exact against the oracle; the norm
  within one bf16 ulp of the oracle (the bar of the reference's own test of this norm,
  tests/test_chain_glue.py:40-43: the fp32 sum of squares is reduced in another order and
  rsqrt is the hardware's), and equal bit for bit on nearly every element.
- ``block.add_rms_moe`` (moe_block_forward_add_rms): total, norm, routing and output equal
  bit for bit what ``ops.add_rms`` followed by ``block.moe(norm, residual=total)`` gives, on
  the decode path (norm inside the router launch, which shares the row routine of
  k_add_rms) and on the tiled and prefill paths (one add_rms launch in front); and the
  output is within the block's bar of the fp32 oracle fed by the oracle's add_rms.
"""

from __future__ import annotations

import pytest
import torch

from oracle import moe_oracle as orc
from tests.helpers import BF16, max_abs, mean_rel

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _say(*a):
    print(*a, flush=True)


def _ulp_close(a, b):
    """Every element at most one bf16 ulp apart (relative 2^-7), as test_chain_glue.py."""
    a, b = a.float().cpu(), b.float().cpu()
    return bool(torch.all((a - b).abs() <= b.abs() * 2.0 ** -7 + 1e-6))


def _inputs(T, H, seed, with_h=True, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(T, H, generator=g) * scale).to(BF16)
    h = (torch.randn(T, H, generator=g) * scale).to(BF16) if with_h else None
    w = (torch.randn(H, generator=g) * 0.2).to(BF16)
    return x, h, w


@pytest.mark.parametrize("T,H", [(1, 2048), (3, 2048), (4, 4096), (64, 2048), (1000, 2048),
                                 (5, 8), (7, 1000), (2, 8192), (33, 512)])
@pytest.mark.parametrize("with_h", [True, False])
def test_add_rms_matches_oracle(pkg, dev, T, H, with_h):
    _say("add_rms", T, H, with_h)
    x, h, w = _inputs(T, H, seed=T * 31 + H, with_h=with_h)
    total, out = pkg.ops.add_rms(x.to(dev), None if h is None else h.to(dev), w.to(dev), EPS)
    again = pkg.ops.add_rms(x.to(dev), None if h is None else h.to(dev), w.to(dev), EPS)[1]
    torch.cuda.synchronize()
    r_total, r_out = orc.add_rms(x, h, w, EPS)
    assert torch.equal(total.cpu(), r_total)
    assert torch.equal(out, again)
    assert _ulp_close(out, r_out)
    same = (out.cpu() == r_out).float().mean().item()
    _say(f"  bit-equal fraction {same:.4f}")
    assert same >= 0.95


def test_add_rms_large_and_tiny_rows(pkg, dev):
    """Rows of very different magnitude normalise to the same scale; eps dominates a row of
    zeros (out = 0) without NaN."""
    x, h, w = _inputs(4, 2048, seed=3, with_h=True)
    x[1] *= 1e4
    h[1] *= 1e4
    x[2] *= 1e-4
    h[2] *= 1e-4
    x[3] = 0
    h[3] = 0
    total, out = pkg.ops.add_rms(x.to(dev), h.to(dev), w.to(dev), EPS)
    torch.cuda.synchronize()
    r_total, r_out = orc.add_rms(x, h, w, EPS)
    assert torch.equal(total.cpu(), r_total)
    assert _ulp_close(out, r_out)
    assert torch.all(out[3] == 0)


def test_add_rms_sum_special_values(pkg, dev):
    """The bf16 rounding of the sum (the hardware's packed convert) against torch's add on
    ties to even, overflow to +-inf, bf16 subnormal sums and signed zeros, plus random
    rows; the norm is checked on the rows whose sum of squares is finite."""
    H = 64
    x = torch.randn(3, H, generator=torch.Generator().manual_seed(1)).to(BF16)
    h = torch.randn(3, H, generator=torch.Generator().manual_seed(2)).to(BF16)
    special = [(256.0, 1.0), (256.0, 3.0), (1.0, 2.0 ** -8), (1.0, 3 * 2.0 ** -9),
               (3.3e38, 3.3e38), (-3.3e38, -3.3e38), (5e-39, 4e-39), (-6e-39, 1e-40),
               (2.0 ** -133, 2.0 ** -133), (-0.0, 0.0), (-0.0, -0.0), (1.5, -1.5)]
    for i, (a, b) in enumerate(special):
        x[0, i] = a
        h[0, i] = b
    w = torch.zeros(H, dtype=BF16)
    total, out = pkg.ops.add_rms(x.to(dev), h.to(dev), w.to(dev), EPS)
    torch.cuda.synchronize()
    r_total, r_out = orc.add_rms(x, h, w, EPS)
    got = total.cpu()
    assert torch.equal(got.view(torch.int16), r_total.view(torch.int16))
    assert _ulp_close(out[1:], r_out[1:])


def test_add_rms_rejects_bad_arguments(pkg, dev):
    lib = pkg._lib.load()
    x = torch.randn(2, 64, device=dev).to(BF16)
    w = torch.zeros(64, device=dev, dtype=BF16)
    out = torch.empty_like(x)
    s = torch.cuda.current_stream(dev).cuda_stream
    # output aliasing the input
    assert lib.moe_add_rmsnorm(x.data_ptr(), None, w.data_ptr(), 2, 64, EPS, None,
                               x.data_ptr(), s) == pkg._lib.MOE_EINVAL
    # H not a multiple of 8
    assert lib.moe_add_rmsnorm(x.data_ptr(), None, w.data_ptr(), 2, 60, EPS, None,
                               out.data_ptr(), s) == pkg._lib.MOE_EINVAL
    # h without a total buffer
    assert lib.moe_add_rmsnorm(x.data_ptr(), x.data_ptr(), w.data_ptr(), 2, 64, EPS, None,
                               out.data_ptr(), s) == pkg._lib.MOE_EINVAL
    # T = 0 is a no-op
    assert lib.moe_add_rmsnorm(x.data_ptr(), None, w.data_ptr(), 0, 64, EPS, None,
                               out.data_ptr(), s) == 0
    with pytest.raises(ValueError):
        pkg.ops.add_rms(x, None, torch.zeros(32, device=dev, dtype=BF16), EPS)


@pytest.fixture(scope="module")
def layer(dev):
    import __graft_entry__

    w = orc.make_weights(2048, 256, 512, 512, seed=11)
    return __graft_entry__._mlp_from_weights(w, dev), w


@pytest.mark.parametrize("T", [1, 2, 3, 4, 20, 300, 1024])
@pytest.mark.parametrize("with_h", [True, False])
def test_fused_block_equals_add_rms_then_block(pkg, dev, layer, T, with_h):
    mlp, _ = layer
    _say("add_rms_moe", T, with_h)
    x, h, w = _inputs(T, 2048, seed=T + 500, with_h=with_h, scale=2.0)
    xd, hd, wd = x.to(dev), None if h is None else h.to(dev), w.to(dev)
    out, total, norm, idx, wts, lg = pkg.block.add_rms_moe(
        xd, hd, wd, EPS, mlp, 8, decode=T <= 4, return_norm=True, return_routing=True)
    s_total, s_norm = pkg.ops.add_rms(xd, hd, wd, EPS)
    b_out, b_idx, b_wts, b_lg = pkg.block.moe(s_norm, mlp, 8, decode=T <= 4, residual=s_total,
                                              return_routing=True)
    torch.cuda.synchronize()
    assert torch.equal(total, s_total)
    assert torch.equal(norm, s_norm)
    assert torch.equal(lg, b_lg)
    assert torch.equal(idx, b_idx) and torch.equal(wts, b_wts)
    assert torch.equal(out, b_out)


@pytest.mark.parametrize("T", [1, 4, 64])
def test_fused_block_against_oracle(pkg, dev, layer, T):
    """total bit-exact and norm within an ulp of the oracle's add_rms; the routing bit-exact
    against the oracle's route of the kernel's logits; the output within the block's bar of
    the fp32 oracle run on the kernel's normalised rows (an ulp of difference in the norm
    could flip a near-tie in the routing, so the experts are fed the same rows)."""
    mlp, wts_cpu = layer
    x, h, w = _inputs(T, 2048, seed=T + 900, with_h=True, scale=2.0)
    out, total, norm, idx, wts, lg = pkg.block.add_rms_moe(
        x.to(dev), h.to(dev), w.to(dev), EPS, mlp, 8, decode=T <= 4, return_norm=True,
        return_routing=True)
    torch.cuda.synchronize()
    r_total, r_norm = orc.add_rms(x, h, w, EPS)
    assert torch.equal(total.cpu(), r_total)
    assert _ulp_close(norm, r_norm)
    # the fp32 experts on our normalised rows and routing, plus the residual
    lgc = lg.cpu()
    _, ref_i = orc.route(lgc[:, :256], 8)
    assert torch.equal(idx.cpu(), ref_i)
    f32 = orc.block_fp32(norm.cpu(), wts_cpu, ref_i, logits=lgc[:, :256]) + r_total.float()
    wc, ic = orc.compact_experts(wts_cpu, ref_i)
    ref_path = orc.block_bf16_routed(norm.cpu(), wc, ic, wts.cpu(), lgc[:, 256:257],
                                     decode=T <= 4)
    ref_path = (ref_path.float() + r_total.float()).to(BF16)
    ours, theirs = mean_rel(out, f32), mean_rel(ref_path, f32)
    _say(f"add_rms_moe T={T}: max {max_abs(out, f32):.3g} mean-rel {ours:.3g} "
         f"(reference path {theirs:.3g})")
    assert max_abs(out, f32) <= 2e-2 * max(1.0, f32.abs().max().item())
    assert ours <= max(5e-3, 1.1 * theirs)


def test_fused_block_fp8_decode(pkg, dev, layer):
    """fp8 routed experts: the fused entry point and add_rms + block agree bit for bit."""
    import copy

    mlp, wts_cpu = layer
    m8 = copy.copy(mlp)
    m8.experts = copy.copy(mlp.experts)
    q, s = pkg.fp8.quantize_rows(mlp.experts.gate_up_proj)
    q2, s2 = pkg.fp8.quantize_rows(mlp.experts.down_proj)
    m8.experts.gate_up_proj, m8.experts.gate_up_scale = q, s
    m8.experts.down_proj, m8.experts.down_scale = q2, s2
    x, h, w = _inputs(2, 2048, seed=77, with_h=True)
    xd, hd, wd = x.to(dev), h.to(dev), w.to(dev)
    out = pkg.block.add_rms_moe(xd, hd, wd, EPS, m8, 8, decode=True)
    s_total, s_norm = pkg.ops.add_rms(xd, hd, wd, EPS)
    ref = pkg.block.moe(s_norm, m8, 8, decode=True, residual=s_total)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_fused_block_graph_replays(pkg, dev, layer):
    """The decode form captured in a HIP graph: every replay equals the eager result."""
    mlp, _ = layer
    x, h, w = _inputs(1, 2048, seed=5, with_h=True)
    xd, hd, wd = x.to(dev), h.to(dev), w.to(dev)
    eager = pkg.block.add_rms_moe(xd, hd, wd, EPS, mlp, 8, decode=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        pkg.block.add_rms_moe(xd, hd, wd, EPS, mlp, 8, decode=True)  # warm-up outside capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = pkg.block.add_rms_moe(xd, hd, wd, EPS, mlp, 8, decode=True)
    for i in range(4):
        got.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, eager), f"replay {i}"
        again = pkg.block.add_rms_moe(xd, hd, wd, EPS, mlp, 8, decode=True)  # eager between
        torch.cuda.synchronize()
        assert torch.equal(again, eager)
