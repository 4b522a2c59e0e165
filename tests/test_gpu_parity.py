"""Parity of the gfx950 kernels (through the C ABI) against the CPU oracle.

Bar: expert indices, counts, offsets, permutation and tile table bit-exact; bf16 values
within the reference tests' tolerance (max-abs <= 2e-2 * max(1, |ref|max), the bound of
engine tests/test_moe_prefill.py:56,80) of the bf16-rounding oracle, and within
max-abs 2e-2 / mean-rel 5e-3 of the fp32 oracle (the north star's bf16 bar).
"""

from __future__ import annotations

import pytest
import torch

from oracle import moe_oracle as orc
from tests.helpers import BF16, knobs, max_abs, mean_rel, router_rows, routing

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _synth():
    import __graft_entry__

    return __graft_entry__.load_package().synth


def _say(*a):
    print(*a, flush=True)


# ----------------------------------------------------------------------------- routing


@pytest.mark.parametrize("E,k", [(256, 8), (16, 4), (8, 2), (64, 8), (128, 1), (512, 8)])
@pytest.mark.parametrize("seed", [0, 1])
def test_route_bitexact(pkg, dev, E, k, seed):
    _say("route", E, k, seed)
    g = torch.Generator().manual_seed(100 + seed)
    logits = torch.cat([router_rows(64, E, seed), torch.randn(64, E, generator=g).to(BF16)])
    w, i, counts = pkg.ops.route(logits.to(dev), k)
    torch.cuda.synchronize()
    ref_w, ref_i = orc.route(logits, k)
    assert torch.equal(i.cpu(), ref_i)
    # weights: the renormalising sum's order may differ by one fp32 ulp -> one bf16 ulp at most
    diff = (w.float().cpu() - ref_w.float()).abs()
    assert (diff <= ref_w.float().abs() * 2.0 ** -7 + 1e-30).all()
    assert torch.equal(counts.cpu(), torch.bincount(ref_i.reshape(-1), minlength=E).int())


def _hard_rows(E, g):
    """Rows where the largest logits are not the largest p in their order: exp underflow
    (p = 0 for distinct logits), subnormal boundary p, tiny logits at the selection
    boundary, exact logit ties, and ordinary rows between them."""
    rows = []
    r = torch.zeros(E)
    r[:3] = 100.0
    r[3:] = -200.0 - torch.arange(E - 3) * 0.5  # p underflows to 0 for distinct logits
    rows.append(r)
    r = torch.full((E,), -60.0)
    r[:2] = 40.0
    r[5::7] = -60.5  # subnormal p at the boundary
    rows.append(r)
    r = torch.randn(E, generator=g) * 1e-4  # every logit under 2^-10
    r[:4] = 2.0
    rows.append(r)
    r = torch.randn(E, generator=g)
    r[E // 2:] = r[: E - E // 2].clone()  # pairs of equal logits
    rows.append(r)
    r = torch.zeros(E)  # all tied
    rows.append(r)
    r = torch.randn(E, generator=g) * 30  # wide spread, no special structure
    rows.append(r)
    return torch.stack(rows).to(BF16)


@pytest.mark.parametrize("E,k", [(256, 8), (64, 8), (16, 4)])
def test_route_hard_rows(pkg, dev, E, k):
    """The exact-selection fallback of the routing kernel on rows built to need it."""
    g = torch.Generator().manual_seed(E + k)
    logits = torch.cat([_hard_rows(E, g), router_rows(16, E, 3)])
    w, i, _ = pkg.ops.route(logits.to(dev), k)
    torch.cuda.synchronize()
    ref_w, ref_i = orc.route(logits, k)
    assert torch.equal(i.cpu(), ref_i)
    diff = (w.float().cpu() - ref_w.float()).abs()
    assert (diff <= ref_w.float().abs() * 2.0 ** -7 + 1e-30).all()


def test_route_bruteforce_small(pkg, dev):
    logits = router_rows(16, 8, 7)
    _, i, _ = pkg.ops.route(logits.to(dev), 3)
    torch.cuda.synchronize()
    assert torch.equal(i.cpu(), orc.route_bruteforce(logits, 3))


# -------------------------------------------------------------------------------- sort


SORT_CASES = [(1, 256, 8), (4, 16, 4), (64, 256, 8), (75, 16, 4), (300, 16, 4), (513, 256, 8),
              (1000, 256, 8), (2049, 64, 2), (700, 512, 8), (4096, 256, 8),
              (5000, 256, 8)]  # 40000 pairs: more than 32 count blocks (the scan's other branch)


@pytest.mark.parametrize("T,E,k", SORT_CASES)
@pytest.mark.parametrize("mode", ["uniform", "skewed", "sparse", "one"])
@pytest.mark.parametrize("shared", [False, True])
def test_sort_bitexact(pkg, dev, T, E, k, mode, shared):
    _say("sort", T, E, k, mode, shared)
    g = torch.Generator().manual_seed(T * 7 + E)
    idx, _ = routing(T, E, k, mode, g)
    bm = 64
    sp = pkg.ops.sort_pairs(idx.to(dev), E, bm=bm, shared=shared)
    torch.cuda.synchronize()
    counts, offsets, order, tiles = orc.sort_pairs(idx, E, bm, tokens=T, shared=shared)
    assert torch.equal(sp.counts.cpu(), torch.from_numpy(counts))
    assert torch.equal(sp.offsets.cpu(), torch.from_numpy(offsets))
    assert torch.equal(sp.order.cpu(), torch.from_numpy(order))
    assert torch.equal(sp.order.cpu().long(), torch.argsort(idx.reshape(-1), stable=True))
    mt = sp.max_tiles
    assert mt == orc.max_tiles(T, k, E, bm, shared)
    tab = sp.table.cpu()
    n = int(tab[3 * mt])
    assert n == len(tiles)
    got = [(int(tab[t]), int(tab[mt + t]), int(tab[2 * mt + t])) for t in range(n)]
    assert got == tiles


def test_sort_deterministic(pkg, dev):
    g = torch.Generator().manual_seed(5)
    idx, _ = routing(3000, 256, 8, "skewed", g)
    a = pkg.ops.sort_pairs(idx.to(dev), 256)
    b = pkg.ops.sort_pairs(idx.to(dev), 256)
    torch.cuda.synchronize()
    mt = a.max_tiles
    n = int(a.table[3 * mt])
    ta, tb = a.table.cpu(), b.table.cpu()
    used = torch.cat([torch.arange(n) + o for o in (0, mt, 2 * mt)] + [torch.tensor([3 * mt])])
    assert torch.equal(a.order, b.order) and torch.equal(ta[used], tb[used])


# ------------------------------------------------------------------------- experts


class _Experts(torch.nn.Module):
    """engine tests/test_moe_prefill.py:14-27's experts holder (weights * 0.1)."""

    def __init__(self, e, h, i, seed=0):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.num_experts = e
        self.gate_up_proj = torch.randn(e, 2 * i, h, generator=g).mul(0.1).to(BF16)
        self.down_proj = torch.randn(e, h, i, generator=g).mul(0.1).to(BF16)
        self.act_fn = torch.nn.functional.silu


@pytest.mark.parametrize("n", [1, 4, 16, 17, 40, 300])
@pytest.mark.parametrize("mode", ["uniform", "skewed", "sparse", "one"])
@pytest.mark.parametrize("shape", [(16, 128, 64, 4), (8, 64, 32, 2), (32, 256, 128, 8)])
def test_experts_forward_matches_oracle(pkg, dev, n, mode, shape):
    e, h, i, k = shape
    _say("experts", n, mode, shape)
    m = _Experts(e, h, i, seed=n)
    g = torch.Generator().manual_seed(n + 1)
    x = torch.randn(n, h, generator=g).to(BF16)
    idx, w = routing(n, e, k, mode, g)
    gpu = _Experts(e, h, i, seed=n)
    gpu.gate_up_proj, gpu.down_proj = m.gate_up_proj.to(dev), m.down_proj.to(dev)
    got = pkg.experts.experts_forward(gpu, x.to(dev), idx.to(dev), w.to(dev))
    again = pkg.experts.experts_forward(gpu, x.to(dev), idx.to(dev), w.to(dev))
    torch.cuda.synchronize()
    ref = orc.experts_forward(x, idx, w, m.gate_up_proj, m.down_proj)
    scale = max(1.0, ref.float().abs().max().item())
    assert got.dtype == BF16 and got.shape == ref.shape
    assert max_abs(got, ref) <= TOL * scale
    assert torch.equal(got, again), "not deterministic"


@pytest.mark.parametrize("n", [600, 1500])
@pytest.mark.parametrize("mode", ["uniform", "skewed", "one"])
@pytest.mark.parametrize("shape", [(32, 256, 128, 8), (16, 2048, 1024, 4)])
def test_experts_prefill_tiles_match_oracle(pkg, dev, n, mode, shape):
    """More than 512 tokens: the 256-row prefill GEMM tiles (H % 256 == 0, I % 128 == 0), at
    a small shape and at the model's hidden size with a doubled intermediate (32 / 16 DMA
    chunks per gate_up / down workgroup)."""
    e, h, i, k = shape
    _say("experts prefill", n, mode, shape)
    assert pkg._lib.load().moe_tile_rows(n) == 256
    m = _Experts(e, h, i, seed=n)
    g = torch.Generator().manual_seed(n + 2)
    x = torch.randn(n, h, generator=g).to(BF16)
    idx, w = routing(n, e, k, mode, g)
    gpu = _Experts(e, h, i, seed=n)
    gpu.gate_up_proj, gpu.down_proj = m.gate_up_proj.to(dev), m.down_proj.to(dev)
    got = pkg.experts.experts_forward(gpu, x.to(dev), idx.to(dev), w.to(dev))
    again = pkg.experts.experts_forward(gpu, x.to(dev), idx.to(dev), w.to(dev))
    torch.cuda.synchronize()
    ref = orc.sorted_experts(x, idx, w, m.gate_up_proj, m.down_proj)
    scale = max(1.0, ref.float().abs().max().item())
    assert max_abs(got, ref) <= TOL * scale
    assert torch.equal(got, again), "not deterministic"


@pytest.mark.parametrize("n", [3, 40])
def test_grouped_stages_match_oracle(pkg, dev, n):
    """gate_up -> act (sorted rows) and down -> y (pair rows) separately."""
    e, h, i, k = 16, 128, 64, 4
    m = _Experts(e, h, i, seed=3)
    g = torch.Generator().manual_seed(n)
    x = torch.randn(n, h, generator=g).to(BF16)
    idx, w = routing(n, e, k, "uniform", g)
    gu, dn = m.gate_up_proj.to(dev), m.down_proj.to(dev)
    sp = pkg.ops.sort_pairs(idx.to(dev), e)
    act = pkg.ops.grouped_gate_up(x.to(dev), k, gu, sp)
    y = pkg.ops.grouped_down(act, n, k, dn, sp)
    out_r = pkg.ops.combine(y, w.to(dev), round_products=True)
    out_e = pkg.ops.combine(y, w.to(dev), round_products=False)
    torch.cuda.synchronize()
    ref_act, ref_y = orc.pair_outputs_bf16(x, idx, m.gate_up_proj, m.down_proj)
    order = sp.order.cpu().long()
    assert max_abs(act.cpu(), ref_act[order]) <= TOL * max(1.0, ref_act.float().abs().max().item())
    assert max_abs(y.cpu(), ref_y) <= TOL * max(1.0, ref_y.float().abs().max().item())
    ref_r = orc.batched_mm_experts(x, idx, w, m.gate_up_proj, m.down_proj)
    ref_e = orc.sorted_experts(x, idx, w, m.gate_up_proj, m.down_proj)
    assert max_abs(out_r, ref_r) <= TOL and max_abs(out_e, ref_e) <= TOL
    # combine itself on identical pair outputs: exact fp32 product path is exact in fp32
    y_ref_bits = ref_y.to(dev)
    out_c = pkg.ops.combine(y_ref_bits, w.to(dev), round_products=False).cpu()
    want = (ref_y.float() * w.reshape(-1, 1).float()).view(n, k, -1).sum(1).to(BF16)
    assert max_abs(out_c, want) <= 2.0 ** -8 * max(1.0, want.float().abs().max().item())


# -------------------------------------------------------------------------------- block


def _gpu_mlp(w, dev):
    import __graft_entry__

    return __graft_entry__._mlp_from_weights(w, dev)


@pytest.mark.parametrize("T", [1, 4, 17, 64])
def test_block_c1_shape(pkg, dev, T):
    """C1 layer (H256, E16, k4, I=IS=128) against both oracles."""
    _say("block c1", T)
    H, E, K, I = 256, 16, 4, 128
    w = orc.make_weights(H, E, I, I, seed=0)
    g = torch.Generator().manual_seed(T)
    x = torch.randn(T, H, generator=g).to(BF16)
    out, idx, wts, logits = pkg.block.moe(x.to(dev), _gpu_mlp(w, dev), K, return_routing=True)
    torch.cuda.synchronize()
    lg = logits.cpu()[:, :E]
    ref_w, ref_i = orc.route(lg, K)
    assert torch.equal(idx.cpu(), ref_i)
    ref_lg = torch.nn.functional.linear(x, w["router"])
    assert max_abs(lg, ref_lg) <= 2.0 ** -7 * max(1.0, ref_lg.float().abs().max().item())
    ref, _, _, _ = orc.block_bf16(x, w, K)
    f32 = orc.block_fp32(x, w, ref_i, logits=lg)
    _say(" vs bf16 oracle", max_abs(out, ref), " vs fp32", max_abs(out, f32), mean_rel(out, f32))
    assert max_abs(out, f32) <= 2e-2 and mean_rel(out, f32) <= 5e-3


def _full_weights(dev, seed=0, zipf=False):
    H, E, I = 2048, 256, 512
    g = torch.Generator(device=dev).manual_seed(seed)

    def rnd(*shape):
        return (torch.randn(*shape, generator=g, device=dev) * 0.02).to(BF16)

    w = {
        "router": rnd(E, H), "gate_up": rnd(E, 2 * I, H), "down": rnd(E, H, I),
        "sh_gate": rnd(I, H), "sh_up": rnd(I, H), "sh_down": rnd(H, I), "sh_gate_w": rnd(1, H),
    }
    v = None
    if zipf:
        r, v = _synth().zipf_router(w["router"].cpu(), seed=seed)
        w["router"] = r.to(dev)
    return w, v


@pytest.fixture(scope="module")
def full_layer(dev):
    return _full_weights(dev, seed=0)


@pytest.mark.parametrize("T", [1, 8, 64])
def test_block_full_shape(pkg, dev, full_layer, T):
    """C2/C3-shaped layer (H2048, E256, k8, I=IS=512): routing bit-exact given the logits,
    values vs the fp32 oracle."""
    _say("block full", T)
    w, _ = full_layer
    g = torch.Generator().manual_seed(T)
    x = torch.randn(T, 2048, generator=g).to(BF16)
    out, idx, wts, logits = pkg.block.moe(x.to(dev), _gpu_mlp(w, dev), 8, return_routing=True)
    torch.cuda.synchronize()
    lg = logits.cpu()[:, :256]
    ref_w, ref_i = orc.route(lg, 8)
    assert torch.equal(idx.cpu(), ref_i)
    ref_lg = torch.nn.functional.linear(x, w["router"].cpu())
    assert max_abs(lg, ref_lg) <= 2.0 ** -7 * max(1.0, ref_lg.float().abs().max().item())
    f32 = orc.block_fp32(x, w, ref_i, logits=lg)
    wc, ic = orc.compact_experts(w, ref_i)
    # the reference torch path (bf16 rounding points) on the same routing
    seg = logits.cpu()[:, 256:257]
    ref = orc.block_bf16_routed(x, wc, ic, wts.cpu(), seg)
    ours, theirs = mean_rel(out, f32), mean_rel(ref, f32)
    _say(f" vs fp32: ours max {max_abs(out, f32):.3g} mean-rel {ours:.3g}; "
         f"reference path mean-rel {theirs:.3g}; ours vs reference path {max_abs(out, ref):.3g}")
    assert max_abs(out, f32) <= 2e-2
    assert max_abs(out, ref) <= 2e-2
    assert ours <= max(5e-3, 1.1 * theirs)


@pytest.mark.parametrize("T", [1024, 4096])
def test_block_full_shape_prefill(pkg, dev, full_layer, T):
    """Prefill-sized chunks of the full layer (the C4 path): routing bit-exact for every
    token given the logits; values against the fp32 oracle on 64 sampled tokens (each
    token's output depends on that token alone)."""
    _say("block full prefill", T)
    w, _ = full_layer
    g = torch.Generator().manual_seed(T)
    x = torch.randn(T, 2048, generator=g).to(BF16)
    out, idx, wts, logits = pkg.block.moe(x.to(dev), _gpu_mlp(w, dev), 8, return_routing=True)
    torch.cuda.synchronize()
    lg = logits.cpu()[:, :256]
    _, ref_i = orc.route(lg, 8)
    assert torch.equal(idx.cpu(), ref_i)
    pick = torch.randperm(T, generator=g)[:64]
    f32 = orc.block_fp32(x[pick], w, ref_i[pick], logits=lg[pick])
    o = out.cpu()[pick]
    # the reference torch path (padded / sorted rounding) on the same tokens and routing
    wc, ic = orc.compact_experts(w, ref_i[pick])
    ref = orc.block_bf16_routed(x[pick], wc, ic, wts.cpu()[pick], logits.cpu()[pick, 256:257])
    ours, theirs = mean_rel(o, f32), mean_rel(ref, f32)
    _say(f" vs fp32 on 64 tokens: max {max_abs(o, f32):.3g} mean-rel {ours:.3g}; reference "
         f"path mean-rel {theirs:.3g}; ours vs reference path {max_abs(o, ref):.3g}")
    assert max_abs(o, f32) <= 2e-2 and max_abs(o, ref) <= 2e-2
    assert ours <= max(5e-3, 1.1 * theirs)
    assert torch.isfinite(out.float()).all()


@pytest.mark.parametrize("T", [1, 64, 1024])
def test_shared_up_below_gate(pkg, dev, full_layer, T):
    """The shared expert's gate and up projections are separate tensors at any distance and
    in either order in memory: here up sits just below gate (a negative gate -> up offset)
    in every regime (decode, expert GEMM, prefill tiles). Same outputs as with the tensors
    in the usual order."""
    _say("shared up below gate", T)
    w, _ = full_layer
    g = torch.Generator().manual_seed(50 + T)
    x = torch.randn(T, 2048, generator=g).to(BF16).to(dev)
    mlp = _gpu_mlp(w, dev)
    both = torch.empty((2,) + tuple(w["sh_gate"].shape), dtype=BF16, device=dev)
    both[0].copy_(w["sh_up"])
    both[1].copy_(w["sh_gate"])
    mlp2 = _gpu_mlp(w, dev)
    mlp2.shared_expert.gate_proj.weight = both[1]
    mlp2.shared_expert.up_proj.weight = both[0]
    a = pkg.block.moe(x, mlp, 8)
    b = pkg.block.moe(x, mlp2, 8)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_block_residual(pkg, dev):
    H, E, K, I = 256, 16, 4, 128
    w = orc.make_weights(H, E, I, I, seed=1)
    g = torch.Generator().manual_seed(9)
    x = torch.randn(5, H, generator=g).to(BF16)
    r = torch.randn(5, H, generator=g).to(BF16)
    mlp = _gpu_mlp(w, dev)
    a = pkg.block.moe(x.to(dev), mlp, K)
    b = pkg.block.moe(x.to(dev), mlp, K, residual=r.to(dev))
    torch.cuda.synchronize()
    want = (r.float() + a.cpu().float()).to(BF16)
    assert torch.equal(b.cpu(), want)


def test_calls_repeat(pkg, dev, full_layer):
    """Repeated calls of every regime (decode path, tiled decode, mid-size, multi-block sort)
    on one reused workspace give the same bits."""
    w, _ = full_layer
    mlp = _gpu_mlp(w, dev)
    g = torch.Generator().manual_seed(5)
    for T in (1, 16, 64, 300):
        x = torch.randn(T, 2048, generator=g).to(BF16).to(dev)
        a = pkg.block.moe(x, mlp, 8)
        b = pkg.block.moe(x, mlp, 8)
        torch.cuda.synchronize()
        assert torch.equal(a, b), T


def test_zero_tokens(pkg, dev):
    """Empty batches: every surface returns an empty [0, H] output without launching."""
    H, E, K, I = 256, 16, 4, 128
    w = orc.make_weights(H, E, I, I, seed=3)
    mlp = _gpu_mlp(w, dev)
    x = torch.empty((0, H), dtype=BF16, device=dev)
    out = pkg.block.moe(x, mlp, K)
    assert out.shape == (0, H)
    idx = torch.empty((0, K), dtype=torch.long, device=dev)
    wts = torch.empty((0, K), dtype=BF16, device=dev)
    got = pkg.ops.experts(x, idx, wts, w["gate_up"].to(dev), w["down"].to(dev),
                          round_products=True)
    torch.cuda.synchronize()
    assert got.shape == (0, H)


@pytest.mark.parametrize("E,K,T", [(8, 8, 3), (8, 8, 40), (48, 1, 5), (48, 1, 70), (64, 2, 1)])
def test_block_edge_routings(pkg, dev, E, K, T):
    """Every expert chosen by every token (k = E), one expert per token (k = 1), and an
    expert count that is not a multiple of the 64-lane wave: routing bit-exact given the
    logits, values against the fp32 oracle."""
    _say("block edge", E, K, T)
    H, I = 256, 128
    w = orc.make_weights(H, E, I, I, seed=E + K)
    g = torch.Generator().manual_seed(T + 11)
    x = torch.randn(T, H, generator=g).to(BF16)
    out, idx, wts, logits = pkg.block.moe(x.to(dev), _gpu_mlp(w, dev), K, return_routing=True)
    torch.cuda.synchronize()
    lg = logits.cpu()[:, :E]
    ref_w, ref_i = orc.route(lg, K)
    assert torch.equal(idx.cpu(), ref_i)
    assert torch.equal(wts.cpu(), ref_w)
    f32 = orc.block_fp32(x, w, ref_i, logits=lg)
    _say(f" vs fp32 max {max_abs(out, f32):.3g} mean-rel {mean_rel(out, f32):.3g}")
    assert max_abs(out, f32) <= 2e-2 and mean_rel(out, f32) <= 5e-3


def _sweep_cases():
    """A fixed, seeded spread of block shapes over every regime (decode path, 16/32-row
    expert GEMM tiles, prefill tiles): hidden, experts, top-k, intermediate, shared
    intermediate, tokens."""
    import random

    rnd = random.Random(2026)
    cases = []
    for _ in range(20):
        H = rnd.choice([256, 512, 1024])
        E = rnd.choice([8, 16, 40, 64, 96])
        k = rnd.choice([1, 2, 4, 8] if E >= 8 else [1, 2])
        I = rnd.choice([128, 256, 512])
        IS = rnd.choice([128, 512])
        T = rnd.choice([1, 2, 4, 7, 33, 130, 600])
        cases.append((H, E, k, I, IS, T))
    return cases


@pytest.mark.parametrize("H,E,K,I,IS,T", _sweep_cases())
def test_block_shape_sweep(pkg, dev, H, E, K, I, IS, T):
    """Routing bit-exact given the logits and values against the fp32 oracle over a seeded
    spread of shapes."""
    _say("sweep", H, E, K, I, IS, T)
    w = orc.make_weights(H, E, I, IS, seed=H + E + K + I + IS + T)
    g = torch.Generator().manual_seed(T * 31 + E)
    x = torch.randn(T, H, generator=g).to(BF16)
    out, idx, wts, logits = pkg.block.moe(x.to(dev), _gpu_mlp(w, dev), K, return_routing=True)
    torch.cuda.synchronize()
    lg = logits.cpu()[:, :E]
    ref_w, ref_i = orc.route(lg, K)
    assert torch.equal(idx.cpu(), ref_i)
    assert torch.equal(wts.cpu(), ref_w)
    f32 = orc.block_fp32(x, w, ref_i, logits=lg)
    # the reference torch path (bf16 rounding points) on the same routing: its own mean-rel
    # to fp32 sets the bar where the outputs are small (mean-rel 5e-3 or 1.1x that)
    wc, ic = orc.compact_experts(w, ref_i)
    ref = orc.block_bf16_routed(x, wc, ic, wts.cpu(), logits.cpu()[:, E:E + 1])
    ours, theirs = mean_rel(out, f32), mean_rel(ref, f32)
    _say(f" vs fp32 max {max_abs(out, f32):.3g} mean-rel {ours:.3g} (reference path {theirs:.3g})")
    assert max_abs(out, f32) <= 2e-2
    assert ours <= max(5e-3, 1.1 * theirs)


@pytest.mark.parametrize("T", [600, 1500])
def test_prefill_shared_tile_order_and_side_launch_agree(pkg, dev, full_layer, T):
    """A grouped prefill launch holding routed and shared tiles gives the same bits whether
    the shared expert's tiles are dispatched first (default), in table order, or run as a
    second launch on the auxiliary stream: every tile is computed the same way, only the
    order and the queue differ. Checked for gate_up and down."""
    import os

    w, _ = full_layer
    g = torch.Generator().manual_seed(T + 5)
    x = torch.randn(T, 2048, generator=g).to(BF16).to(dev)
    logits = pkg.ops.router_logits(x, w["router"])
    _, idx, _ = pkg.ops.route(logits, 8, experts=256)
    sp = pkg.ops.sort_pairs(idx, 256, shared=True)
    runs = {}
    for name, env in (("first", {}), ("table", {"MOE_PREFILL_SHARED_FIRST": "0"}),
                      ("side", {"MOE_PREFILL_SIDE": "1"})):
        env = {"MOE_PREFILL_SIDE": None, "MOE_PREFILL_SHARED_FIRST": None, **env}
        with knobs(**env):
            act, act_sh = pkg.ops.grouped_gate_up(x, 8, w["gate_up"], sp,
                                                  shared=(w["sh_gate"], w["sh_up"]))
            y, y_sh = pkg.ops.grouped_down(act, T, 8, w["down"], sp, shared=(w["sh_down"], act_sh))
            torch.cuda.synchronize()
            runs[name] = (act.clone(), act_sh.clone(), y.clone(), y_sh.clone())
    for name in ("table", "side"):
        for a, b in zip(runs["first"], runs[name]):
            assert torch.equal(a, b), name
