"""End-to-end routing from the token rows, and the C3 (batch 64, Zipf(1.1)) workload.

The other parity tests check the routing kernel on the GPU's own router logits. Here the
whole chain runs from ``x``: the GPU's expert indices are compared with the oracle's
routing of CPU ``F.linear(x, W_r)`` logits (the reference's torch path,
engine/fast/model.py:1159-1162; the reference test compares routings up to ties,
tests/test_prefill_kernels.py:142-160). The router's fp32 summation order differs from the
CPU's, so a logit may differ by one bf16 ulp. A token may then be routed differently only
where the CPU logits of the two experts involved are within two bf16 ulps of each other (each
of the two may be off by one ulp in opposite directions). CPU F.linear is itself not
batch-invariant (oneDNN picks its blocking by shape), so the reference path's own routing of a
token can change with the batch it is in, by the same mechanism. Tokens
whose GPU logits equal the CPU logits bit for bit must be routed identically, and their
weights must be bit-equal. The mismatch counts are printed.
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import moe_oracle as orc
from tests.helpers import BF16, max_abs, mean_rel

pytestmark = pytest.mark.gpu

H, E, K, I = 2048, 256, 8, 512


def _say(*a):
    print(*a, flush=True)


def _synth():
    import __graft_entry__

    return __graft_entry__.load_package().synth


def _gpu_mlp(w, dev):
    import __graft_entry__

    return __graft_entry__._mlp_from_weights(w, dev)


def _weights(dev, seed, zipf=False):
    g = torch.Generator(device=dev).manual_seed(seed)

    def rnd(*shape):
        return (torch.randn(*shape, generator=g, device=dev) * 0.02).to(BF16)

    w = {"router": rnd(E, H), "gate_up": rnd(E, 2 * I, H), "down": rnd(E, H, I),
         "sh_gate": rnd(I, H), "sh_up": rnd(I, H), "sh_down": rnd(H, I), "sh_gate_w": rnd(1, H)}
    v = None
    if zipf:
        r, v = _synth().zipf_router(w["router"].cpu(), seed=seed)
        w["router"] = r.to(dev)
    return w, v


@pytest.fixture(scope="module")
def uniform_layer(dev):
    return _weights(dev, seed=21)


@pytest.fixture(scope="module")
def zipf_layer(dev):
    return _weights(dev, seed=2000, zipf=True)


def _bf16_ulp(v: float) -> float:
    """One bf16 ulp at magnitude |v| (8 significant bits)."""
    a = abs(v)
    if a < 2.0 ** -126:
        return 2.0 ** -133
    return 2.0 ** (math.floor(math.log2(a)) - 7)


def check_routing_from_x(x, router, idx, wts, logits, k=K, experts=E):
    """(tokens routed differently, tokens with bit-equal logits, ulp gaps of the swaps).

    Logits: where |logit| >= 1/16 (every routing-relevant logit at these shapes) the GPU
    logit is within one bf16 ulp of the CPU one. Everywhere, its distance from the float64
    product is at most one bf16 ulp of that product plus 2^-16 sum_i |x_i w_i| (room for the
    fp32 summation's rounding, which dominates for logits near zero; CPU F.linear needs
    that room too). Routing: a token routed differently must have, at every slot where the
    two disagree, CPU logits of the two experts within two bf16 ulps: each logit is off by
    at most one ulp, so two neighbours of the CPU order can swap only if they were at most
    two ulps apart."""
    ref_lg = F.linear(x, router.cpu())
    exact = x.double() @ router.cpu().double().t()
    scale = x.double().abs() @ router.cpu().double().abs().t()
    ref_w, ref_i = orc.route(ref_lg, k)
    gi, gw = idx.cpu(), wts.cpu()
    gl = logits.cpu()[:, :experts]
    big = ref_lg.float().abs() >= 1.0 / 16
    d = (gl.float() - ref_lg.float()).abs()
    assert torch.all(d[big] <= ref_lg.float().abs()[big] * 2.0 ** -7), "logits off by > 1 ulp"
    ulp = torch.exp2(torch.floor(torch.log2(exact.abs().clamp_min(2.0 ** -126))) - 7)
    bound = ulp + 2.0 ** -16 * scale
    err_gpu = (gl.double() - exact).abs()
    err_cpu = (ref_lg.double() - exact).abs()
    assert torch.all(err_gpu <= bound), float((err_gpu - bound).max())
    print(f"  logits: max |err| vs float64 GPU {err_gpu.max().item():.3g}, CPU F.linear "
          f"{err_cpu.max().item():.3g}; max err / bound GPU {(err_gpu / bound).max().item():.3g}, "
          f"CPU {(err_cpu / bound).max().item():.3g}", flush=True)
    bad = (gi != ref_i).any(1).nonzero().flatten().tolist()
    gaps = []
    for t in bad:
        row = ref_lg[t].float()
        for j in range(k):
            a, b = int(gi[t, j]), int(ref_i[t, j])
            if a == b:
                continue
            gap = abs(row[a].item() - row[b].item())
            ulp = _bf16_ulp(max(abs(row[a].item()), abs(row[b].item())))
            gaps.append(round(gap / ulp, 3))
            assert gap <= 2 * ulp, (
                f"token {t} slot {j}: GPU expert {a} (logit {row[a].item()}) vs CPU expert {b} "
                f"(logit {row[b].item()}): {gap} > two ulps {2 * ulp}")
    same = (gl == ref_lg).all(1)
    assert torch.equal(gi[same], ref_i[same]), "identical logits routed differently"
    assert torch.equal(gw[same], ref_w[same]), "identical logits weighted differently"
    return len(bad), int(same.sum()), gaps


@pytest.mark.parametrize("name,T", [("c2", 1), ("c3", 64), ("c4", 4096), ("mid", 300)])
def test_routing_from_x_matches_cpu_linear(pkg, dev, uniform_layer, zipf_layer, name, T):
    """C2 (decode router), C3 (Zipf, tiled router), C4 (prefill) and a mid-size batch:
    indices from x against the oracle's routing of CPU logits."""
    w, v = zipf_layer if name == "c3" else uniform_layer
    g = torch.Generator().manual_seed(4000 + T)
    x = torch.randn(T, H, generator=g)
    if v is not None:
        x = x + _synth().ZIPF_MU * v[None, :]
    x = x.to(BF16)
    out, idx, wts, logits = pkg.block.moe(x.to(dev), _gpu_mlp(w, dev), K, return_routing=True)
    torch.cuda.synchronize()
    n_bad, n_same, gaps = check_routing_from_x(x, w["router"], idx, wts, logits)
    _say(f"e2e routing {name} T={T}: {n_bad} of {T} tokens routed differently from CPU "
         f"F.linear logits (CPU logit gaps of the swapped slots, in bf16 ulps: {gaps}); "
         f"{n_same} tokens with bit-equal logits")


@pytest.mark.parametrize("decode", [True, False])
def test_c3_zipf_full_workload(pkg, dev, zipf_layer, decode):
    """The C3 workload as the bench builds it: 64 tokens x + mu v on the Zipf(1.1) router.
    Routing (indices, weights), counts, offsets, order and tile table bit-exact against the
    oracle on the GPU logits; values against the fp32 oracle within the bf16 bar and against
    the reference torch path of the same mode: decode=True (the bench's C3 mode and
    FusedDecode._moe's: routing-weight products rounded to bf16) and decode=False (exact
    fp32 products, the grouped path's)."""
    w, v = zipf_layer
    T = 64
    g = torch.Generator().manual_seed(77)
    x = (torch.randn(T, H, generator=g) + _synth().ZIPF_MU * v[None, :]).to(BF16)
    mlp = _gpu_mlp(w, dev)
    out, idx, wts, logits = pkg.block.moe(x.to(dev), mlp, K, decode=decode, return_routing=True)
    torch.cuda.synchronize()
    lg = logits.cpu()[:, :E]
    ref_w, ref_i = orc.route(lg, K)
    assert torch.equal(idx.cpu(), ref_i)
    assert torch.equal(wts.cpu(), ref_w)
    distinct = int(torch.unique(ref_i).numel())
    counts = torch.bincount(ref_i.reshape(-1), minlength=E)
    _say(f"C3: {distinct} distinct experts, hottest expert {int(counts.max())} pairs")
    assert 120 <= distinct <= 160  # Zipf(1.1) sampling: ~140 (5-95%: 131-151)
    bm = pkg._lib.load().moe_tile_rows(T)
    sp = pkg.ops.sort_pairs(idx, E, bm=bm, shared=True)
    torch.cuda.synchronize()
    c, o, order, tiles = orc.sort_pairs(ref_i, E, bm, tokens=T, shared=True)
    assert torch.equal(sp.counts.cpu(), torch.from_numpy(c))
    assert torch.equal(sp.offsets.cpu(), torch.from_numpy(o))
    assert torch.equal(sp.order.cpu(), torch.from_numpy(order))
    mt = sp.max_tiles
    tab = sp.table.cpu()
    n = int(tab[3 * mt])
    assert [(int(tab[t]), int(tab[mt + t]), int(tab[2 * mt + t])) for t in range(n)] == tiles
    f32 = orc.block_fp32(x, w, ref_i, logits=lg)
    wc, ic = orc.compact_experts(w, ref_i)
    ref = orc.block_bf16_routed(x, wc, ic, wts.cpu(), logits.cpu()[:, E:E + 1], decode=decode)
    ours, theirs = mean_rel(out, f32), mean_rel(ref, f32)
    _say(f"C3 decode={decode} vs fp32: max {max_abs(out, f32):.3g} mean-rel {ours:.3g}; reference path "
         f"mean-rel {theirs:.3g}; ours vs reference path {max_abs(out, ref):.3g}")
    assert max_abs(out, f32) <= 2e-2 and max_abs(out, ref) <= 2e-2
    assert ours <= max(5e-3, 1.1 * theirs)


def test_c3_zipf_fp8_t32(pkg, dev, zipf_layer):
    """The Zipf routing at 32 tokens with fp8-e4m3 experts (C5's weight format): routing
    bit-exact on the GPU logits, values against the fp32 oracle on the dequantised weights
    (the fp8 bar: max-abs 2e-2, mean-rel 6e-3)."""
    w, v = zipf_layer
    T = 32
    fp8 = pkg.fp8
    q, s = fp8.quantize_rows(w["gate_up"])
    q2, s2 = fp8.quantize_rows(w["down"])
    mlp = _gpu_mlp(w, dev)
    mlp.experts.gate_up_proj, mlp.experts.gate_up_scale = q, s
    mlp.experts.down_proj, mlp.experts.down_scale = q2, s2
    g = torch.Generator().manual_seed(78)
    x = (torch.randn(T, H, generator=g) + _synth().ZIPF_MU * v[None, :]).to(BF16)
    out, idx, wts, logits = pkg.block.moe(x.to(dev), mlp, K, decode=True, return_routing=True)
    torch.cuda.synchronize()
    lg = logits.cpu()[:, :E]
    ref_w, ref_i = orc.route(lg, K)
    assert torch.equal(idx.cpu(), ref_i) and torch.equal(wts.cpu(), ref_w)
    wq = dict(w, gate_up=q, down=q2, gate_up_scale=s, down_scale=s2)
    f32 = orc.block_fp32(x, wq, ref_i, logits=lg)
    _say(f"C3 fp8 T=32 vs dequantised fp32: max {max_abs(out, f32):.3g} "
         f"mean-rel {mean_rel(out, f32):.3g}")
    assert max_abs(out, f32) <= 2e-2 and mean_rel(out, f32) <= 6e-3
