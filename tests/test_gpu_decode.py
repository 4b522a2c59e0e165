"""The three-launch decode path (T <= 4 tokens, hidden and intermediates multiples of 512).

It regroups the block's work (dot products over whole weight rows, routing recomputed per
workgroup, combine fused into the down projection) but keeps every rounding point of the
tiled path, so:
- routing (indices and bf16 weights) is bit-identical to the tiled path's and to the
  oracle's route() on the same logits;
- outputs match the fp32 oracle to the bf16 bar (max-abs 2e-2, mean-rel 5e-3 or 1.1x the
  reference torch path's own mean-rel) and the tiled path to a few bf16 ulps (the two
  differ only in fp32 summation order inside each projection);
- residual: out(x, r) == bf16(r + out(x)) exactly, as for the tiled path.
"""

from __future__ import annotations


import pytest
import torch

from oracle import moe_oracle as orc
from tests.helpers import BF16, knobs, max_abs, mean_rel, routing

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _tiled():
    """Run the body with the decode path switched off (MOE_DECODE=0)."""
    return knobs(MOE_DECODE="0")


def _weights(dev, seed, H=2048, E=256, I=512, IS=512):
    g = torch.Generator(device=dev).manual_seed(seed)

    def rnd(*shape):
        return (torch.randn(*shape, generator=g, device=dev) * 0.02).to(BF16)

    return {"router": rnd(E, H), "gate_up": rnd(E, 2 * I, H), "down": rnd(E, H, I),
            "sh_gate": rnd(IS, H), "sh_up": rnd(IS, H), "sh_down": rnd(H, IS),
            "sh_gate_w": rnd(1, H)}


@pytest.fixture(scope="module")
def layer(dev):
    return _weights(dev, seed=21)


def _mlp(w, dev):
    import __graft_entry__

    return __graft_entry__._mlp_from_weights(w, dev)


@pytest.mark.parametrize("T", [1, 2, 3, 4])
def test_decode_block_matches_oracle_and_tiled(pkg, dev, layer, T):
    _say("decode block", T)
    mlp = _mlp(layer, dev)
    x = torch.randn(T, 2048, generator=torch.Generator().manual_seed(100 + T)).to(BF16).to(dev)
    out, idx, wts, logits = pkg.block.moe(x, mlp, 8, decode=True, return_routing=True)
    again = pkg.block.moe(x, mlp, 8, decode=True)
    with _tiled():
        t_out, t_idx, t_wts, t_lg = pkg.block.moe(x, mlp, 8, decode=True, return_routing=True)
    torch.cuda.synchronize()
    assert torch.equal(out, again), "not deterministic"
    lg = logits.cpu()[:, :256]
    ref_w, ref_i = orc.route(lg, 8)
    assert torch.equal(idx.cpu(), ref_i)
    assert torch.equal(wts.cpu(), ref_w)
    # the two paths' router logits differ only in summation order
    assert max_abs(logits, t_lg) <= 2.0 ** -7 * max(1.0, t_lg.float().abs().max().item())
    xc = x.cpu()
    f32 = orc.block_fp32(xc, {k_: v.cpu() for k_, v in layer.items()}, ref_i, logits=lg)
    wc, ic = orc.compact_experts({k_: v.cpu() for k_, v in layer.items()}, ref_i)
    ref = orc.block_bf16_routed(xc, wc, ic, wts.cpu(), logits.cpu()[:, 256:257])
    ours, theirs = mean_rel(out, f32), mean_rel(ref, f32)
    _say(f" vs fp32 max {max_abs(out, f32):.3g} mean-rel {ours:.3g} (reference path "
         f"{theirs:.3g}); vs tiled max {max_abs(out, t_out):.3g}")
    assert max_abs(out, f32) <= 2e-2
    assert ours <= max(5e-3, 1.1 * theirs)
    if torch.equal(idx, t_idx):
        assert max_abs(out, t_out) <= 4e-3


def test_decode_residual_exact(pkg, dev, layer):
    mlp = _mlp(layer, dev)
    g = torch.Generator().manual_seed(7)
    x = torch.randn(3, 2048, generator=g).to(BF16).to(dev)
    r = torch.randn(3, 2048, generator=g).to(BF16).to(dev)
    a = pkg.block.moe(x, mlp, 8, decode=True)
    b = pkg.block.moe(x, mlp, 8, decode=True, residual=r)
    torch.cuda.synchronize()
    assert torch.equal(b.cpu(), (r.cpu().float() + a.cpu().float()).to(BF16))


@pytest.mark.parametrize("mode", ["uniform", "skewed", "sparse", "one"])
@pytest.mark.parametrize("n", [1, 2, 4])
@pytest.mark.parametrize("shape", [(16, 512, 512, 4), (32, 1024, 1024, 8)])
def test_decode_experts_forward(pkg, dev, n, mode, shape):
    """Routed experts only (the Transformers experts surface), given routings including
    repeated experts inside one token ("one") and across tokens ("skewed", "sparse")."""
    e, h, i, k = shape
    _say("decode experts", n, mode, shape)
    g = torch.Generator().manual_seed(n * 7 + len(mode))
    gu = (torch.randn(e, 2 * i, h, generator=g) * 0.05).to(BF16)
    dn = (torch.randn(e, h, i, generator=g) * 0.05).to(BF16)
    x = torch.randn(n, h, generator=g).to(BF16)
    idx, w = routing(n, e, k, mode, g)
    args = (x.to(dev), idx.to(dev), w.to(dev), gu.to(dev), dn.to(dev))
    got = pkg.ops.experts(*args, round_products=True)
    with _tiled():
        tiled = pkg.ops.experts(*args, round_products=True)
    torch.cuda.synchronize()
    ref = orc.experts_forward(x, idx, w, gu, dn)
    scale = max(1.0, ref.float().abs().max().item())
    _say(f" vs oracle {max_abs(got, ref):.3g}; vs tiled {max_abs(got, tiled):.3g}")
    assert max_abs(got, ref) <= 2e-2 * scale
    assert max_abs(got, tiled) <= 8e-3 * scale


@pytest.mark.parametrize("T", [1, 2, 3, 4])
def test_decode_fp8_block(pkg, dev, layer, T):
    """fp8-e4m3 routed experts on the decode path against the dequantised fp32 oracle and
    the tiled fp8 path."""
    mlp = _mlp(layer, dev)
    q, s = pkg.fp8.quantize_rows(layer["gate_up"])
    q2, s2 = pkg.fp8.quantize_rows(layer["down"])
    mlp.experts.gate_up_proj, mlp.experts.gate_up_scale = q, s
    mlp.experts.down_proj, mlp.experts.down_scale = q2, s2
    x = torch.randn(T, 2048, generator=torch.Generator().manual_seed(T)).to(BF16).to(dev)
    out, idx, wts, logits = pkg.block.moe(x, mlp, 8, decode=True, return_routing=True)
    with _tiled():
        t_out, t_idx, _, _ = pkg.block.moe(x, mlp, 8, decode=True, return_routing=True)
    torch.cuda.synchronize()
    lg = logits.cpu()[:, :256]
    _, ref_i = orc.route(lg, 8)
    assert torch.equal(idx.cpu(), ref_i)
    wq = {k_: v.cpu() for k_, v in layer.items()}
    wq.update(gate_up=q.cpu(), down=q2.cpu(), gate_up_scale=s.cpu(), down_scale=s2.cpu())
    f32_q = orc.block_fp32(x.cpu(), wq, ref_i, logits=lg)
    _say(f"decode fp8 T={T}: vs dequantised fp32 max {max_abs(out, f32_q):.3g} mean-rel "
         f"{mean_rel(out, f32_q):.3g}; vs tiled {max_abs(out, t_out):.3g}")
    assert max_abs(out, f32_q) <= 2e-2 and mean_rel(out, f32_q) <= 6e-3
    if torch.equal(idx, t_idx):
        assert max_abs(out, t_out) <= 4e-3


@pytest.mark.parametrize("shared_in", ["router", "gate_up"])
def test_decode_stages_compose_to_block(pkg, dev, layer, shared_in):
    """The operator-level stages (decode_router -> decode_gate_up -> decode_down) give the
    block's bits, with the shared gate/up rows in either of the first two launches."""
    mlp = _mlp(layer, dev)
    x = torch.randn(2, 2048, generator=torch.Generator().manual_seed(3)).to(BF16).to(dev)
    pack = pkg.block.pack_router(mlp)
    sh = mlp.shared_expert
    sh_gu = (sh.gate_proj.weight, sh.up_proj.weight)
    if shared_in == "router":
        logits, act_sh = pkg.ops.decode_router(x, pack, shared=sh_gu)
        act, idx32, wts, idx64 = pkg.ops.decode_gate_up(x, layer["gate_up"], 8, logits=logits,
                                                        experts=256)
    else:
        logits, _ = pkg.ops.decode_router(x, pack)
        act, idx32, wts, idx64, act_sh = pkg.ops.decode_gate_up(
            x, layer["gate_up"], 8, logits=logits, experts=256, shared=sh_gu)
    out = pkg.ops.decode_down(act, 2, 8, layer["down"], idx32, wts,
                              shared=(sh.down_proj.weight, act_sh), logits=logits, experts=256)
    b_out, b_idx, b_wts, b_lg = pkg.block.moe(x, mlp, 8, decode=True, return_routing=True)
    torch.cuda.synchronize()
    assert torch.equal(logits, b_lg)
    assert torch.equal(idx64, b_idx) and torch.equal(idx32.long(), b_idx)
    assert torch.equal(wts, b_wts)
    assert torch.equal(out, b_out)


@pytest.mark.parametrize("fp8", [False, True])
def test_decode_one_token_down_kernels_agree(pkg, dev, layer, fp8):
    """One token: the wave-per-pair down kernel and the wave-per-row one compute the same
    dot products in the same order, so they give the same bits."""
    mlp = _mlp(layer, dev)
    if fp8:
        q, s = pkg.fp8.quantize_rows(layer["gate_up"])
        q2, s2 = pkg.fp8.quantize_rows(layer["down"])
        mlp.experts.gate_up_proj, mlp.experts.gate_up_scale = q, s
        mlp.experts.down_proj, mlp.experts.down_scale = q2, s2
    g = torch.Generator().manual_seed(77)
    x = torch.randn(1, 2048, generator=g).to(BF16).to(dev)
    r = torch.randn(1, 2048, generator=g).to(BF16).to(dev)
    a = pkg.block.moe(x, mlp, 8, decode=True, residual=r)
    with knobs(MOE_DECODE_DOWN="rows"):
        b = pkg.block.moe(x, mlp, 8, decode=True, residual=r)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("T", [3, 4])
@pytest.mark.parametrize("routes", ["random", "shared_experts"])
def test_decode_gate_up_row_blocks_agree(pkg, dev, layer, T, routes):
    """Three or four tokens: the gate_up kernel that takes four row blocks per workgroup
    (token rows staged in LDS) and the one-block kernel compute the same dot products in
    the same order, so the block's outputs and routing agree bit for bit, also when tokens
    share experts (one workgroup then serves several pairs)."""
    mlp = _mlp(layer, dev)
    g = torch.Generator().manual_seed(90 + T)
    x = torch.randn(T, 2048, generator=g)
    if routes == "shared_experts":
        x[1:] = x[0] + 0.05 * x[1:]  # near-identical tokens: mostly the same experts
    x = x.to(BF16).to(dev)
    r = torch.randn(T, 2048, generator=g).to(BF16).to(dev)
    got = {}
    for blocks in ("4", "2", "1"):
        with knobs(MOE_DECODE_GU_BLOCKS=blocks):
            got[blocks] = pkg.block.moe(x, mlp, 8, decode=True, residual=r, return_routing=True)
    torch.cuda.synchronize()
    distinct = int(torch.unique(got["1"][1]).numel())
    _say(f"decode gate_up row blocks T={T} {routes}: {distinct} distinct experts")
    if routes == "shared_experts":
        assert distinct < T * 8
    for blocks in ("4", "2"):
        for a, b in zip(got[blocks], got["1"]):
            assert torch.equal(a, b), blocks


@pytest.mark.parametrize("E,k", [(256, 8), (64, 8), (16, 4)])
def test_decode_gate_up_hard_routing_rows(pkg, dev, E, k):
    """One token per call on rows built to need the exact-selection fallback (p ties from
    exp underflow, subnormal boundary p, tiny boundary logits, exact logit ties) and the
    reference's tie families: indices bit-exact against the oracle, weights within one bf16
    ulp, and the activations bit-equal to the same launch given those indices."""
    from tests.test_gpu_parity import _hard_rows
    from tests.helpers import router_rows

    g = torch.Generator().manual_seed(E * 3 + k)
    rows = torch.cat([_hard_rows(E, g), router_rows(8, E, 11)])
    H, I = 512, 512
    gd = torch.Generator(device=dev).manual_seed(E)
    gu = (torch.randn(E, 2 * I, H, generator=gd, device=dev) * 0.05).to(BF16)
    for r in range(rows.shape[0]):
        x = torch.randn(1, H, generator=g).to(BF16).to(dev)
        lg = rows[r : r + 1].to(dev)
        act, idx32, wts, idx64 = pkg.ops.decode_gate_up(x, gu, k, logits=lg, experts=E)
        act2, _, _, _ = pkg.ops.decode_gate_up(x, gu, k, top_k_index=idx64)
        torch.cuda.synchronize()
        ref_w, ref_i = orc.route(rows[r : r + 1], k)
        assert torch.equal(idx64.cpu(), ref_i), f"row {r}"
        assert torch.equal(idx32.long().cpu(), ref_i)
        d = (wts.float().cpu() - ref_w.float()).abs()
        assert (d <= ref_w.float().abs() * 2.0 ** -7 + 1e-30).all(), f"row {r}"
        assert torch.equal(act, act2), f"row {r}"


@pytest.mark.parametrize("T", [1, 3])
def test_hidden_1536_takes_tiled_path(pkg, dev, T):
    """H = 1536 (a multiple of 512 the decode kernels are not built for) at decode sizes:
    the block takes the tiled path and matches the oracle."""
    import __graft_entry__

    H, E, K, I = 1536, 32, 4, 512
    w = orc.make_weights(H, E, I, I, seed=15)
    g = torch.Generator().manual_seed(T)
    x = torch.randn(T, H, generator=g).to(BF16)
    mlp = __graft_entry__._mlp_from_weights(w, dev)
    out, idx, wts, logits = pkg.block.moe(x.to(dev), mlp, K, decode=True, return_routing=True)
    torch.cuda.synchronize()
    lg = logits.cpu()[:, :E]
    ref_w, ref_i = orc.route(lg, K)
    assert torch.equal(idx.cpu(), ref_i)
    f32 = orc.block_fp32(x, w, ref_i, logits=lg)
    wc, ic = orc.compact_experts(w, ref_i)
    ref = orc.block_bf16_routed(x, wc, ic, wts.cpu(), logits.cpu()[:, E:E + 1], decode=True)
    ours, theirs = mean_rel(out, f32), mean_rel(ref, f32)
    print(f"H=1536 T={T}: max {max_abs(out, f32):.3g} mean-rel {ours:.3g} "
          f"(reference path {theirs:.3g})", flush=True)
    assert max_abs(out, f32) <= 2e-2 and max_abs(out, ref) <= 2e-2
    assert ours <= max(5e-3, 1.1 * theirs)
