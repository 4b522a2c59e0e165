"""The no-allocation block entry point (moe_block_forward_noalloc, a static device scratch
array instead of a caller workspace) against moe_block_forward through the C ABI: the same
bits on two calls in a row, the second with fewer tokens (the scratch keeps the first call's
contents), in every regime the scratch limit admits; oversized calls are refused."""

from __future__ import annotations

import pytest
import torch

from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def _args(pkg, x, mlp, k, out, idx, wts, logits, residual=None):
    gu, gus, dn, dns, wd = pkg.block._expert_tensors(mlp.experts)
    pack = pkg.block.pack_router(mlp)
    sh = mlp.shared_expert
    p = pkg._lib.ptr
    T, H = x.shape
    E, two_i, _ = gu.shape
    return (p(x), T, H, E, k, two_i // 2, sh.gate_proj.weight.shape[0], p(pack), pack.shape[0],
            p(gu), p(gus), p(dn), p(dns), wd, p(sh.gate_proj.weight), p(sh.up_proj.weight),
            p(sh.down_proj.weight), p(residual),
            pkg._lib.ROUND_PRODUCT if T <= 16 else pkg._lib.EXACT_PRODUCT,
            p(out), p(idx), p(wts), p(logits))


def _run(pkg, x, mlp, k, noalloc, residual=None):
    lib = pkg._lib.load()
    T, H = x.shape
    dev = x.device
    n_pack = pkg.block.pack_router(mlp).shape[0]
    out = torch.empty((T, H), dtype=BF16, device=dev)
    idx = torch.empty((T, k), dtype=torch.long, device=dev)
    wts = torch.empty((T, k), dtype=BF16, device=dev)
    logits = torch.empty((T, n_pack), dtype=BF16, device=dev)
    a = _args(pkg, x, mlp, k, out, idx, wts, logits, residual)
    stream = pkg._lib.stream_of(x)
    if noalloc:
        rc = lib.moe_block_forward_noalloc(*a, stream)
    else:
        gu = mlp.experts.gate_up_proj
        nbytes = lib.moe_block_workspace_bytes(T, H, gu.shape[0], k, gu.shape[1] // 2,
                                               mlp.shared_expert.gate_proj.weight.shape[0],
                                               n_pack)
        ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev)
        rc = lib.moe_block_forward(*a, pkg._lib.ptr(ws), ws.numel(), stream)
    pkg._lib.check(rc, "block")
    return out, idx, wts, logits


@pytest.fixture(scope="module")
def full_mlp(dev):
    import __graft_entry__

    return __graft_entry__._mlp_from_weights(orc.make_weights(2048, 256, 512, 512, seed=41), dev)


@pytest.mark.parametrize("big,small", [(300, 5), (64, 1), (17, 2), (4, 3)])
def test_noalloc_matches_workspace_entry_point(pkg, dev, full_mlp, big, small):
    print(f"no-alloc {big} -> {small}", flush=True)
    g = torch.Generator().manual_seed(big * 7 + small)
    for T in (big, small):
        x = torch.randn(T, 2048, generator=g).to(BF16).to(dev)
        r = torch.randn(T, 2048, generator=g).to(BF16).to(dev)
        got = _run(pkg, x, full_mlp, 8, True, residual=r)
        want = _run(pkg, x, full_mlp, 8, False, residual=r)
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a, b), T


def test_noalloc_fp8_and_small_shape(pkg, dev):
    """fp8 experts (mixed launches) and a C1-sized layer, two calls in a row."""
    import __graft_entry__

    w = orc.make_weights(256, 16, 128, 128, seed=42)
    mlp = __graft_entry__._mlp_from_weights(w, dev)
    q, s = pkg.fp8.quantize_rows(mlp.experts.gate_up_proj)
    q2, s2 = pkg.fp8.quantize_rows(mlp.experts.down_proj)
    fmlp = __graft_entry__._mlp_from_weights(w, dev)
    fmlp.experts.gate_up_proj, fmlp.experts.gate_up_scale = q, s
    fmlp.experts.down_proj, fmlp.experts.down_scale = q2, s2
    g = torch.Generator().manual_seed(5)
    for m in (mlp, fmlp):
        for T in (40, 3):
            x = torch.randn(T, 256, generator=g).to(BF16).to(dev)
            got = _run(pkg, x, m, 4, True)
            want = _run(pkg, x, m, 4, False)
            torch.cuda.synchronize()
            for a, b in zip(got, want):
                assert torch.equal(a, b), T


def test_noalloc_refuses_oversized_calls(pkg, dev, full_mlp):
    lib = pkg._lib.load()
    T = 4096
    assert lib.moe_block_workspace_bytes(T, 2048, 256, 8, 512, 512, 320) > \
        pkg._lib.NOALLOC_SCRATCH_BYTES
    x = torch.zeros((T, 2048), dtype=BF16, device=dev)
    with pytest.raises(ValueError, match="static scratch"):
        _run(pkg, x, full_mlp, 8, True)
