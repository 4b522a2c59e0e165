"""The golden fixtures (tests/golden/, written from Transformers' Qwen3_5MoeSparseMoeBlock by
tests/golden/make_golden.py): the CPU oracle reproduces them bit for bit, and the gfx950
block reproduces their routing bit for bit and their outputs within the bf16 bar."""

from __future__ import annotations

from pathlib import Path

import pytest
import torch
from safetensors import safe_open

from oracle import moe_oracle as orc
from tests.golden.make_golden import weights_digest
from tests.helpers import max_abs, mean_rel

GOLDEN = Path(__file__).parent / "golden"
NAMES = ["c1_tiny_layer", "cpu_check_tiny"]


def _load(name):
    with safe_open(str(GOLDEN / f"{name}.safetensors"), "pt") as f:
        meta = f.metadata()
        t = {k: f.get_tensor(k) for k in f.keys()}
    H, E, I, IS = (int(meta[k]) for k in ("hidden", "experts", "inter", "shared_inter"))
    w = orc.make_weights(H, E, I, IS, seed=int(meta["weight_seed"]))
    assert weights_digest(w) == meta["weights_sha256"], "weight regeneration drifted"
    return meta, t, w


def _tie_rule(idx, logits):
    """Transformers' torch.topk order rewritten with the tie rule the kernels and the oracle
    use (descending probability, then ascending index)."""
    p = torch.softmax(logits.float(), -1)
    out = []
    for r in range(idx.shape[0]):
        row = sorted(idx[r].tolist(), key=lambda e: (-p[r, e].item(), e))
        out.append(row)
    return torch.tensor(out, dtype=idx.dtype)


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_golden(name):
    meta, t, w = _load(name)
    k = int(meta["top_k"])
    out, idx, wts, logits = orc.block_bf16(t["x"], w, k)
    assert torch.equal(logits, t["logits"])
    # cpu_check_tiny row 1 has an exact tie (experts 2 and 5, logit 0.1406): torch.topk
    # returned (5, 2), the tie rule gives (2, 5); same set, same weights.
    assert torch.equal(idx, _tie_rule(t["top_k_index"], t["logits"]))
    assert torch.equal(wts.sort(-1).values, t["top_k_weights"].sort(-1).values)
    if torch.equal(idx, t["top_k_index"]):
        assert torch.equal(out, t["out"])
    else:  # the k terms are summed in another order: one bf16 ulp at most
        assert max_abs(out, t["out"]) <= 2.0 ** -8 * t["out"].float().abs().max().item()


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_gpu_block_on_golden(pkg, dev, name):
    import __graft_entry__

    meta, t, w = _load(name)
    k = int(meta["top_k"])
    mlp = __graft_entry__._mlp_from_weights(w, dev)
    out, idx, wts, logits = pkg.block.moe(t["x"].to(dev), mlp, k, return_routing=True)
    torch.cuda.synchronize()
    assert torch.equal(idx.cpu(), _tie_rule(t["top_k_index"], t["logits"]))
    assert max_abs(out.cpu(), t["out"]) <= 2e-2
    f32 = orc.block_fp32(t["x"], w, t["top_k_index"], logits=t["logits"])
    print(f"golden {name}: vs fixture max {max_abs(out.cpu(), t['out']):.3g}; vs fp32 max "
          f"{max_abs(out.cpu(), f32):.3g} mean-rel {mean_rel(out.cpu(), f32):.3g}; fixture vs fp32 "
          f"mean-rel {mean_rel(t['out'], f32):.3g}", flush=True)
    # measured: bit-equal to the fixture (the Transformers block's own output), whose
    # mean-rel to fp32 is 4.2e-3 / 4.9e-3
    assert max_abs(out.cpu(), f32) <= 2e-3
    assert mean_rel(out.cpu(), f32) <= max(5e-3, 1.1 * mean_rel(t["out"], f32))
