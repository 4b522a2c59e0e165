"""fp8 experts written by checkpoint.quantize_checkpoint and loaded back run the block with
the same bits as experts quantised in memory (fp8.quantize_rows), on the decode, tiled and
prefill paths."""

from __future__ import annotations

import pytest
import torch

from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu

H, E, K, I = 512, 16, 4, 512


@pytest.fixture(scope="module")
def fp8_dir(tmp_path_factory):
    from safetensors.torch import save_file

    w = orc.make_weights(H, E, I, I, seed=4)
    root = tmp_path_factory.mktemp("ck")
    src = root / "bf16"
    src.mkdir()
    t = {}
    for j in range(E):
        base = f"model.layers.0.mlp.experts.{j}."
        t[base + "gate_proj.weight"] = w["gate_up"][j, :I].contiguous()
        t[base + "up_proj.weight"] = w["gate_up"][j, I:].contiguous()
        t[base + "down_proj.weight"] = w["down"][j].contiguous()
    save_file(t, str(src / "model.safetensors"))
    return w, src, root / "fp8"


@pytest.mark.parametrize("T", [1, 3, 40, 700])
def test_loaded_fp8_block_matches_in_memory(pkg, dev, fp8_dir, T):
    import __graft_entry__

    w, src, dst = fp8_dir
    if not dst.exists():
        pkg.checkpoint.quantize_checkpoint(src, dst)
    mine = __graft_entry__._mlp_from_weights(w, dev)
    q, s = pkg.fp8.quantize_rows(w["gate_up"])  # on the CPU, as the conversion runs
    q2, s2 = pkg.fp8.quantize_rows(w["down"])
    mine.experts.gate_up_proj, mine.experts.gate_up_scale = q.to(dev), s.to(dev)
    mine.experts.down_proj, mine.experts.down_scale = q2.to(dev), s2.to(dev)
    loaded = __graft_entry__._mlp_from_weights(w, dev)
    loaded.experts = pkg.checkpoint.load_layer(dst, 0, dev)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(T)).to(torch.bfloat16).to(dev)
    a = pkg.block.moe(x, mine, K, decode=T <= 4)
    b = pkg.block.moe(x, loaded, K, decode=T <= 4)
    torch.cuda.synchronize()
    print(f"fp8 checkpoint T={T}: equal={torch.equal(a, b)}", flush=True)
    assert torch.equal(a, b)
