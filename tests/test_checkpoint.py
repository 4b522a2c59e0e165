"""The on-disk fp8 expert format (checkpoint.py): conversion from both bf16 snapshot layouts
and loading, on the CPU.

The masters are chosen so that quantisation is exact: every row holds 448 * 2^-10 (so its
scale is exactly 2^-10) and otherwise multiples of 2^-10 that e4m3 represents exactly. The
loaded fp8 weights times their scales must then give back the bf16 masters bit for bit,
which pins the fused row order (gate rows, then up rows), the [E, H, I] down layout and
the per-row scales independently of the quantiser's own arithmetic.
"""

from __future__ import annotations

import json

import pytest
import torch

E, H, I = 4, 32, 16
LAYERS = 3
BF16 = torch.bfloat16
E4M3_SMALL = torch.tensor([0.0, 1.0, -1.0, 2.0, -3.0, 4.0, 6.0, -8.0, 12.0, -16.0, 28.0, 64.0])


def _masters(seed):
    """[E, rows, K] bf16 masters whose rows quantise exactly (scale 2^-10)."""
    g = torch.Generator().manual_seed(seed)

    def mat(rows, k):
        pick = torch.randint(0, len(E4M3_SMALL), (E, rows, k), generator=g)
        v = E4M3_SMALL[pick]
        v[:, :, 0] = 448.0 * torch.where(torch.rand(E, rows, generator=g) < 0.5, -1.0, 1.0)
        return (v * 2.0 ** -10).to(BF16)

    return mat(2 * I, H), mat(H, I)


def _write_per_expert(path, layers):
    from safetensors.torch import save_file

    t = {"model.embed_tokens.weight": torch.zeros(8, H, dtype=BF16)}
    for i, (gu, dn) in enumerate(layers):
        for j in range(E):
            base = f"model.layers.{i}.mlp.experts.{j}."
            t[base + "gate_proj.weight"] = gu[j, :I].contiguous()
            t[base + "up_proj.weight"] = gu[j, I:].contiguous()
            t[base + "down_proj.weight"] = dn[j].contiguous()
        t[f"model.layers.{i}.mlp.gate.weight"] = torch.zeros(E, H, dtype=BF16)
    path.mkdir()
    save_file(t, str(path / "model.safetensors"))


def _write_fused_sharded(path, layers):
    from safetensors.torch import save_file

    path.mkdir()
    wm = {}
    for i, (gu, dn) in enumerate(layers):
        shard = f"model-{i:05d}-of-{LAYERS:05d}.safetensors"
        t = {f"model.language_model.layers.{i}.mlp.experts.gate_up_proj": gu,
             f"model.language_model.layers.{i}.mlp.experts.down_proj": dn}
        save_file(t, str(path / shard))
        wm.update(dict.fromkeys(t, shard))
    (path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))


@pytest.fixture(scope="module")
def layers():
    return [_masters(10 + i) for i in range(LAYERS)]


@pytest.mark.parametrize("layout", ["per_expert", "fused_sharded"])
def test_convert_and_load_exact(pkg, tmp_path, layers, layout):
    ck = pkg.checkpoint
    src, dst = tmp_path / "bf16", tmp_path / "fp8"
    (_write_per_expert if layout == "per_expert" else _write_fused_sharded)(src, layers)
    assert sorted(ck.expert_layers(src)) == list(range(LAYERS))
    ck.quantize_checkpoint(src, dst)
    index = json.loads((dst / ck.FP8_INDEX).read_text())
    assert index["metadata"]["format"] == ck.FORMAT
    assert len(index["weight_map"]) == 4 * LAYERS
    for i, (gu, dn) in enumerate(layers):
        ex = ck.load_layer(dst, i)
        assert ex.gate_up_proj.dtype == torch.float8_e4m3fn and ex.gate_up_proj.shape == (E, 2 * I, H)
        assert ex.down_proj.dtype == torch.float8_e4m3fn and ex.down_proj.shape == (E, H, I)
        assert ex.gate_up_scale.shape == (E, 2 * I) and ex.down_scale.shape == (E, H)
        assert torch.all(ex.gate_up_scale == 2.0 ** -10) and torch.all(ex.down_scale == 2.0 ** -10)
        back = (ex.gate_up_proj.float() * ex.gate_up_scale[..., None]).to(BF16)
        assert torch.equal(back, gu)
        back = (ex.down_proj.float() * ex.down_scale[..., None]).to(BF16)
        assert torch.equal(back, dn)


def test_convert_subset_then_rest(pkg, tmp_path, layers):
    """Converting some layers, then the others, merges into one index."""
    ck = pkg.checkpoint
    src, dst = tmp_path / "bf16", tmp_path / "fp8"
    _write_per_expert(src, layers)
    ck.quantize_checkpoint(src, dst, layers=[1])
    with pytest.raises(KeyError):
        ck.load_layer(dst, 0)
    ck.quantize_checkpoint(src, dst, layers=[0, 2])
    for i in range(LAYERS):
        ck.load_layer(dst, i)
    with pytest.raises(ValueError):
        ck.quantize_checkpoint(src, dst, layers=[7])


def test_attach_replaces_experts(pkg, tmp_path, layers):
    ck = pkg.checkpoint
    src, dst = tmp_path / "bf16", tmp_path / "fp8"
    _write_fused_sharded(src, layers)
    ck.quantize_checkpoint(src, dst)

    class Experts(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.gate_up_proj = torch.nn.Parameter(torch.zeros(E, 2 * I, H, dtype=BF16))

    class Mlp(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.experts = Experts()

    mlps = [Mlp() for _ in range(LAYERS)]
    ck.attach(mlps, dst)
    for i, m in enumerate(mlps):
        assert m.experts.gate_up_proj.dtype == torch.float8_e4m3fn
        q, s = pkg.fp8.quantize_rows(layers[i][0])
        assert torch.equal(m.experts.gate_up_proj.view(torch.uint8), q.view(torch.uint8))
        assert torch.equal(m.experts.gate_up_scale, s)


def test_incomplete_checkpoints_are_rejected(pkg, tmp_path, layers):
    from safetensors.torch import save_file

    ck = pkg.checkpoint
    src = tmp_path / "bf16"
    src.mkdir()
    gu, dn = layers[0]
    t = {}
    for j in range(E):
        base = f"model.layers.0.mlp.experts.{j}."
        t[base + "gate_proj.weight"] = gu[j, :I].contiguous()
        t[base + "up_proj.weight"] = gu[j, I:].contiguous()
        if j != 2:
            t[base + "down_proj.weight"] = dn[j].contiguous()
    save_file(t, str(src / "model.safetensors"))
    with pytest.raises(ValueError, match="expert 2 has no down_proj"):
        ck.quantize_checkpoint(src, tmp_path / "fp8")
    with pytest.raises(FileNotFoundError):
        ck.quantize_checkpoint(tmp_path / "nowhere", tmp_path / "fp8b")
