"""On-disk fp8-e4m3 expert weights: quantise a bf16 checkpoint once, load the fp8 layers.

The reference has no fp8 format; its checkpoints are Hugging Face safetensors snapshots (a
``model.safetensors`` or shards listed by ``model.safetensors.index.json``), read as in
engine/mtp.py:153-187. Expert tensors appear either per expert
(``{prefix}layers.{i}.mlp.experts.{j}.{gate,up,down}_proj.weight``, the Hub layout) or
fused (``{prefix}layers.{i}.mlp.experts.{gate_up_proj,down_proj}``, Transformers'
Qwen3_5MoeExperts parameters, modeling_qwen3_5_moe.py:721-731).

The fp8 directory holds one safetensors shard per layer, ``experts-fp8-{i:05d}.safetensors``,
with the fused names and a scale beside each matrix:

    {prefix}layers.{i}.mlp.experts.gate_up_proj   float8_e4m3fn [E, 2I, H]  (rows 0..I-1 gate)
    {prefix}layers.{i}.mlp.experts.gate_up_scale  float32       [E, 2I]
    {prefix}layers.{i}.mlp.experts.down_proj      float8_e4m3fn [E, H, I]
    {prefix}layers.{i}.mlp.experts.down_scale     float32       [E, H]

and ``experts-fp8.index.json`` (``{"metadata": {...}, "weight_map": {name: shard}}``, the
Hub index's shape). Scales are per output row, amax / 448 (``fp8.quantize_rows``), the
layout the fp8 kernels read. Conversion streams one layer at a time, so host memory holds
one layer's bf16 experts (1.5 GiB at H 2048, E 256, I 512), not the model.
"""

from __future__ import annotations

import json
import re
from pathlib import Path

import torch

from .fp8 import quantize_rows

INDEX = "model.safetensors.index.json"
FP8_INDEX = "experts-fp8.index.json"
FORMAT = "moe-mi355x-fp8-e4m3-rowscale-v1"

_FUSED = re.compile(r"^(.*)layers\.(\d+)\.mlp\.experts\.(gate_up_proj|down_proj)$")
_PER_EXPERT = re.compile(r"^(.*)layers\.(\d+)\.mlp\.experts\.(\d+)\.(gate|up|down)_proj\.weight$")


def _weight_map(src: Path) -> dict[str, str]:
    """Tensor name -> shard file of a local safetensors snapshot (engine/mtp.py:153-168)."""
    from safetensors import safe_open

    if (src / INDEX).exists():
        return json.loads((src / INDEX).read_text())["weight_map"]
    single = src / "model.safetensors"
    if not single.exists():
        raise FileNotFoundError(f"{src} has neither {INDEX} nor model.safetensors")
    with safe_open(str(single), framework="pt") as reader:
        return dict.fromkeys(reader.keys(), "model.safetensors")


def expert_layers(src: str | Path) -> dict[int, dict]:
    """The expert tensors of each layer of a bf16 snapshot: {layer: {"prefix", "fused": {kind:
    (name, shard)}, "per_expert": {(j, proj): (name, shard)}}}."""
    layers: dict[int, dict] = {}
    for name, shard in _weight_map(Path(src)).items():
        m = _FUSED.match(name)
        if m:
            d = layers.setdefault(int(m.group(2)), {"prefix": m.group(1), "fused": {},
                                                     "per_expert": {}})
            d["fused"][m.group(3)] = (name, shard)
            continue
        m = _PER_EXPERT.match(name)
        if m:
            d = layers.setdefault(int(m.group(2)), {"prefix": m.group(1), "fused": {},
                                                     "per_expert": {}})
            d["per_expert"][(int(m.group(3)), m.group(4))] = (name, shard)
    return layers


def _read(src: Path, entries) -> dict[str, torch.Tensor]:
    from safetensors import safe_open

    by_shard: dict[str, list[str]] = {}
    for name, shard in entries:
        by_shard.setdefault(shard, []).append(name)
    out = {}
    for shard, names in by_shard.items():
        with safe_open(str(src / shard), framework="pt") as reader:
            for name in names:
                out[name] = reader.get_tensor(name)
    return out


def _layer_bf16(src: Path, info: dict) -> tuple[torch.Tensor, torch.Tensor]:
    """(gate_up [E, 2I, H], down [E, H, I]) of one layer, fused from either layout."""
    fused, per = info["fused"], info["per_expert"]
    if fused:
        if set(fused) != {"gate_up_proj", "down_proj"}:
            raise ValueError(f"layer has only {sorted(fused)} of gate_up_proj / down_proj")
        t = _read(src, fused.values())
        return t[fused["gate_up_proj"][0]], t[fused["down_proj"][0]]
    experts = sorted({j for j, _ in per})
    if experts != list(range(len(experts))):
        raise ValueError("per-expert tensors must number the experts 0..E-1")
    for j in experts:
        for proj in ("gate", "up", "down"):
            if (j, proj) not in per:
                raise ValueError(f"expert {j} has no {proj}_proj")
    t = _read(src, per.values())
    gate_up = torch.stack([torch.cat((t[per[(j, "gate")][0]], t[per[(j, "up")][0]]), dim=0)
                           for j in experts])
    down = torch.stack([t[per[(j, "down")][0]] for j in experts])
    return gate_up, down


def names(prefix: str, layer: int) -> dict[str, str]:
    base = f"{prefix}layers.{layer}.mlp.experts."
    return {k: base + k for k in ("gate_up_proj", "gate_up_scale", "down_proj", "down_scale")}


def quantize_checkpoint(src: str | Path, dst: str | Path, layers=None) -> Path:
    """Write the fp8 expert shards and index of bf16 snapshot ``src`` into ``dst``
    (``layers``: an iterable of layer numbers, default all). Returns the index path."""
    from safetensors.torch import save_file

    src, dst = Path(src), Path(dst)
    found = expert_layers(src)
    if not found:
        raise ValueError(f"{src} holds no MoE expert tensors")
    todo = sorted(found) if layers is None else sorted(layers)
    missing = [i for i in todo if i not in found]
    if missing:
        raise ValueError(f"layers {missing} have no expert tensors in {src}")
    dst.mkdir(parents=True, exist_ok=True)
    meta = {"format": FORMAT, "scale": "per output row: amax / 448", "source": str(src)}
    weight_map = {}
    for i in todo:
        gate_up, down = _layer_bf16(src, found[i])
        if gate_up.dim() != 3 or down.dim() != 3 or gate_up.shape[0] != down.shape[0] or \
                gate_up.shape[2] != down.shape[1] or gate_up.shape[1] != 2 * down.shape[2]:
            raise ValueError(f"layer {i}: gate_up {tuple(gate_up.shape)} and down "
                             f"{tuple(down.shape)} are not [E, 2I, H] / [E, H, I]")
        q, s = quantize_rows(gate_up)
        q2, s2 = quantize_rows(down)
        n = names(found[i]["prefix"], i)
        shard = f"experts-fp8-{i:05d}.safetensors"
        save_file({n["gate_up_proj"]: q, n["gate_up_scale"]: s, n["down_proj"]: q2,
                   n["down_scale"]: s2}, str(dst / shard), metadata={"format": "pt"})
        weight_map.update(dict.fromkeys(n.values(), shard))
        del gate_up, down, q, s, q2, s2
    index = dst / FP8_INDEX
    old = json.loads(index.read_text()) if index.exists() else {"weight_map": {}}
    old["weight_map"].update(weight_map)
    old["metadata"] = meta
    index.write_text(json.dumps(old, indent=1, sort_keys=True))
    return index


class Fp8LayerExperts(torch.nn.Module):
    """One layer's fp8 experts as the MoE surfaces read them (``gate_up_proj``,
    ``gate_up_scale``, ``down_proj``, ``down_scale``, ``num_experts``)."""

    def __init__(self, t: dict[str, torch.Tensor], n: dict[str, str]):
        super().__init__()
        self.gate_up_proj = t[n["gate_up_proj"]]
        self.gate_up_scale = t[n["gate_up_scale"]]
        self.down_proj = t[n["down_proj"]]
        self.down_scale = t[n["down_scale"]]
        self.num_experts = self.gate_up_proj.shape[0]
        self.act_fn = torch.nn.functional.silu


def load_layer(dst: str | Path, layer: int, device="cpu") -> Fp8LayerExperts:
    """Layer ``layer``'s fp8 experts from an fp8 directory, on ``device``."""
    from safetensors import safe_open

    dst = Path(dst)
    index = json.loads((dst / FP8_INDEX).read_text())
    if index.get("metadata", {}).get("format") != FORMAT:
        raise ValueError(f"{dst / FP8_INDEX} is not a {FORMAT} index")
    wanted = {name: shard for name, shard in index["weight_map"].items()
              if re.search(rf"(^|\.)layers\.{layer}\.mlp\.experts\.", name)}
    if len(wanted) != 4:
        raise KeyError(f"layer {layer} is not in {dst}")
    prefix = next(iter(wanted)).split(f"layers.{layer}.mlp.experts.")[0]
    n = names(prefix, layer)
    out = {}
    for name, shard in wanted.items():
        with safe_open(str(dst / shard), framework="pt", device=str(device)) as reader:
            out[name] = reader.get_tensor(name)
    fp8 = torch.float8_e4m3fn
    if out[n["gate_up_proj"]].dtype != fp8 or out[n["down_proj"]].dtype != fp8 or \
            out[n["gate_up_scale"]].dtype != torch.float32:
        raise ValueError(f"layer {layer}: unexpected dtypes in {dst}")
    return Fp8LayerExperts(out, n)


def attach(mlps, dst: str | Path, device=None) -> None:
    """Point each block ``mlps[i]`` (e.g. ``model.layers[i].mlp``) at layer i's fp8 experts,
    loaded onto ``device`` (default: the device of its current expert weights)."""
    for i, mlp in enumerate(mlps):
        dev = device if device is not None else mlp.experts.gate_up_proj.device
        mlp.experts = load_layer(dst, i, dev)
