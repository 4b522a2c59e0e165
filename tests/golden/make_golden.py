"""Writes the golden fixtures of tests/golden/ from the installed Transformers MoE block.

The fixtures pin the CPU oracle against a third-party implementation of the reference's
semantics (Transformers' Qwen3_5MoeSparseMoeBlock with the batched_mm experts path, which
engine/experts.py:99-100 calls for decode-sized batches). Transformers 5.15.0 is installed;
the reference pins 5.22.1. The weights are regenerated from a seed by
oracle.moe_oracle.make_weights (the fixture stores a checksum of them); the inputs, the
router's indices and weights and the block outputs are stored.

Run from the repository root: python tests/golden/make_golden.py
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import torch
from safetensors.torch import save_file

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import moe_oracle as orc  # noqa: E402

CASES = {
    # name: (hidden, experts, top_k, inter, shared_inter, tokens, weight seed, input seed)
    "c1_tiny_layer": (256, 16, 4, 128, 128, 4, 0, 0),
    "cpu_check_tiny": (64, 8, 2, 32, 32, 5, 0, 1),
}


def weights_digest(w: dict) -> str:
    h = hashlib.sha256()
    for k in sorted(w):
        h.update(k.encode())
        h.update(w[k].contiguous().view(torch.uint8).numpy().tobytes())
    return h.hexdigest()


def run_case(H, E, K, I, IS, T, wseed, xseed):
    from transformers.models.qwen3_5_moe.configuration_qwen3_5_moe import Qwen3_5MoeTextConfig
    from transformers.models.qwen3_5_moe.modeling_qwen3_5_moe import Qwen3_5MoeSparseMoeBlock

    cfg = Qwen3_5MoeTextConfig(hidden_size=H, num_experts=E, num_experts_per_tok=K,
                               moe_intermediate_size=I, shared_expert_intermediate_size=IS)
    cfg._experts_implementation = "batched_mm"
    blk = Qwen3_5MoeSparseMoeBlock(cfg).to(torch.bfloat16)
    w = orc.make_weights(H, E, I, IS, seed=wseed)
    with torch.no_grad():
        blk.gate.weight.copy_(w["router"])
        blk.experts.gate_up_proj.copy_(w["gate_up"])
        blk.experts.down_proj.copy_(w["down"])
        blk.shared_expert.gate_proj.weight.copy_(w["sh_gate"])
        blk.shared_expert.up_proj.weight.copy_(w["sh_up"])
        blk.shared_expert.down_proj.weight.copy_(w["sh_down"])
        blk.shared_expert_gate.weight.copy_(w["sh_gate_w"])
        x = torch.randn(T, H, generator=torch.Generator().manual_seed(xseed)).to(torch.bfloat16)
        out = blk(x[None])
        out = (out[0] if isinstance(out, tuple) else out).reshape(T, H)
        logits, top_w, top_i = blk.gate(x)
    return w, {"x": x, "out": out.contiguous(), "logits": logits.contiguous(),
               "top_k_weights": top_w.contiguous(), "top_k_index": top_i.contiguous()}


def main():
    import transformers

    for name, (H, E, K, I, IS, T, wseed, xseed) in CASES.items():
        w, tensors = run_case(H, E, K, I, IS, T, wseed, xseed)
        meta = {"hidden": str(H), "experts": str(E), "top_k": str(K), "inter": str(I),
                "shared_inter": str(IS), "tokens": str(T), "weight_seed": str(wseed),
                "input_seed": str(xseed), "weights_sha256": weights_digest(w),
                "transformers": transformers.__version__, "torch": torch.__version__,
                "source": "transformers Qwen3_5MoeSparseMoeBlock, experts_implementation=batched_mm"}
        save_file(tensors, str(Path(__file__).parent / f"{name}.safetensors"), metadata=meta)
        print(f"wrote {name}: out max {tensors['out'].float().abs().max():.4f}")


if __name__ == "__main__":
    main()
