"""The Transformers boundary as the engine uses it, on the GPU.

The reference registers its experts function with ``ExpertsInterface.register(NAME, fn)``
(engine/experts.py:105-108) and selects it with ``experts_implementation`` when it loads
the model (engine/generator.py:653-661). Transformers then reaches it through
``use_experts_implementation.forward`` inside ``Qwen3_5MoeSparseMoeBlock.forward``
(modeling_qwen3_5_moe.py:787-800). Here a real ``Qwen3_5MoeSparseMoeBlock`` of the
installed Transformers is built in bf16 on the GPU with ``experts_implementation`` set to
``register()``'s name, and run at 1, 17 and 300 tokens. The same module is also passed as
``mlp`` to the block-level surface (``block.moe``), which reads its parameters in place.
"""

from __future__ import annotations

import pytest
import torch

from oracle import moe_oracle as orc
from tests.helpers import BF16, max_abs, mean_rel

pytestmark = pytest.mark.gpu

H, E, K, I = 2048, 256, 8, 512


def _say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def tf_block(pkg, dev):
    from transformers.models.qwen3_5_moe.configuration_qwen3_5_moe import Qwen3_5MoeTextConfig
    from transformers.models.qwen3_5_moe.modeling_qwen3_5_moe import Qwen3_5MoeSparseMoeBlock

    cfg = Qwen3_5MoeTextConfig(hidden_size=H, num_experts=E, num_experts_per_tok=K,
                               moe_intermediate_size=I, shared_expert_intermediate_size=I)
    cfg._experts_implementation = pkg.experts.register()
    with torch.device(dev):
        blk = Qwen3_5MoeSparseMoeBlock(cfg).to(BF16)
    g = torch.Generator(device=dev).manual_seed(91)
    with torch.no_grad():
        for p in blk.parameters():
            p.copy_(torch.randn(p.shape, generator=g, device=dev) * 0.02)
    w = {"router": blk.gate.weight.detach(), "gate_up": blk.experts.gate_up_proj.detach(),
         "down": blk.experts.down_proj.detach(),
         "sh_gate": blk.shared_expert.gate_proj.weight.detach(),
         "sh_up": blk.shared_expert.up_proj.weight.detach(),
         "sh_down": blk.shared_expert.down_proj.weight.detach(),
         "sh_gate_w": blk.shared_expert_gate.weight.detach()}
    return blk, w


@pytest.mark.parametrize("T", [1, 17, 300])
def test_registered_experts_inside_transformers_block(pkg, dev, tf_block, T):
    """blk(x) with the registered implementation == the oracle's block on the routing the
    block's own router (torch on the GPU) chose, within the bf16 bar."""
    blk, w = tf_block
    assert blk.experts.config._experts_implementation == pkg.experts.NAME
    g = torch.Generator().manual_seed(300 + T)
    x = torch.randn(T, H, generator=g).to(BF16)
    with torch.no_grad():
        out = blk(x.to(dev)[None])
        out = (out[0] if isinstance(out, tuple) else out).reshape(T, H)
        _, wts, idx = blk.gate(x.to(dev))
    torch.cuda.synchronize()
    wc, ic = orc.compact_experts(w, idx.cpu())
    # the routed experts through Transformers' batched_mm rounding up to 16 tokens and the
    # padded / sorted rounding above (engine/experts.py:93-102)
    ref = orc.block_bf16_routed(x, wc, ic, wts.cpu(), None, decode=T <= 16)
    f32 = orc.block_fp32(x, w, idx.cpu(), logits=torch.nn.functional.linear(x, w["router"].cpu()))
    ours, theirs = mean_rel(out, f32), mean_rel(ref, f32)
    _say(f"transformers block T={T}: vs reference path max {max_abs(out, ref):.3g}; vs fp32 "
         f"max {max_abs(out, f32):.3g} mean-rel {ours:.3g} (reference path {theirs:.3g})")
    assert max_abs(out, ref) <= 2e-2 and max_abs(out, f32) <= 2e-2
    assert ours <= max(5e-3, 1.1 * theirs)


@pytest.mark.parametrize("T", [1, 17, 300])
def test_block_surface_on_transformers_module(pkg, dev, tf_block, T):
    """block.moe(x, blk, k) on the Transformers module itself (not an attribute tree):
    routing bit-exact given the logits, values against the fp32 oracle."""
    blk, w = tf_block
    g = torch.Generator().manual_seed(400 + T)
    x = torch.randn(T, H, generator=g).to(BF16)
    out, idx, wts, logits = pkg.block.moe(x.to(dev), blk, K, return_routing=True)
    torch.cuda.synchronize()
    lg = logits.cpu()[:, :E]
    ref_w, ref_i = orc.route(lg, K)
    assert torch.equal(idx.cpu(), ref_i) and torch.equal(wts.cpu(), ref_w)
    f32 = orc.block_fp32(x, w, ref_i, logits=lg)
    wc, ic = orc.compact_experts(w, ref_i)
    ref = orc.block_bf16_routed(x, wc, ic, wts.cpu(), logits.cpu()[:, E:E + 1], decode=T <= 16)
    ours, theirs = mean_rel(out, f32), mean_rel(ref, f32)
    _say(f"block.moe on the transformers module T={T}: max {max_abs(out, f32):.3g} "
         f"mean-rel {ours:.3g} (reference path {theirs:.3g})")
    assert max_abs(out, f32) <= 2e-2 and max_abs(out, ref) <= 2e-2
    assert ours <= max(5e-3, 1.1 * theirs)
