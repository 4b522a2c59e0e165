"""The routed-experts implementation registered with Transformers (surface 1).

Same contract as the reference's ``baseline_matmul`` (engine/experts.py:93-108):
``experts_forward(self, hidden_states, top_k_index, top_k_weights)`` returns the routed
experts' combined output [T, H], and ``register()`` adds it to Transformers'
``ExpertsInterface`` so ``from_pretrained(..., experts_implementation=NAME)`` selects it.

Both of the reference's regimes map onto the same gfx950 kernels (stable sort by
expert, expert-deduplicated grouped GEMMs, combine); only the rounding of the routing
weight products differs, as in the reference:
- at most ``BATCHED_TOKENS`` tokens: Transformers' ``batched_mm`` semantics,
  bf16(w * y) summed in fp32 (transformers/integrations/moe.py:112-176);
- above: the padded / sorted semantics, w * y exact in fp32 (engine/experts.py:34-90).
There is no host synchronisation and no per-expert loop at any token count, so
``PADDED_MAX_ROWS``' skew fallback (engine/experts.py:31) has no counterpart.
"""

from __future__ import annotations

import torch

from . import ops

NAME = "mi355x_grouped"
# Up to this many tokens per call the batched_mm rounding applies (engine/experts.py:27).
BATCHED_TOKENS = 16


def experts_forward(
    self: torch.nn.Module,
    hidden_states: torch.Tensor,
    top_k_index: torch.Tensor,
    top_k_weights: torch.Tensor,
) -> torch.Tensor:
    """Routed-expert output for ``hidden_states`` [T, H]; weights read in place.

    ``self`` provides ``gate_up_proj`` [E, 2I, H], ``down_proj`` [E, H, I] (bf16, or
    float8_e4m3fn with ``gate_up_scale`` / ``down_scale`` per-row fp32 scales) and uses
    SiLU gating (the Qwen3.5/3.6 MoE experts)."""
    gu = self.gate_up_proj
    dn = self.down_proj
    return ops.experts(
        hidden_states,
        top_k_index,
        top_k_weights,
        gu.data if isinstance(gu, torch.nn.Parameter) else gu,
        dn.data if isinstance(dn, torch.nn.Parameter) else dn,
        round_products=hidden_states.shape[0] <= BATCHED_TOKENS,
        gate_up_scale=getattr(self, "gate_up_scale", None),
        down_scale=getattr(self, "down_scale", None),
    ).to(hidden_states.dtype)


def register() -> str:
    """Make ``NAME`` a valid ``experts_implementation``; return it (engine/experts.py:105)."""
    from transformers.integrations.moe import ExpertsInterface

    ExpertsInterface.register(NAME, experts_forward)
    return NAME
