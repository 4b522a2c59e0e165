"""fp8-e4m3 expert weights: per-output-row quantisation for the MI355X GEMV / GEMM.

The reference has no fp8 path; this is the format the MI355X kernels read. Each output
row n of an expert matrix W [rows, K] gets one fp32 scale s_n = amax(|W_n|) / 448 (448 is
the largest finite e4m3fn value) and q_n = e4m3fn(W_n / s_n) (round to nearest even,
saturating). The kernels convert q to bf16 exactly in registers and apply s_n to the
fp32 accumulator: y_n = s_n * sum_k q_nk x_k.
"""

from __future__ import annotations

import torch

E4M3_MAX = 448.0


def quantize_rows(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(q float8_e4m3fn, scale fp32 [..., rows]) of ``w`` [..., rows, K] per output row."""
    wf = w.float()
    amax = wf.abs().amax(dim=-1)
    scale = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
    q = (wf / scale.unsqueeze(-1)).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    return q.contiguous(), scale.contiguous()


def dequantize_rows(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """fp32 ``scale * q`` (the weight the fp8 kernels multiply by)."""
    return q.float() * scale.unsqueeze(-1)


class Fp8Experts(torch.nn.Module):
    """Experts holder with fp8 weights: ``gate_up_proj`` [E, 2I, H] and ``down_proj``
    [E, H, I] (float8_e4m3fn) with ``gate_up_scale`` [E, 2I] / ``down_scale`` [E, H]."""

    def __init__(self, gate_up: torch.Tensor, down: torch.Tensor):
        super().__init__()
        self.num_experts = gate_up.shape[0]
        q, s = quantize_rows(gate_up)
        self.gate_up_proj, self.gate_up_scale = q, s
        q, s = quantize_rows(down)
        self.down_proj, self.down_scale = q, s
        self.act_fn = torch.nn.functional.silu


def quantize_experts(experts: torch.nn.Module) -> Fp8Experts:
    """An ``Fp8Experts`` from a bf16 experts module (Transformers ``Qwen3_5MoeExperts``)."""
    return Fp8Experts(experts.gate_up_proj.detach(), experts.down_proj.detach())
