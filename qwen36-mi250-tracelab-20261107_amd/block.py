"""Block-level MoE (router + top-k + routed experts + gated shared expert) on MI355X.

``moe(x, mlp, top_k)`` has the call surface of the reference's block-level MoE
(``FastModel._moe`` engine/fast/model.py:1139-1179, ``prefill_kernels.moe``
engine/fast/prefill_kernels.py:676-742): ``mlp`` is a Transformers
``Qwen3_5MoeSparseMoeBlock`` (or any object with the same attributes: ``gate.weight``,
``shared_expert.{gate,up,down}_proj.weight``, ``shared_expert_gate.weight``,
``experts.{gate_up_proj,down_proj}``) and the result is the block's output [T, H].
``moe(x, mlp, top_k, residual=r)`` returns ``r + MoE(x)`` rounded as
``FusedDecode._moe`` (engine/fast/fused.py:887-932). ``add_rms_moe(x, h, w, eps, mlp,
top_k)`` puts the layer's post-attention add + RMSNorm in front (``moe_block_forward_add_rms``).

Everything runs in one C-ABI call (``moe_block_forward``): router GEMV/GEMM, softmax /
top-k, count + stable sort + tile table, grouped gate_up (routed experts and the shared
expert in one launch), grouped down, combine. Rounding of the routing-weight products
follows ``FastModel._moe``: bf16(w * y) for decode steps and for at most
``DECODE_EXPERT_TOKENS`` tokens (the batched_mm path), exact fp32 products above.

fp8-e4m3 experts: ``experts.gate_up_proj`` / ``down_proj`` of dtype float8_e4m3fn with
per-output-row fp32 scales in ``experts.gate_up_scale`` [E, 2I] / ``experts.down_scale``
[E, H] (see ``fp8.quantize_experts``).
"""

from __future__ import annotations

import torch

from . import _lib
from ._lib import check, ptr, stream_of
from .ops import _need_cuda, expert_weight

DECODE_EXPERT_TOKENS = 16  # engine/fast/model.py:48

_PACK_ATTR = "_mi355x_router_pack"


def pack_router(mlp) -> torch.Tensor:
    """The router rows and the shared-expert gate row as one [n_pack, H] bf16 tensor
    (rows 0..E-1 router, row E shared gate, zero rows up to a multiple of 64), built once
    per block and cached on it (the packing engine/fast/fused.py:699-746 does for its
    router|shared GEMV). Rebuilt when either source weight changes."""
    router = mlp.gate.weight
    seg = mlp.shared_expert_gate.weight
    key = (router.data_ptr(), router._version, seg.data_ptr(), seg._version, router.device)
    cached = getattr(mlp, _PACK_ATTR, None)
    if cached is not None and cached[0] == key:
        return cached[1]
    experts, hidden = router.shape
    n_pack = (experts + 1 + 63) // 64 * 64
    pack = torch.zeros((n_pack, hidden), dtype=torch.bfloat16, device=router.device)
    with torch.no_grad():
        pack[:experts].copy_(router)
        pack[experts].copy_(seg.reshape(-1))
    setattr(mlp, _PACK_ATTR, (key, pack))
    return pack


def _expert_tensors(experts):
    gu = experts.gate_up_proj
    dn = experts.down_proj
    gus = getattr(experts, "gate_up_scale", None)
    dns = getattr(experts, "down_scale", None)
    gu, gus, wd = expert_weight(gu.data if isinstance(gu, torch.nn.Parameter) else gu, gus, "gate_up")
    dn, dns, wd2 = expert_weight(dn.data if isinstance(dn, torch.nn.Parameter) else dn, dns, "down")
    if wd != wd2:
        raise ValueError("gate_up_proj and down_proj must share one weight dtype")
    if not (gu.is_contiguous() and dn.is_contiguous()):
        raise ValueError("expert weights must be contiguous row-major")
    return gu, gus, dn, dns, wd


def supported(x: torch.Tensor, mlp, top_k: int) -> bool:
    """Whether ``moe`` runs this block (engine/fast/prefill_kernels.py:666-673's role)."""
    try:
        gu, _, dn, _, _ = _expert_tensors(mlp.experts)
    except ValueError:
        return False
    e, two_i, h = gu.shape
    inter_s = mlp.shared_expert.gate_proj.weight.shape[0]
    return (
        x.dtype == torch.bfloat16
        and x.device.type == "cuda"
        and h % 32 == 0
        and (two_i // 2) % 32 == 0
        and inter_s % 32 == 0
        and 1 <= top_k <= min(64, e)
        and e <= 1024
    )


def moe(x: torch.Tensor, mlp, top_k: int, decode: bool = False,
        residual: torch.Tensor | None = None, *, return_routing: bool = False):
    """MoE(x) [T, H] bf16 for ``x`` [T, H] (or residual + MoE(x)). With ``return_routing``
    also (top_k_index int64 [T, k], top_k_weights bf16 [T, k], router logits [T, n_pack])."""
    shape = x.shape
    x2 = _bf16_rows(x, "x")
    if residual is not None:
        residual = residual.reshape(x2.shape).to(torch.bfloat16).contiguous()
    res = _run(x2, mlp, top_k, decode, return_routing, residual=residual)
    out = res[0].reshape(shape)
    return (out, *res[1:]) if return_routing else out


def add_rms_moe(x: torch.Tensor, h: torch.Tensor | None, norm_weight: torch.Tensor, eps: float,
                mlp, top_k: int, decode: bool = False, *, return_norm: bool = False,
                return_routing: bool = False):
    """``total + MoE(norm)`` with ``(total, norm) = add_rms(x, h, norm_weight, eps)``: the
    post-attention add + RMSNorm and the MoE block of one decoder layer, as
    ``x, h = kernels.add_rms(x, h, post_attention_layernorm.weight, eps)`` then the block
    with ``x`` as its residual (engine/fast/model.py:888-891, fused.py:1074-1076). ``h``
    None: no add (``total`` is ``x``). On the decode path the norm runs inside the router
    launch. With ``return_norm`` also (total, norm); with ``return_routing`` also the
    routing, as ``moe``."""
    shape = x.shape
    x2 = _bf16_rows(x, "x")
    h2 = None if h is None else _bf16_rows(h, "h").reshape(x2.shape)
    w = norm_weight.reshape(-1)
    if w.dtype != torch.bfloat16 or w.numel() != x2.shape[1]:
        raise ValueError(f"norm_weight must be bfloat16 [{x2.shape[1]}]")
    w = w.contiguous()
    total = torch.empty_like(x2) if h2 is not None else x2
    norm = torch.empty_like(x2)
    res = _run(x2, mlp, top_k, decode, return_routing,
               norm=(x2, h2, w, float(eps), total if h2 is not None else None, norm))
    out = res[0].reshape(shape)
    extra = (total.reshape(shape), norm.reshape(shape)) if return_norm else ()
    if return_norm or return_routing:
        return (out, *extra, *res[1:])
    return out


def _bf16_rows(t: torch.Tensor, name: str) -> torch.Tensor:
    t2 = t.reshape(-1, t.shape[-1])
    _need_cuda(t2)
    if t2.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16 (got {t2.dtype})")
    return t2.contiguous()


def _run(x2, mlp, top_k, decode, return_routing, residual=None, norm=None):
    tokens, hidden = x2.shape
    gu, gus, dn, dns, wd = _expert_tensors(mlp.experts)
    experts, two_i, _ = gu.shape
    inter = two_i // 2
    sh = mlp.shared_expert
    sg = sh.gate_proj.weight
    su = sh.up_proj.weight
    sd = sh.down_proj.weight
    inter_s = sg.shape[0]
    for w, name in ((sg, "shared gate"), (su, "shared up"), (sd, "shared down")):
        if w.dtype != torch.bfloat16 or not w.is_contiguous():
            raise ValueError(f"{name} weight must be contiguous bfloat16")
    pack = pack_router(mlp)
    n_pack = pack.shape[0]
    round_products = decode or tokens <= DECODE_EXPERT_TOKENS
    mode = _lib.ROUND_PRODUCT if round_products else _lib.EXACT_PRODUCT
    dev = x2.device
    out = torch.empty((tokens, hidden), dtype=torch.bfloat16, device=dev)
    idx = torch.empty((tokens, top_k), dtype=torch.long, device=dev) if return_routing else None
    wts = torch.empty((tokens, top_k), dtype=torch.bfloat16, device=dev) if return_routing else None
    logits = (torch.empty((tokens, n_pack), dtype=torch.bfloat16, device=dev)
              if return_routing else None)
    if tokens:
        lib = _lib.load()
        nbytes = lib.moe_block_workspace_bytes(tokens, hidden, experts, top_k, inter, inter_s, n_pack)
        ws = _lib.workspace(dev, nbytes)
        block_args = (tokens, hidden, experts, top_k, inter, inter_s, ptr(pack), n_pack, ptr(gu),
                      ptr(gus), ptr(dn), ptr(dns), wd, ptr(sg), ptr(su), ptr(sd))
        tail = (ptr(out), ptr(idx), ptr(wts), ptr(logits), ptr(ws), ws.numel(), stream_of(x2))
        if norm is None:
            check(lib.moe_block_forward(ptr(x2), *block_args, ptr(residual), mode, *tail),
                  "moe block")
        else:
            nx, nh, nw, eps, total, nout = norm
            check(lib.moe_block_forward_add_rms(
                ptr(nx), ptr(nh), ptr(nw), eps, *block_args, mode, ptr(total), ptr(nout), *tail),
                "add_rms + moe block")
    return out, idx, wts, logits
