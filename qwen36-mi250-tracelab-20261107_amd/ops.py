"""Operator-level Python surface of the MI355X MoE kernels.

Each function mirrors one operation of the reference engine's MoE path, with the same
argument meaning, and launches the hand-written gfx950 kernels of libmoe_mi355x.so on
the current HIP stream of its inputs' device. Outputs are new tensors from torch's
caching allocator; weights are read in place. Nothing here synchronises with the host.

  router_logits      router | shared-gate GEMV/GEMM     (engine/fast/fused.py:745-746, mfma.py:90)
  route              softmax / top-k / renormalise      (engine/fast/prefill_kernels.py:650-663)
  sort_pairs         counts / stable order / tiles      (engine/fast/moe_prefill.py:509-521,562-566)
  grouped_gate_up    expert gate_up + SwiGLU            (engine/fast/moe_prefill.py:156-211)
  grouped_down       expert down at each pair's row     (engine/fast/moe_prefill.py:212-257)
  combine            weighted sum + gated shared expert (engine/fast/prefill_kernels.py:253-273)
  moe_decode         routed experts, batched_mm rounding (engine/fast/kernels.py:171-217)
  moe_prefill        routed experts, fp32 weighting      (engine/fast/moe_prefill.py:546-582)
  decode_router      router | shared gate_up, T <= 4    (engine/fast/fused.py:745-746, 798-840)
  decode_gate_up     top-k + routed gate_up, T <= 4      (engine/fast/fused.py:554-632)
  decode_down        down + combine + shared, T <= 4     (engine/fast/fused.py:635-692)
  add_rms            residual add + RMSNorm              (engine/fast/kernels.py:636-650)
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from ._lib import check, ptr, stream_of

FP8 = torch.float8_e4m3fn


@dataclass
class SortedPairs:
    """The grouped-GEMM bookkeeping of one routing (all device tensors)."""

    counts: torch.Tensor  # [E] int32 pairs per expert
    offsets: torch.Tensor  # [E] int32 first sorted row per expert (exclusive cumsum)
    order: torch.Tensor  # [T*k] int32 sorted row -> pair (stable argsort of the ids)
    table: torch.Tensor  # [3*max_tiles + 1] int32 tile table
    max_tiles: int
    bm: int


def _need_cuda(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise _lib.MoeLibraryError(
                "the MI355X MoE kernels run on a HIP device only (got a tensor on "
                f"{t.device}); there is no CPU path"
            )


def _bf16(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16 (got {t.dtype})")
    return t.contiguous()


def expert_weight(w: torch.Tensor, scale: torch.Tensor | None, name: str):
    """(tensor, scale or None, weight dtype code) for bf16 or fp8-e4m3 expert weights."""
    if w.dtype == torch.bfloat16:
        if scale is not None:
            raise ValueError(f"{name}: bf16 weights take no scale")
        return w, None, _lib.WEIGHTS_BF16
    if w.dtype == FP8:
        if scale is None or scale.dtype != torch.float32:
            raise ValueError(f"{name}: fp8 weights need fp32 per-row scales")
        if scale.shape != w.shape[:-1]:
            raise ValueError(f"{name}: scale shape {tuple(scale.shape)} != {tuple(w.shape[:-1])}")
        return w, scale.contiguous(), _lib.WEIGHTS_FP8_E4M3
    raise ValueError(f"{name} must be bfloat16 or float8_e4m3fn (got {w.dtype})")


def _check_row_major(*ws: torch.Tensor) -> None:
    for w in ws:
        if not w.is_contiguous():
            raise ValueError("expert weights must be contiguous row-major")


def supported(x: torch.Tensor, gate_up: torch.Tensor, down: torch.Tensor) -> bool:
    """Shapes and layouts the kernels handle (engine/fast/moe_prefill.py:529-543 plays the
    same role): bf16 activations, bf16 or fp8 row-major experts, hidden and intermediate
    multiples of 32, at most 1024 experts."""
    if x.dtype != torch.bfloat16 or x.device.type != "cuda":
        return False
    if gate_up.dim() != 3 or down.dim() != 3:
        return False
    experts, two_i, hidden = gate_up.shape
    inter = two_i // 2
    return (
        gate_up.dtype in (torch.bfloat16, FP8)
        and down.dtype == gate_up.dtype
        and down.shape == (experts, hidden, inter)
        and gate_up.is_contiguous()
        and down.is_contiguous()
        and hidden % 32 == 0
        and inter % 32 == 0
        and 1 <= experts <= 1024
    )


def router_logits(x: torch.Tensor, w_pack: torch.Tensor) -> torch.Tensor:
    """``bf16(x @ w_pack.T)`` [T, n_pack] for the packed router | shared-gate weight."""
    _need_cuda(x, w_pack)
    x = _bf16(x, "x")
    w_pack = _bf16(w_pack, "w_pack")
    tokens, hidden = x.shape
    n_pack = w_pack.shape[0]
    out = torch.empty((tokens, n_pack), dtype=torch.bfloat16, device=x.device)
    lib = _lib.load()
    check(lib.moe_router_logits(ptr(x), tokens, hidden, ptr(w_pack), n_pack, ptr(out), stream_of(x)),
          "router_logits")
    return out


def route(logits: torch.Tensor, top_k: int, experts: int | None = None):
    """(top_w bf16 [T, k], top_i int64 [T, k], per-expert pair counts int32 [E]) of
    softmax_fp32(logits) -> top-k (ties to the lower expert) -> renormalised, as
    engine/fast/prefill_kernels.py:650-663. ``experts`` defaults to logits' width."""
    _need_cuda(logits)
    logits = _bf16(logits, "logits") if logits.stride(-1) != 1 else logits
    if logits.dtype != torch.bfloat16:
        raise ValueError("logits must be bfloat16")
    tokens = logits.shape[0]
    experts = logits.shape[1] if experts is None else experts
    top_w = torch.empty((tokens, top_k), dtype=torch.bfloat16, device=logits.device)
    top_i = torch.empty((tokens, top_k), dtype=torch.long, device=logits.device)
    counts = torch.zeros(experts, dtype=torch.int32, device=logits.device)
    lib = _lib.load()
    check(lib.moe_route_topk(ptr(logits), logits.stride(0), tokens, experts, top_k, ptr(top_i),
                             ptr(top_w), ptr(counts), stream_of(logits)), "route")
    return top_w, top_i, counts


def sort_pairs(top_k_index: torch.Tensor, experts: int, bm: int | None = None,
               shared: bool = False) -> SortedPairs:
    """Per-expert counts, exclusive offsets, the stable sorted order of the flattened pair
    ids (== torch.argsort(ids, stable=True)) and the BM-row tile table."""
    _need_cuda(top_k_index)
    if top_k_index.dtype != torch.long:
        raise ValueError("top_k_index must be int64")
    idx = top_k_index.contiguous()
    tokens, top_k = idx.shape
    lib = _lib.load()
    bm = lib.moe_tile_rows(tokens) if bm is None else bm
    max_tiles = lib.moe_max_tiles(tokens, top_k, experts, bm, int(shared))
    dev = idx.device
    counts = torch.empty(experts, dtype=torch.int32, device=dev)
    offsets = torch.empty(experts, dtype=torch.int32, device=dev)
    order = torch.empty(tokens * top_k, dtype=torch.int32, device=dev)
    table = torch.empty(3 * max_tiles + 1, dtype=torch.int32, device=dev)
    nscratch = lib.moe_sort_scratch_bytes(tokens * top_k, experts)
    scratch = torch.empty(max(nscratch, 1), dtype=torch.uint8, device=dev)
    check(lib.moe_sort(ptr(idx), tokens, top_k, experts, bm, int(shared), ptr(counts), ptr(offsets),
                       ptr(order), ptr(table), max_tiles, ptr(scratch), stream_of(idx)), "sort_pairs")
    return SortedPairs(counts, offsets, order, table, max_tiles, bm)


def grouped_gate_up(x: torch.Tensor, top_k: int, gate_up: torch.Tensor, sp: SortedPairs,
                    scale: torch.Tensor | None = None, shared=None):
    """act [T*k, I] in sorted-row order: bf16(bf16(silu(bf16 g)) * bf16 u).
    ``shared`` = (gate_proj.weight, up_proj.weight) of the shared expert (the table must
    be built with ``shared=True``): returns (act, act_shared [T, IS]) from one launch."""
    _need_cuda(x, gate_up)
    x = _bf16(x, "x")
    w, s, wd = expert_weight(gate_up, scale, "gate_up")
    _check_row_major(w)
    tokens, hidden = x.shape
    experts, two_i, _ = w.shape
    inter = two_i // 2
    act = torch.empty((tokens * top_k, inter), dtype=torch.bfloat16, device=x.device)
    sg = su = act_sh = None
    inter_s = 0
    if shared is not None:
        sg, su = (_bf16(t, "shared weight") for t in shared)
        inter_s = sg.shape[0]
        act_sh = torch.empty((tokens, inter_s), dtype=torch.bfloat16, device=x.device)
    lib = _lib.load()
    check(lib.moe_grouped_gate_up(ptr(x), tokens, hidden, experts, top_k, inter, ptr(w), ptr(s), wd,
                                  ptr(sp.order), ptr(sp.table), sp.max_tiles, sp.bm, ptr(act),
                                  ptr(sg), ptr(su), inter_s, ptr(act_sh), stream_of(x)),
          "grouped_gate_up")
    return act if shared is None else (act, act_sh)


def grouped_down(act: torch.Tensor, tokens: int, top_k: int, down: torch.Tensor, sp: SortedPairs,
                 scale: torch.Tensor | None = None, shared=None):
    """y [T*k, H]: bf16(act[r] . Wd[e]) written at pair order[r]'s own row.
    ``shared`` = (down_proj.weight, act_shared): returns (y, y_shared [T, H])."""
    _need_cuda(act, down)
    act = _bf16(act, "act")
    w, s, wd = expert_weight(down, scale, "down")
    _check_row_major(w)
    experts, hidden, inter = w.shape
    y = torch.empty((tokens * top_k, hidden), dtype=torch.bfloat16, device=act.device)
    sd = act_sh = y_sh = None
    inter_s = 0
    if shared is not None:
        sd, act_sh = _bf16(shared[0], "shared down"), _bf16(shared[1], "act_shared")
        inter_s = sd.shape[1]
        y_sh = torch.empty((tokens, hidden), dtype=torch.bfloat16, device=act.device)
    lib = _lib.load()
    check(lib.moe_grouped_down(ptr(act), tokens, hidden, experts, top_k, inter, ptr(w), ptr(s), wd,
                               ptr(sp.order), ptr(sp.table), sp.max_tiles, sp.bm, ptr(y),
                               ptr(sd), inter_s, ptr(act_sh), ptr(y_sh), stream_of(act)),
          "grouped_down")
    return y if shared is None else (y, y_sh)


def combine(y: torch.Tensor, top_w: torch.Tensor, shared: torch.Tensor | None = None,
            shared_gate_logit: torch.Tensor | None = None, residual: torch.Tensor | None = None,
            round_products: bool = False) -> torch.Tensor:
    """out [T, H] = bf16(sum_j w y) (+ bf16(bf16(sigmoid(g)) * shared)) (+ residual).
    ``round_products`` rounds each w * y to bf16 before the fp32 sum (batched_mm)."""
    _need_cuda(y, top_w)
    tokens, top_k = top_w.shape
    hidden = y.shape[-1]
    y = _bf16(y, "y")
    top_w = _bf16(top_w, "top_w")
    if shared is not None:
        shared = _bf16(shared, "shared")
        if shared_gate_logit is None:
            raise ValueError("shared output needs the shared-expert gate logits")
        if shared_gate_logit.dtype != torch.bfloat16:
            raise ValueError("shared_gate_logit must be bfloat16")
    if residual is not None:
        residual = _bf16(residual, "residual")
    out = torch.empty((tokens, hidden), dtype=torch.bfloat16, device=y.device)
    ld_seg = shared_gate_logit.stride(0) if shared_gate_logit is not None else 0
    mode = _lib.ROUND_PRODUCT if round_products else _lib.EXACT_PRODUCT
    lib = _lib.load()
    check(lib.moe_combine(ptr(y), ptr(top_w), tokens, hidden, top_k, ptr(shared),
                          ptr(shared_gate_logit), ld_seg, ptr(residual), ptr(out), mode,
                          stream_of(y)), "combine")
    return out


def experts(x: torch.Tensor, top_k_index: torch.Tensor, top_k_weights: torch.Tensor,
            gate_up: torch.Tensor, down: torch.Tensor, *, round_products: bool,
            gate_up_scale: torch.Tensor | None = None,
            down_scale: torch.Tensor | None = None) -> torch.Tensor:
    """Routed-expert output [T, H] (no shared expert): sort, grouped gate_up, grouped down
    and combine in one C-ABI call."""
    _need_cuda(x, top_k_index, top_k_weights, gate_up, down)
    x = _bf16(x, "x")
    if top_k_index.dtype != torch.long:
        top_k_index = top_k_index.long()
    idx = top_k_index.contiguous()
    wts = top_k_weights.to(torch.bfloat16).contiguous()
    gu, gus, wd = expert_weight(gate_up, gate_up_scale, "gate_up")
    dn, dns, wd2 = expert_weight(down, down_scale, "down")
    if wd != wd2:
        raise ValueError("gate_up and down must share one weight dtype")
    _check_row_major(gu, dn)
    tokens, hidden = x.shape
    top_k = idx.shape[1]
    nexp, two_i, _ = gu.shape
    inter = two_i // 2
    if dn.shape != (nexp, hidden, inter):
        raise ValueError(f"down shape {tuple(dn.shape)} != {(nexp, hidden, inter)}")
    out = torch.empty((tokens, hidden), dtype=torch.bfloat16, device=x.device)
    if tokens == 0:
        return out
    lib = _lib.load()
    nbytes = lib.moe_experts_workspace_bytes(tokens, hidden, nexp, top_k, inter)
    ws = _lib.workspace(x.device, nbytes)
    mode = _lib.ROUND_PRODUCT if round_products else _lib.EXACT_PRODUCT
    check(lib.moe_experts_forward(ptr(x), tokens, hidden, nexp, top_k, inter, ptr(idx), ptr(wts),
                                  ptr(gu), ptr(gus), ptr(dn), ptr(dns), wd, mode, ptr(out), ptr(ws),
                                  ws.numel(), stream_of(x)), "experts")
    return out


def moe_decode(x, top_k_index, top_k_weights, gate_up, down, **scales) -> torch.Tensor:
    """Routed experts with Transformers batched_mm rounding (engine/fast/kernels.py:171):
    each w * y rounded to bf16 before the fp32 sum."""
    return experts(x, top_k_index, top_k_weights, gate_up, down, round_products=True, **scales)


def moe_prefill(x, top_k_index, top_k_weights, gate_up, down, **scales) -> torch.Tensor:
    """Routed experts with the grouped / padded rounding (engine/fast/moe_prefill.py:546):
    w * y exact in fp32, summed in fp32, rounded once."""
    return experts(x, top_k_index, top_k_weights, gate_up, down, round_products=False, **scales)


# ----------------------------------------------------------------- decode stages (T <= 4)


def decode_fits(tokens: int, hidden: int, experts: int, top_k: int, inter: int,
                inter_shared: int = 0) -> bool:
    """Whether a shape takes the three-launch decode path."""
    return bool(_lib.load().moe_decode_fits(tokens, hidden, experts, top_k, inter, inter_shared))


def decode_router(x: torch.Tensor, w_pack: torch.Tensor, shared: tuple | None = None):
    """(logits [T, n_pack], act_sh [T, IS] or None): the router rows and, with
    ``shared=(sh_gate, sh_up)``, the shared expert's SwiGLU in the same launch."""
    _need_cuda(x, w_pack)
    x = _bf16(x, "x")
    w_pack = _bf16(w_pack, "w_pack")
    tokens, hidden = x.shape
    n_pack = w_pack.shape[0]
    logits = torch.empty((tokens, n_pack), dtype=torch.bfloat16, device=x.device)
    sg = su = act_sh = None
    inter_s = 0
    if shared is not None:
        sg, su = (_bf16(w, "shared weight") for w in shared)
        inter_s = sg.shape[0]
        act_sh = torch.empty((tokens, inter_s), dtype=torch.bfloat16, device=x.device)
    check(_lib.load().moe_decode_router(ptr(x), tokens, hidden, ptr(w_pack), n_pack, ptr(sg),
                                        ptr(su), inter_s, ptr(logits), ptr(act_sh),
                                        stream_of(x)), "decode_router")
    return logits, act_sh


def decode_gate_up(x: torch.Tensor, gate_up: torch.Tensor, top_k: int, *, logits=None,
                   experts: int | None = None, top_k_index=None, scale=None, shared=None):
    """(act [T*k, I], idx32 [T, k], top_k_weights [T, k] bf16 or None, top_k_index int64
    or None). With ``logits`` the routing (softmax / top-k over the first ``experts``
    columns) runs inside the launch; else ``top_k_index`` gives it. With
    ``shared=(gate_proj.weight, up_proj.weight)`` the launch also computes the shared
    expert's activation, returned as a fifth item act_shared [T, IS]."""
    _need_cuda(x, gate_up)
    x = _bf16(x, "x")
    gu, gus, wd = expert_weight(gate_up, scale, "gate_up")
    e_all, two_i, hidden = gu.shape
    experts = e_all if experts is None else experts
    tokens = x.shape[0]
    dev = x.device
    idx32 = torch.empty((tokens, top_k), dtype=torch.int32, device=dev)
    act = torch.empty((tokens * top_k, two_i // 2), dtype=torch.bfloat16, device=dev)
    wts = idx64 = idx_in = None
    n_pack = 0
    if logits is not None:
        logits = _bf16(logits, "logits")
        n_pack = logits.shape[1]
        wts = torch.empty((tokens, top_k), dtype=torch.bfloat16, device=dev)
        idx64 = torch.empty((tokens, top_k), dtype=torch.long, device=dev)
    else:
        if top_k_index is None:
            raise ValueError("decode_gate_up needs logits or top_k_index")
        idx_in = top_k_index.to(torch.long).contiguous()
    sg = su = act_sh = None
    inter_s = 0
    if shared is not None:
        sg, su = (_bf16(t, "shared weight") for t in shared)
        inter_s = sg.shape[0]
        act_sh = torch.empty((tokens, inter_s), dtype=torch.bfloat16, device=dev)
    check(_lib.load().moe_decode_gate_up(ptr(x), tokens, hidden, experts, top_k, two_i // 2,
                                         ptr(logits), n_pack, ptr(idx_in), ptr(gu), ptr(gus), wd,
                                         ptr(idx32), ptr(wts), ptr(idx64), ptr(act), ptr(sg),
                                         ptr(su), inter_s, ptr(act_sh), stream_of(x)),
          "decode_gate_up")
    if shared is not None:
        return act, idx32, wts, idx64, act_sh
    return act, idx32, wts, idx64


def decode_down(act: torch.Tensor, tokens: int, top_k: int, down: torch.Tensor,
                idx32: torch.Tensor, top_k_weights: torch.Tensor, *, round_products: bool = True,
                scale=None, shared: tuple | None = None, logits=None, experts: int | None = None,
                residual=None) -> torch.Tensor:
    """out [T, H]: the routed down projections combined in routing order, plus (with
    ``shared=(sh_down, act_sh)`` and the logits holding the shared-gate logit at column
    ``experts``) the gated shared expert, plus ``residual``."""
    _need_cuda(act, down, idx32, top_k_weights)
    act = _bf16(act, "act")
    dn, dns, wd = expert_weight(down, scale, "down")
    e_all, hidden, inter = dn.shape
    experts = e_all if experts is None else experts
    wts = _bf16(top_k_weights, "top_k_weights")
    idx32 = idx32.to(torch.int32).contiguous()
    sd = act_sh = None
    inter_s = n_pack = 0
    if shared is not None:
        sd, act_sh = (_bf16(t, "shared") for t in shared)
        inter_s = sd.shape[1]
        logits = _bf16(logits, "logits")
        n_pack = logits.shape[1]
    if residual is not None:
        residual = _bf16(residual, "residual")
    out = torch.empty((tokens, hidden), dtype=torch.bfloat16, device=act.device)
    mode = _lib.ROUND_PRODUCT if round_products else _lib.EXACT_PRODUCT
    check(_lib.load().moe_decode_down(ptr(act), tokens, hidden, experts, top_k, inter, ptr(idx32),
                                      ptr(wts), ptr(dn), ptr(dns), wd, ptr(sd), inter_s,
                                      ptr(act_sh), ptr(logits), n_pack, ptr(residual), mode,
                                      ptr(out), stream_of(act)), "decode_down")
    return out


def add_rms(x: torch.Tensor, h: torch.Tensor | None, weight: torch.Tensor, eps: float):
    """``(x + h, RMSNorm(x + h) * (1 + weight))`` in one launch; ``h`` None skips the add and
    returns ``x`` as the first value. Same arguments and results as the reference's
    ``kernels.add_rms`` (engine/fast/kernels.py:636-650): total = bf16(x + h),
    out = bf16(total * rsqrt(mean(total^2) + eps) * (1 + weight)) with fp32 in between."""
    _need_cuda(x, h, weight)
    x2 = _bf16(x, "x").reshape(-1, x.shape[-1])
    rows, n = x2.shape
    h2 = None if h is None else _bf16(h, "h").reshape(rows, n)
    w = _bf16(weight, "weight").reshape(-1)
    if w.numel() != n:
        raise ValueError(f"weight must have {n} elements (got {w.numel()})")
    out = torch.empty_like(x2)
    total = torch.empty_like(x2) if h2 is not None else x2
    check(_lib.load().moe_add_rmsnorm(ptr(x2), ptr(h2), ptr(w), rows, n, float(eps),
                                      ptr(total) if h2 is not None else None, ptr(out),
                                      stream_of(x2)), "add_rms")
    return total.reshape(x.shape), out.reshape(x.shape)
