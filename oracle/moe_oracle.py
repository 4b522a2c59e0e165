"""CPU oracle of the routed-expert MoE block — TEST INFRASTRUCTURE ONLY.

This module is the checker, never the product: only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import it. It restates, in plain torch (CPU) and numpy,
the reference path the MI355X kernels replace, with each function citing what it follows:

- Transformers ``Qwen3_5MoeSparseMoeBlock`` (installed transformers 5.15; the reference
  pins 5.22.1): modeling_qwen3_5_moe.py:704-800, integrations/moe.py:112-176.
- the engine's experts implementation, /root/reference/engine/experts.py:34-102.
- the engine's grouped-GEMM bookkeeping, engine/fast/moe_prefill.py:92-154,509-582 and its
  tile-table test, tests/test_moe_prefill.py:126-146.
- the post-attention add + RMSNorm, engine/fast/kernels.py:507-523,636-650.
- the routing tie rule of the engine's kernels, engine/fast/fused.py:553-570,
  engine/fast/prefill_kernels.py:194-219 (descending probability, ties to the lower index).

Two modes of the block: ``block_bf16`` rounds where the torch bf16 reference rounds
(F.linear / bmm outputs, activation, products) and is the parity target for values;
``block_fp32`` computes the experts in fp32 from the same routing and is the tolerance
reference the north star names.

How each function is pinned (tests/test_oracle.py): ``route`` by brute force on tie-heavy
rows, explicit tie cases, torch.topk up to ties and float64 renormalisation; ``sort_pairs``
by the closed-form tile table and stable-permutation invariants; ``batched_mm_experts`` bit
for bit against Transformers' batched_mm_experts_forward; ``sorted_experts`` /
``padded_experts`` against each other and Transformers' eager experts loop; ``block_bf16``
bit for bit against Transformers' Qwen3_5MoeSparseMoeBlock; ``block_fp32`` against a
float64 restatement; the e4m3 codec against all 256 encodings of torch's cast; ``add_rms``
bit for bit against Transformers' Qwen3_5MoeRMSNorm, a one-hot closed form, power-of-two
scale invariance and exact integer sums. Nothing here is left parity unpinned.
"""

from __future__ import annotations

import numpy as np
import torch
from torch.nn import functional as F

BF16 = torch.bfloat16


# ------------------------------------------------------------------------------ routing


def softmax_probs(logits: torch.Tensor) -> torch.Tensor:
    """fp32 softmax of bf16 router logits (modeling_qwen3_5_moe.py:770)."""
    return torch.softmax(logits.float(), dim=-1, dtype=torch.float)


def route(logits: torch.Tensor, top_k: int, experts: int | None = None):
    """(top_w bf16 [T,k], top_i int64 [T,k]) with the kernels' tie rule.

    modeling_qwen3_5_moe.py:768-775 computes softmax -> topk -> renormalise -> bf16; the
    engine's kernels (fused.py:560-568, prefill_kernels.py:208-214) break ties to the lower
    expert index, which ``torch.topk`` does not guarantee; a stable descending sort does.
    """
    if experts is not None:
        logits = logits[:, :experts]
    probs = softmax_probs(logits)
    vals, idx = torch.sort(probs, dim=-1, descending=True, stable=True)
    top_p, top_i = vals[:, :top_k], idx[:, :top_k]
    top_w = (top_p / top_p.sum(dim=-1, keepdim=True)).to(BF16)
    return top_w, top_i


def route_bruteforce(logits: torch.Tensor, top_k: int):
    """Pure-Python loops: repeatedly take the largest remaining probability, the lowest
    index among equals. For small inputs only; pins ``route``'s indices."""
    probs = softmax_probs(logits).tolist()
    out = []
    for row in probs:
        taken = set()
        picks = []
        for _ in range(top_k):
            best, best_i = None, None
            for i, p in enumerate(row):
                if i in taken:
                    continue
                if best is None or p > best:
                    best, best_i = p, i
            taken.add(best_i)
            picks.append(best_i)
        out.append(picks)
    return torch.tensor(out, dtype=torch.long)


# -------------------------------------------------------------------------- sort / tiles


def sort_pairs(top_i: torch.Tensor | np.ndarray, experts: int, bm: int, tokens: int | None = None,
               shared: bool = False):
    """(counts, offsets, order, tiles) of the flattened pair ids p = t*k + j.

    counts = bincount (engine/experts.py:72); offsets = exclusive cumsum (:77);
    order = stable argsort (:71); tiles = for each expert e and j < ceil(c_e / bm),
    (e, offsets[e] + j*bm, offsets[e] + c_e), the closed form of
    tests/test_moe_prefill.py:138-146 (the table of moe_prefill.py:92-154); with
    ``shared``, tiles (E, P + j*bm, P + T) follow for the shared expert.
    """
    ids = np.asarray(top_i, dtype=np.int64).reshape(-1)
    counts = np.bincount(ids, minlength=experts).astype(np.int32)
    offsets = (np.cumsum(counts) - counts).astype(np.int32)
    order = np.argsort(ids, kind="stable").astype(np.int32)
    tiles = []
    for e in range(experts):
        c, s = int(counts[e]), int(offsets[e])
        for j in range(-(-c // bm)):
            tiles.append((e, s + j * bm, s + c))
    if shared:
        P = ids.size
        for j in range(-(-tokens // bm)):
            tiles.append((experts, P + j * bm, P + tokens))
    return counts, offsets, order, tiles


def max_tiles(tokens: int, top_k: int, experts: int, bm: int, shared: bool = False) -> int:
    """ceil(P/bm) + min(E, P) (+ ceil(T/bm)): bounds the tile count of any routing."""
    P = tokens * top_k
    return -(-P // bm) + min(experts, P) + (-(-tokens // bm) if shared else 0)


# ------------------------------------------------------------------------------ experts


def batched_mm_experts(x, top_i, top_w, gate_up, down):
    """Transformers ``batched_mm_experts_forward`` (integrations/moe.py:112-176), the
    reference's decode path (engine/experts.py:99-100): gather each pair's expert weights,
    bf16 bmm for gate_up, silu(gate) * up, bf16 bmm for down, times the routing weight
    (bf16 product), fp32 sum over k, bf16."""
    tokens, top_k = top_i.shape
    ids = top_i.reshape(-1).clamp(0, gate_up.shape[0] - 1)
    xs = x.repeat_interleave(top_k, dim=0)
    proj = torch.bmm(gate_up[ids], xs.unsqueeze(-1)).squeeze(-1)
    gate, up = proj.chunk(2, dim=-1)
    hidden = F.silu(gate) * up
    out = torch.bmm(down[ids], hidden.unsqueeze(-1)).squeeze(-1)
    weighted = out * top_w.reshape(-1).unsqueeze(-1)
    return weighted.view(tokens, top_k, -1).sum(dim=1).to(x.dtype)


def sorted_experts(x, top_i, top_w, gate_up, down):
    """engine/experts.py:34-57: tokens sorted by expert, per-expert F.linear, routing
    weight applied in fp32 (exact on bf16 operands), fp32 sum over k, bf16."""
    tokens, top_k = top_i.shape
    ids = top_i.reshape(-1)
    order = torch.argsort(ids, stable=True)
    counts = torch.bincount(ids, minlength=gate_up.shape[0]).tolist()
    inputs = x[order // top_k]
    outputs = torch.empty((inputs.shape[0], down.shape[1]), dtype=x.dtype)
    start = 0
    for expert, count in enumerate(counts):
        if count == 0:
            continue
        rows = slice(start, start + count)
        gate, up = F.linear(inputs[rows], gate_up[expert]).chunk(2, dim=-1)
        outputs[rows] = F.linear(F.silu(gate) * up, down[expert])
        start += count
    weighted = outputs.float() * top_w.reshape(-1)[order, None].float()
    unsorted = torch.empty_like(weighted)
    unsorted[order] = weighted
    return unsorted.view(tokens, top_k, -1).sum(dim=1).to(x.dtype)


def padded_experts(x, top_i, top_w, gate_up, down):
    """engine/experts.py:60-90: one zero-padded bmm per projection over [E, capacity]."""
    tokens, top_k = top_i.shape
    experts = gate_up.shape[0]
    ids = top_i.reshape(-1)
    order = torch.argsort(ids, stable=True)
    counts = torch.bincount(ids, minlength=experts)
    capacity = int(counts.max())
    sorted_ids = ids[order]
    offsets = torch.cumsum(counts, dim=0) - counts
    slot = torch.arange(order.numel()) - offsets[sorted_ids]
    buf = x.new_zeros(experts, capacity, x.shape[-1])
    buf[sorted_ids, slot] = x[order // top_k]
    gate, up = torch.bmm(buf, gate_up.transpose(1, 2)).chunk(2, dim=-1)
    padded = torch.bmm(F.silu(gate) * up, down.transpose(1, 2))
    outputs = padded[sorted_ids, slot]
    weighted = outputs.float() * top_w.reshape(-1)[order, None].float()
    unsorted = torch.empty_like(weighted)
    unsorted[order] = weighted
    return unsorted.view(tokens, top_k, -1).sum(dim=1).to(x.dtype)


BATCHED_TOKENS = 16  # engine/experts.py:27


def experts_forward(x, top_i, top_w, gate_up, down):
    """engine/experts.py:93-102: batched_mm up to 16 tokens, padded above."""
    if x.shape[0] <= BATCHED_TOKENS:
        return batched_mm_experts(x, top_i, top_w, gate_up, down)
    return sorted_experts(x, top_i, top_w, gate_up, down)


def pair_outputs_bf16(x, top_i, gate_up, down):
    """Per-pair bf16 expert outputs y[p] = bf16(W_d . bf16(silu(bf16 g)) * bf16 u) [T*k, H]
    and the per-pair activations act[p] [T*k, I] (pair order, not sorted)."""
    tokens, top_k = top_i.shape
    ids = top_i.reshape(-1)
    xs = x.repeat_interleave(top_k, dim=0)
    act = torch.empty((ids.numel(), down.shape[2]), dtype=x.dtype)
    y = torch.empty((ids.numel(), down.shape[1]), dtype=x.dtype)
    for e in ids.unique().tolist():
        p = (ids == e).nonzero().squeeze(-1)
        gate, up = F.linear(xs[p], gate_up[e]).chunk(2, dim=-1)
        a = F.silu(gate) * up
        act[p] = a
        y[p] = F.linear(a, down[e])
    return act, y


# ------------------------------------------------------------------------------- block


def add_rms(x, h, weight, eps):
    """``kernels.add_rms`` (engine/fast/kernels.py:636-650, math of ``_add_rms_kernel``
    kernels.py:507-523): total = bf16(x + h) (``h`` None: total is x), out =
    bf16(total * rsqrt(mean(total^2) + eps) * (1 + weight)) in fp32, the zero-centred
    RMSNorm of Transformers' Qwen3_5MoeRMSNorm (modeling_qwen3_5_moe.py:801-815) and of
    engine/fast/model.py:75-79. Returns (total, out)."""
    total = x if h is None else x + h
    t = total.float()
    out = t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + eps) * (1.0 + weight.float())
    return total, out.to(x.dtype)


def shared_expert(x, sg, su, sd):
    """Qwen3_5MoeMLP.forward (modeling_qwen3_5_moe.py:715-717) in bf16."""
    return F.linear(F.silu(F.linear(x, sg)) * F.linear(x, su), sd)


DECODE_EXPERT_TOKENS = 16  # engine/fast/model.py:48


def block_bf16(x, w, top_k, decode=False):
    """``FastModel._moe`` (engine/fast/model.py:1139-1179) = Qwen3_5MoeSparseMoeBlock
    (modeling_qwen3_5_moe.py:787-800) with the engine's experts: shared expert, router,
    routed experts (batched_mm rounding for decode / <= 16 tokens, fp32 weighting above),
    sigmoid shared gate, sum. ``w`` is a dict of bf16 CPU tensors (see ``make_weights``).
    Returns (out, top_i, top_w, logits)."""
    shared = shared_expert(x, w["sh_gate"], w["sh_up"], w["sh_down"])
    logits = F.linear(x, w["router"])
    top_w, top_i = route(logits, top_k)
    gu, dn = w["gate_up"], w["down"]
    if decode or x.shape[0] <= DECODE_EXPERT_TOKENS:
        routed = batched_mm_experts(x, top_i, top_w, gu, dn)
    else:
        routed = sorted_experts(x, top_i, top_w, gu, dn)
    gate = torch.sigmoid(F.linear(x, w["sh_gate_w"]))
    out = routed + gate * shared
    return out, top_i, top_w, logits


def block_bf16_routed(x, w, top_i, top_w, logits, decode=False):
    """``block_bf16`` for a given routing (top_i, bf16 top_w) and bf16 router logits
    [T, >E] (column E = the shared-expert gate logit): lets a test feed the GPU's own
    routing and a compacted set of experts."""
    shared = shared_expert(x, w["sh_gate"], w["sh_up"], w["sh_down"])
    gu, dn = w["gate_up"], w["down"]
    if decode or x.shape[0] <= DECODE_EXPERT_TOKENS:
        routed = batched_mm_experts(x, top_i, top_w, gu, dn)
    else:
        routed = sorted_experts(x, top_i, top_w, gu, dn)
    gate = torch.sigmoid(logits[:, -1:]) if logits is not None else torch.sigmoid(
        F.linear(x, w["sh_gate_w"]))
    return routed + gate * shared


def compact_experts(w, top_i):
    """(w', top_i') with only the experts ``top_i`` uses, copied to the CPU, and the
    indices renumbered into them (for checking full-size layers whose experts live on
    the GPU)."""
    uniq = torch.unique(top_i.cpu())
    remap = torch.full((int(uniq.max()) + 1,), -1, dtype=torch.long)
    remap[uniq] = torch.arange(uniq.numel())
    out = {k: (v.cpu() if k not in ("gate_up", "down", "gate_up_scale", "down_scale") else v)
           for k, v in w.items()}
    dev_idx = uniq.to(w["gate_up"].device)
    for k in ("gate_up", "down", "gate_up_scale", "down_scale"):
        if k in w:
            out[k] = w[k][dev_idx].cpu()
    return out, remap[top_i.cpu()]


def block_fp32(x, w, top_i, top_w=None, logits=None):
    """The block in fp32 for a given routing (bit-exact indices are a separate contract):
    every matmul and activation in fp32 from the bf16 weights, renormalised fp32 routing
    weights, no intermediate rounding. The tolerance reference for values. fp8 experts:
    ``w`` also holds ``gate_up_scale`` / ``down_scale`` and the fp32 weight is scale * q.
    Expert tensors may live on any device; each used expert is copied to the CPU."""
    xf = x.float().cpu()
    if logits is None:
        logits = F.linear(x, w["router"])
    if top_w is None or top_w.dtype != torch.float32:
        probs = softmax_probs(logits)
        sel = probs.gather(-1, top_i)
        top_w = sel / sel.sum(dim=-1, keepdim=True)
    gu, dn = w["gate_up"], w["down"]
    gus, dns = w.get("gate_up_scale"), w.get("down_scale")
    tokens, top_k = top_i.shape
    out = torch.zeros((tokens, xf.shape[1]), dtype=torch.float32)
    for e in top_i.unique().tolist():
        t, j = (top_i == e).nonzero(as_tuple=True)
        ge = gu[e].float().cpu()  # per expert: the full tensors may live on the GPU
        de = dn[e].float().cpu()
        if gus is not None:
            ge = ge * gus[e].float().cpu().unsqueeze(-1)
            de = de * dns[e].float().cpu().unsqueeze(-1)
        g, u = F.linear(xf[t], ge).chunk(2, dim=-1)
        y = F.linear(F.silu(g) * u, de)
        out.index_add_(0, t, y * top_w[t, j, None])
    sh = F.linear(F.silu(F.linear(xf, w["sh_gate"].float().cpu())) * F.linear(xf, w["sh_up"].float().cpu()),
                  w["sh_down"].float().cpu())
    gate = torch.sigmoid(F.linear(xf, w["sh_gate_w"].float().cpu()))
    return out + gate * sh


# ----------------------------------------------------------------------------- weights


def make_weights(hidden, experts, inter, inter_s, seed=0, std=0.02, router_std=None):
    """Synthetic bf16 weights ~ N(0, std) in Transformers' layouts (CPU, seeded)."""
    g = torch.Generator().manual_seed(seed)

    def rnd(*shape, s=std):
        return (torch.randn(*shape, generator=g) * s).to(BF16)

    return {
        "router": rnd(experts, hidden, s=router_std or std),
        "gate_up": rnd(experts, 2 * inter, hidden),
        "down": rnd(experts, hidden, inter),
        "sh_gate": rnd(inter_s, hidden),
        "sh_up": rnd(inter_s, hidden),
        "sh_down": rnd(hidden, inter_s),
        "sh_gate_w": rnd(1, hidden),
    }


# -------------------------------------------------------------------------------- fp8


def quantize_rows(w: torch.Tensor):
    """Per-output-row e4m3fn quantisation, s = amax/448, q = e4m3(w/s) (RNE, saturating)."""
    wf = w.float()
    amax = wf.abs().amax(dim=-1)
    scale = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    q = (wf / scale.unsqueeze(-1)).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q, scale


def dequantize_rows(q, scale):
    return q.float() * scale.unsqueeze(-1)


E4M3_TABLE_CHECKS = {
    # (bits, value) pairs of the OCP e4m3fn format: sign 1, exponent 4 (bias 7), mantissa 3.
    0x00: 0.0,
    0x01: 2.0 ** -9,  # smallest subnormal
    0x07: 7 * 2.0 ** -9,  # largest subnormal
    0x08: 2.0 ** -6,  # smallest normal
    0x38: 1.0,
    0x7E: 448.0,  # largest finite
    0xB8: -1.0,
}


def e4m3_decode(byte: int) -> float:
    """Textbook decode of one OCP e4m3fn byte (NaN for S.1111.111)."""
    s = -1.0 if byte & 0x80 else 1.0
    e = (byte >> 3) & 0xF
    m = byte & 0x7
    if e == 0xF and m == 0x7:
        return float("nan")
    if e == 0:
        return s * m * 2.0 ** -9
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
