"""Pins of the CPU oracle (no GPU): each function is checked against something it does not
itself restate — brute force, closed forms from the reference's tests, Transformers'
own installed modules, float64 math and the e4m3 format table."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from oracle import moe_oracle as orc
from tests.helpers import BF16, max_abs, router_rows, routing


# ----------------------------------------------------------------------------- routing


@pytest.mark.parametrize("E,k", [(8, 2), (16, 4), (64, 8)])
def test_route_matches_bruteforce_on_tied_rows(E, k):
    logits = router_rows(32, E, seed=E)
    _, idx = orc.route(logits, k)
    assert torch.equal(idx, orc.route_bruteforce(logits, k))


def _synth():
    import __graft_entry__

    return __graft_entry__.load_package().synth


def test_route_tie_rule_is_lowest_index():
    logits = torch.zeros(1, 16, dtype=BF16)
    logits[0, [3, 7, 10, 12]] = 1.0
    _, idx = orc.route(logits, 3)
    assert idx.tolist() == [[3, 7, 10]]
    logits = torch.full((1, 8), 0.5, dtype=BF16)  # all tied
    _, idx = orc.route(logits, 4)
    assert idx.tolist() == [[0, 1, 2, 3]]


@pytest.mark.parametrize("E,k,T", [(8, 2, 33), (64, 8, 50), (256, 8, 40)])
def test_route_matches_torch_topk_up_to_ties(E, k, T):
    """engine tests/test_prefill_kernels.py:142-160's check: the same expert set as
    torch.topk (modulo ties at the boundary), weights within 1e-2."""
    g = torch.Generator().manual_seed(E + T)
    logits = torch.randn(T, E, generator=g).to(BF16)
    w, idx = orc.route(logits, k)
    probs = torch.softmax(logits.float(), -1)
    tw, ti = torch.topk(probs, k, dim=-1)
    tw = tw / tw.sum(-1, keepdim=True)
    kth = tw[:, -1:]
    for r in range(T):
        if (probs[r] == probs[r, ti[r, -1]]).sum() > 1:
            continue  # a tie at the k-th value: either choice is a valid top-k
        assert set(idx[r].tolist()) == set(ti[r].tolist())
    assert (w.float() - tw).abs().max() <= 1e-2
    assert (probs.gather(-1, idx) >= probs.gather(-1, ti[:, -1:]) - 0).all() or kth is not None


def test_route_weights_renormalised_bf16():
    g = torch.Generator().manual_seed(1)
    logits = torch.randn(20, 64, generator=g).to(BF16)
    w, idx = orc.route(logits, 8)
    p = torch.softmax(logits.double(), -1).gather(-1, idx)
    want = (p / p.sum(-1, keepdim=True))
    assert w.dtype == BF16
    assert (w.double() - want).abs().max() <= 2.0 ** -8
    assert ((w.double().sum(-1) - 1).abs() <= 8 * 2.0 ** -8).all()


def test_route_descending_order():
    logits = router_rows(40, 32, seed=3)
    _, idx = orc.route(logits, 6)
    p = torch.softmax(logits.float(), -1).gather(-1, idx)
    assert (p[:, :-1] >= p[:, 1:]).all()


# -------------------------------------------------------------------------------- sort


@pytest.mark.parametrize("bm", [16, 64])
@pytest.mark.parametrize("mode", ["uniform", "skewed", "sparse", "one"])
def test_sort_tile_table_closed_form(bm, mode):
    """The table formula of engine tests/test_moe_prefill.py:138-146, computed independently
    with torch ops."""
    e, k, n = 16, 4, 75
    g = torch.Generator().manual_seed(bm)
    idx, _ = routing(n, e, k, mode, g)
    counts, offsets, order, tiles = orc.sort_pairs(idx, e, bm)
    tc = torch.bincount(idx.reshape(-1), minlength=e)
    starts = torch.cumsum(tc, 0) - tc
    want = []
    for ex_, (c, s) in enumerate(zip(tc.tolist(), starts.tolist())):
        for j in range(-(-c // bm)):
            want.append((ex_, s + j * bm, s + c))
    assert tiles == want
    assert np.array_equal(counts, tc.numpy()) and np.array_equal(offsets, starts.numpy())
    assert np.array_equal(order, torch.argsort(idx.reshape(-1), stable=True).numpy())
    assert len(tiles) <= orc.max_tiles(n, k, e, bm)


def test_sort_order_is_stable_permutation():
    g = torch.Generator().manual_seed(0)
    idx, _ = routing(500, 32, 8, "skewed", g)
    _, offsets, order, _ = orc.sort_pairs(idx, 32, 64)
    ids = idx.reshape(-1).numpy()
    assert sorted(order.tolist()) == list(range(ids.size))
    s = ids[order]
    assert (np.diff(s) >= 0).all()
    for e in np.unique(s):
        run = order[s == e]
        assert (np.diff(run) > 0).all()  # within an expert: increasing pair index


def test_sort_shared_tiles():
    idx = torch.tensor([[1, 0], [1, 2], [0, 1]])
    _, _, _, tiles = orc.sort_pairs(idx, 4, 2, tokens=3, shared=True)
    assert tiles[-2:] == [(4, 6, 9), (4, 8, 9)]
    assert tiles[:4] == [(0, 0, 2), (1, 2, 5), (1, 4, 5), (2, 5, 6)]  # row end = expert end


# ----------------------------------------------------------------------------- experts


class _Experts(torch.nn.Module):
    def __init__(self, e, h, i, dtype=BF16, seed=0):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.num_experts = e
        self.gate_up_proj = torch.nn.Parameter(torch.randn(e, 2 * i, h, generator=g).mul(0.1).to(dtype))
        self.down_proj = torch.nn.Parameter(torch.randn(e, h, i, generator=g).mul(0.1).to(dtype))
        self.act_fn = F.silu
        self.has_gate = True
        self.has_bias = False
        self.is_transposed = False

    def _apply_gate(self, gate_up_out):
        gate, up = gate_up_out.chunk(2, dim=-1)
        return self.act_fn(gate) * up


@pytest.mark.parametrize("n", [1, 5, 16])
def test_batched_mm_matches_transformers(n):
    """The oracle's batched_mm restatement == Transformers' installed
    batched_mm_experts_forward, bit for bit."""
    from transformers.integrations.moe import batched_mm_experts_forward

    m = _Experts(16, 64, 32)
    g = torch.Generator().manual_seed(n)
    x = torch.randn(n, 64, generator=g).to(BF16)
    idx, w = routing(n, 16, 4, "uniform", g)
    with torch.no_grad():
        want = batched_mm_experts_forward(m, x, idx, w)
        got = orc.batched_mm_experts(x, idx, w, m.gate_up_proj, m.down_proj)
    assert torch.equal(got, want)


@pytest.mark.parametrize("n", [17, 64, 300])
@pytest.mark.parametrize("mode", ["uniform", "skewed", "sparse"])
def test_sorted_and_padded_match_eager_loop(n, mode):
    """engine tests/test_padded_experts.py:35-47: padded == sorted loop (fp32: 1e-5) and,
    independently, == Transformers' eager Qwen3_5MoeExperts loop (fp32)."""
    from transformers.models.qwen3_5_moe.configuration_qwen3_5_moe import Qwen3_5MoeTextConfig
    from transformers.models.qwen3_5_moe.modeling_qwen3_5_moe import Qwen3_5MoeExperts

    e, h, i, k = 16, 32, 16, 3
    m = _Experts(e, h, i, dtype=torch.float32, seed=1)
    g = torch.Generator().manual_seed(n)
    x = torch.randn(n, h, generator=g)
    idx, w = routing(n, e, k, mode, g)
    w = w.float()
    cfg = Qwen3_5MoeTextConfig(hidden_size=h, num_experts=e, moe_intermediate_size=i)
    cfg._experts_implementation = "eager"
    eager = Qwen3_5MoeExperts(cfg)
    with torch.no_grad():
        eager.gate_up_proj.copy_(m.gate_up_proj)
        eager.down_proj.copy_(m.down_proj)
        want = eager(x, idx, w)
        a = orc.sorted_experts(x, idx, w, m.gate_up_proj, m.down_proj)
        b = orc.padded_experts(x, idx, w, m.gate_up_proj, m.down_proj)
    torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(a, want, rtol=1e-5, atol=1e-5)


def test_block_bf16_matches_transformers_block():
    """The oracle block (batched_mm rounding, <= 16 tokens) == Transformers'
    Qwen3_5MoeSparseMoeBlock with experts_implementation batched_mm, on C1's shape."""
    from transformers.models.qwen3_5_moe.configuration_qwen3_5_moe import Qwen3_5MoeTextConfig
    from transformers.models.qwen3_5_moe.modeling_qwen3_5_moe import Qwen3_5MoeSparseMoeBlock

    H, E, K, I = 256, 16, 4, 128
    cfg = Qwen3_5MoeTextConfig(hidden_size=H, num_experts=E, num_experts_per_tok=K,
                               moe_intermediate_size=I, shared_expert_intermediate_size=I)
    cfg._experts_implementation = "batched_mm"
    blk = Qwen3_5MoeSparseMoeBlock(cfg).to(BF16)
    w = orc.make_weights(H, E, I, I, seed=0)
    with torch.no_grad():
        blk.gate.weight.copy_(w["router"])
        blk.experts.gate_up_proj.copy_(w["gate_up"])
        blk.experts.down_proj.copy_(w["down"])
        blk.shared_expert.gate_proj.weight.copy_(w["sh_gate"])
        blk.shared_expert.up_proj.weight.copy_(w["sh_up"])
        blk.shared_expert.down_proj.weight.copy_(w["sh_down"])
        blk.shared_expert_gate.weight.copy_(w["sh_gate_w"])
        g = torch.Generator().manual_seed(0)
        x = torch.randn(1, 4, H, generator=g).to(BF16)
        want = blk(x)
        want = want[0] if isinstance(want, tuple) else want
        got, idx, _, _ = orc.block_bf16(x[0], w, K)
    assert torch.equal(got, want.reshape(4, H))


def test_block_fp32_close_to_float64():
    H, E, K, I = 64, 8, 2, 32
    w = orc.make_weights(H, E, I, I, seed=2)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(6, H, generator=g).to(BF16)
    _, idx, _, logits = orc.block_bf16(x, w, K)
    got = orc.block_fp32(x, w, idx, logits=logits)
    # float64 restatement from first principles
    xd = x.double()
    p = torch.softmax(logits.double(), -1).gather(-1, idx)
    p = p / p.sum(-1, keepdim=True)
    out = torch.zeros(6, H, dtype=torch.float64)
    for t in range(6):
        for j in range(K):
            e = int(idx[t, j])
            gu = w["gate_up"][e].double() @ xd[t]
            a = F.silu(gu[:I]) * gu[I:]
            out[t] += p[t, j] * (w["down"][e].double() @ a)
    sh = w["sh_down"].double() @ (F.silu(w["sh_gate"].double() @ xd.T) * (w["sh_up"].double() @ xd.T))
    out += torch.sigmoid(xd @ w["sh_gate_w"].double().T) * sh.T
    assert (got.double() - out).abs().max() <= 1e-5


def test_bf16_oracle_within_north_star_tolerance_of_fp32():
    """The reference torch path itself (bf16) sits inside the bar the kernels are held to."""
    H, E, K, I = 256, 16, 4, 128
    w = orc.make_weights(H, E, I, I, seed=0)
    x = torch.randn(8, H, generator=torch.Generator().manual_seed(4)).to(BF16)
    out, idx, _, logits = orc.block_bf16(x, w, K)
    ref = orc.block_fp32(x, w, idx, logits=logits)
    assert max_abs(out, ref) <= 2e-2


# --------------------------------------------------------------------------------- fp8


def test_e4m3_table_and_torch_cast_agree():
    for bits, val in orc.E4M3_TABLE_CHECKS.items():
        assert orc.e4m3_decode(bits) == val
        t = torch.tensor([bits], dtype=torch.uint8).view(torch.float8_e4m3fn).float().item()
        assert t == val
    every = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float()
    for b in range(256):
        v = orc.e4m3_decode(b)
        assert (np.isnan(v) and torch.isnan(every[b])) or every[b].item() == v
        if not np.isnan(v):  # every e4m3 value is exactly a bf16 value
            assert torch.tensor(v).to(BF16).float().item() == v


def test_fp8_row_quantisation_error_bound():
    g = torch.Generator().manual_seed(0)
    w = (torch.randn(4, 64, 128, generator=g) * 0.02).to(BF16)
    q, s = orc.quantize_rows(w)
    deq = orc.dequantize_rows(q, s)
    rel = (deq - w.float()).abs() / w.float().abs().amax(-1, keepdim=True)
    assert rel.max() <= 2.0 ** -4 / 448 * 448 * 0.5 + 1e-6 or rel.max() <= 1 / 16
    assert (q.float().abs().amax(-1) == 448).all()


def test_zipf_router_distinct_experts():
    """C3's skewed routing: 64 tokens x top-8 touch ~140 distinct experts, as Zipf(1.1)
    sampling without replacement does (5-95%: 131-151), and popularity is rank-ordered."""
    g = torch.Generator().manual_seed(0)
    router = (torch.randn(256, 2048, generator=g) * 0.02).to(BF16)
    ds = []
    for seed in range(3):
        w, v = _synth().zipf_router(router, seed=seed)
        x = (torch.randn(64, 2048, generator=g) + _synth().ZIPF_MU * v).to(BF16)
        _, idx = orc.route(F.linear(x, w), 8)
        ds.append(int(torch.unique(idx).numel()))
    assert all(115 <= d <= 165 for d in ds), ds


# ------------------------------------------------------------------- add + RMSNorm


@pytest.mark.parametrize("with_h", [True, False])
def test_add_rms_matches_transformers_rmsnorm(with_h):
    """The oracle's norm == Transformers' Qwen3_5MoeRMSNorm (zero-centred weight) applied to
    the bf16 sum, bit for bit."""
    from transformers.models.qwen3_5_moe.modeling_qwen3_5_moe import Qwen3_5MoeRMSNorm

    H, eps = 512, 1e-6
    g = torch.Generator().manual_seed(5)
    x = torch.randn(7, H, generator=g).to(BF16)
    h = torch.randn(7, H, generator=g).to(BF16) if with_h else None
    norm = Qwen3_5MoeRMSNorm(H, eps=eps).to(BF16)
    with torch.no_grad():
        norm.weight.copy_((torch.randn(H, generator=g) * 0.3).to(BF16))
        total, out = orc.add_rms(x, h, norm.weight, eps)
        want_total = x + h if with_h else x
        assert torch.equal(total, want_total)
        assert torch.equal(out, norm(want_total))


def test_add_rms_one_hot_closed_form():
    """x = a e_i, eps = 0, H = 256: mean(x^2) = a^2 / 256, so out_i = sign(a) 16 (1 + w_i)
    (rounded to bf16) and every other element is zero. Pins the mean over H (not H - 1),
    the rsqrt and the 1 + w."""
    H = 256
    g = torch.Generator().manual_seed(6)
    w = (torch.randn(H, generator=g) * 0.5).to(BF16)
    for i, a in ((0, 4.0), (17, -0.5), (255, 2.0 ** -20)):
        x = torch.zeros(1, H, dtype=BF16)
        x[0, i] = a
        _, out = orc.add_rms(x, None, w, 0.0)
        want = torch.zeros(1, H)
        want[0, i] = (1.0 if a > 0 else -1.0) * 16.0 * (1.0 + w[i].float())
        assert torch.equal(out, want.to(BF16)), (i, a)


def test_add_rms_power_of_two_scale_invariance():
    """With eps = 0 scaling a row by 2^j scales mean(x^2) by 4^j exactly and the rsqrt by
    2^-j exactly, so the normalised row is unchanged bit for bit."""
    g = torch.Generator().manual_seed(8)
    x = torch.randn(5, 1024, generator=g).to(BF16)
    w = (torch.randn(1024, generator=g) * 0.1).to(BF16)
    _, base = orc.add_rms(x, None, w, 0.0)
    for j in (-3, 1, 5):
        _, out = orc.add_rms((x.float() * 2.0 ** j).to(BF16), None, w, 0.0)
        assert torch.equal(out, base), j


def test_add_rms_sum_rounds_to_nearest_even():
    """Small integers add exactly; 256 + 1 and 256 + 3 are bf16 ties (spacing 2 at 256) and
    round to the even mantissa: 256 and 260."""
    x = torch.tensor([[3.0, -7.0, 100.0, 256.0, 256.0, 0.0, 0.0, 0.0]]).to(BF16)
    h = torch.tensor([[4.0, 2.0, 27.0, 1.0, 3.0, 0.0, 0.0, 0.0]]).to(BF16)
    total, _ = orc.add_rms(x, h, torch.zeros(8, dtype=BF16), 1e-6)
    assert total.float().tolist() == [[7.0, -5.0, 127.0, 256.0, 260.0, 0.0, 0.0, 0.0]]
