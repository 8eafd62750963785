"""Pins the CPU oracle (oracle/moe_oracle.py) without the reference code: closed forms, invariants,
brute force on tiny inputs and library routines (torch.nn.functional), each chosen so that a plausible
mistake (dropped term, wrong index, swapped operands) fails. Mistakes are planted in copies of the
oracle functions, never in product code."""
import itertools
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import moe_oracle as O

BF = torch.bfloat16


def _close(a, b, rtol=2e-2, atol=1e-2):
    torch.testing.assert_close(a.float(), b.float(), rtol=rtol, atol=atol)


# ---------------------------------------------------------------------------------------------- RMSNorm

def test_rms_norm_constant_row_closed_form():
    for c in (0.5, -3.0, 7.25):
        x = torch.full((1, 64), c, dtype=BF)
        w = torch.linspace(0.5, 1.5, 64).to(BF)
        got = O.rms_norm(x, w, 1e-6)
        unit = torch.tensor(c / math.sqrt(c * c + 1e-6)).to(BF).float()
        want = (w.float() * unit).to(BF)[None]
        assert torch.equal(got, want)


def test_rms_norm_zero_row_and_dtype():
    x = torch.zeros(2, 32, dtype=BF)
    w = torch.ones(32, dtype=torch.float32)
    y = O.rms_norm(x, w, 1e-6)
    assert y.dtype == torch.float32 and torch.count_nonzero(y) == 0


def test_rms_norm_matches_library_and_rows_are_independent():
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(9, 2048, generator=g) * 3).to(BF)
    w = (1 + 0.02 * torch.randn(2048, generator=g)).to(BF)
    got = O.rms_norm(x, w, 1e-6)
    lib = F.rms_norm(x.float(), (2048,), w.float(), 1e-6)
    _close(got, lib, rtol=1e-2, atol=1e-2)
    perm = torch.randperm(9, generator=g)
    assert torch.equal(O.rms_norm(x[perm], w, 1e-6), got[perm])


def test_rms_norm_planted_sum_instead_of_mean_is_caught():
    def bad(x, w, eps):
        xf = x.float()
        return (w.float() * (xf * torch.rsqrt((xf * xf).sum(-1, keepdim=True) + eps)).to(BF).float()).to(BF)

    x = torch.randn(4, 256).to(BF)
    w = torch.ones(256, dtype=BF)
    lib = F.rms_norm(x.float(), (256,), w.float(), 1e-6)
    with pytest.raises(AssertionError):
        _close(bad(x, w, 1e-6), lib, rtol=1e-2, atol=1e-2)


# ----------------------------------------------------------------------------------------------- router

def _brute_topk(keys, k):
    """Top-k by (value descending, index ascending) through Python tuple ordering."""
    return [e for _, e in sorted(((-float(v), e) for e, v in enumerate(keys)))[:k]]


def test_softmax_router_uniform_logits():
    ids, w = O.router_select(torch.zeros(3, 64), scoring="softmax", top_k=6)
    assert ids.tolist() == [[0, 1, 2, 3, 4, 5, 64]] * 3
    torch.testing.assert_close(w[:, :6], torch.full((3, 6), 1 / 6))
    assert torch.equal(w[:, 6], torch.ones(3))


def test_softmax_router_brute_force_and_library_weights():
    g = torch.Generator().manual_seed(1)
    for trial in range(200):
        E, K = 8, 3
        logits = torch.randint(-3, 4, (1, E), generator=g).float() / 2  # many exact ties
        bias = torch.randint(-1, 2, (E,), generator=g).float() / 2 if trial % 2 else None
        ids, w = O.router_select(logits, bias, scoring="softmax", top_k=K, append_shared=False)
        z = logits[0] + (bias if bias is not None else 0)
        want = _brute_topk(z.tolist(), K)
        assert ids[0].tolist() == want
        ref_w = torch.softmax(z[want], dim=0)  # renormalised softmax = softmax over the selected
        torch.testing.assert_close(w[0], ref_w, rtol=1e-6, atol=1e-7)


def test_softmax_router_weights_sum_to_one_distinct_ids():
    g = torch.Generator().manual_seed(2)
    logits = torch.randn(64, 64, generator=g)
    ids, w = O.router_select(logits, torch.randn(64, generator=g) * 0.5, scoring="softmax", top_k=6, scale=1.0)
    assert all(len(set(r[:6])) == 6 for r in ids.tolist())
    torch.testing.assert_close(w[:, :6].sum(1), torch.ones(64), rtol=0, atol=6 * 2 ** -23 * 2)


def _brute_group(logits, bias, G, TOPG, K, scale):
    E = logits.numel()
    GS = E // G
    s = [1.0 / (1.0 + math.exp(-float(v))) for v in logits]
    r = [float(torch.tensor(sv, dtype=torch.float32) + bias[e]) for e, sv in enumerate(s)]
    gscore = []
    for gi in range(G):
        vals = sorted(r[gi * GS:(gi + 1) * GS], reverse=True)
        gscore.append(vals[0] + (vals[1] if GS > 1 else float("-inf")))
    kept = set(_brute_topk(gscore, TOPG))
    keys = [r[e] if e // GS in kept else float("-inf") for e in range(E)]
    sel = _brute_topk(keys, K)
    tot = sum(s[e] for e in sel)
    return sel, [s[e] / (tot + 1e-20) * scale for e in sel]


def test_sigmoid_group_router_brute_force():
    g = torch.Generator().manual_seed(3)
    for trial in range(100):
        E, G, TOPG, K = 16, 4, 2, 4
        logits = torch.randn(1, E, generator=g)
        bias = torch.randn(E, generator=g) * 0.1
        ids, w = O.router_select(logits, bias, scoring="sigmoid", n_group=G, topk_group=TOPG, top_k=K, scale=2.5)
        sel, ws = _brute_group(logits[0], bias, G, TOPG, K, 2.5)
        assert ids[0, :K].tolist() == sel
        assert ids[0, K].item() == E and w[0, K].item() == 1.0
        torch.testing.assert_close(w[0, :K], torch.tensor(ws), rtol=1e-5, atol=1e-6)


def test_sigmoid_single_group_is_plain_topk_of_biased_scores():
    g = torch.Generator().manual_seed(4)
    logits = torch.randn(5, 32, generator=g)
    bias = torch.randn(32, generator=g)
    ids, _ = O.router_select(logits, bias, scoring="sigmoid", top_k=8, append_shared=False)
    r = torch.sigmoid(logits) + bias
    for t in range(5):
        assert ids[t].tolist() == _brute_topk(r[t].tolist(), 8)


# ------------------------------------------------------------------------------------------------ align

def _brute_align(flat, E1, BM):
    P = len(flat)
    rows = []
    bexp = []
    for e in range(E1):
        mine = [p for p, v in enumerate(flat) if v == e]
        if not mine:
            continue
        n = -(-len(mine) // BM) * BM
        rows += mine + [P] * (n - len(mine))
        bexp += [e] * (n // BM)
    nb = (P + E1 * (BM - 1) + BM - 1) // BM
    rows += [P] * (nb * BM - len(rows))
    bexp += [-1] * (nb - len(bexp))
    return rows, bexp, nb


@pytest.mark.parametrize("BM", [1, 4, 64])
def test_align_brute_force(BM):
    rng = np.random.default_rng(5)
    for trial in range(60):
        E1 = int(rng.integers(1, 10))
        P = int(rng.integers(0, 200))
        flat = rng.integers(0, E1, P)
        s, b, nb, off = O.align_blocks(flat, E1, BM)
        rows, bexp, nb2 = _brute_align(flat.tolist(), E1, BM)
        assert nb == nb2 and s.tolist() == rows and b.tolist() == bexp
        assert off[-1] == sum(-(-int((flat == e).sum()) // BM) * BM for e in range(E1))


def test_align_invariants_and_dropped_ids():
    rng = np.random.default_rng(6)
    flat = rng.integers(-2, 67, 3584)
    s, b, nb, off = O.align_blocks(flat, 65, 64)
    P = flat.size
    placed = s[s < P]
    valid = np.nonzero((flat >= 0) & (flat < 65))[0]
    assert sorted(placed.tolist()) == valid.tolist()  # each valid pair exactly once, invalid dropped
    used = b[b >= 0]
    assert np.all(np.diff(used) >= 0) and np.all(b[used.size:] == -1)
    for blk in range(used.size):
        ids = s[blk * 64:(blk + 1) * 64]
        ids = ids[ids < P]
        assert np.all(flat[ids] == b[blk]) and np.all(np.diff(ids) > 0)


# --------------------------------------------------------------------------------------------- quantise

def test_quantize_closed_forms():
    w = torch.tensor([[127.0, 2.5, 3.5, -2.5, -127.0, 0.5], [0, 0, 0, 0, 0, 0]]).to(BF)
    q, s = O.quantize_rows_int8(w)
    assert q[0].tolist() == [127, 2, 4, -2, -127, 0]  # round half to even
    assert s[0].item() == 1.0
    assert q[1].tolist() == [0] * 6
    assert s[1].item() == pytest.approx(1e-8 / 127, rel=1e-6)


def test_quantize_max_maps_to_127_and_error_bound():
    g = torch.Generator().manual_seed(7)
    w = (torch.randn(33, 200, generator=g) * 0.02).to(BF)
    for sd in (torch.float32, torch.bfloat16):
        q, s = O.quantize_rows_int8(w, sd)
        assert torch.all(q.abs().amax(1) >= 126)
        err = (q.float() * s.float()[:, None] - w.float()).abs()
        assert torch.all(err <= s.float()[:, None] * 0.5 * 1.01 + s.float()[:, None] * (sd == torch.bfloat16))


# ------------------------------------------------------------------------------------------------ MoE

def _tiny(seed=0, E=5, H=32, I=16, N=6, K=2):
    g = torch.Generator().manual_seed(seed)
    w_gu = (torch.randn(E + 1, 2 * I, H, generator=g) * 0.2).to(BF)
    w_d = (torch.randn(E + 1, H, I, generator=g) * 0.2).to(BF)
    x = torch.randn(N, H, generator=g).to(BF)
    sel = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(N)])
    ids = torch.cat([sel, torch.full((N, 1), E)], 1)
    wts = torch.cat([torch.rand(N, K, generator=g), torch.ones(N, 1)], 1)
    return x, w_gu, w_d, ids, wts


def _fp64_moe(x, w_gu, w_d, ids, wts, swap=False, no_silu=False):
    I = w_d.shape[-1]
    y = torch.zeros(x.shape, dtype=torch.float64)
    for t in range(x.shape[0]):
        for k in range(ids.shape[1]):
            e = int(ids[t, k])
            g = w_gu[e, :I].double() @ x[t].double()
            u = w_gu[e, I:].double() @ x[t].double()
            if swap:
                g, u = u, g
            act = g if no_silu else g * torch.sigmoid(g)
            y[t] += float(wts[t, k]) * (w_d[e].double() @ (act * u))
    return y


def test_moe_matches_fp64_brute_force():
    x, w_gu, w_d, ids, wts = _tiny()
    y = O.moe(x, w_gu, w_d, ids, wts)
    _close(y, _fp64_moe(x, w_gu, w_d, ids, wts))


def test_moe_planted_mistakes_are_caught():
    x, w_gu, w_d, ids, wts = _tiny(1)
    y = O.moe(x, w_gu, w_d, ids, wts)
    for kw in (dict(swap=True), dict(no_silu=True)):
        with pytest.raises(AssertionError):
            _close(y, _fp64_moe(x, w_gu, w_d, ids, wts, **kw))
    with pytest.raises(AssertionError):  # transposed slot weights
        _close(y, _fp64_moe(x, w_gu, w_d, ids, wts.flip(1)))


def test_moe_batch_equals_single_tokens_and_permutes():
    x, w_gu, w_d, ids, wts = _tiny(2, N=9)
    y = O.moe(x, w_gu, w_d, ids, wts)
    for t in range(9):
        _close(O.moe(x[t:t + 1], w_gu, w_d, ids[t:t + 1], wts[t:t + 1]), y[t:t + 1], rtol=1e-2, atol=4e-3)
    perm = torch.randperm(9)
    _close(O.moe(x[perm], w_gu, w_d, ids[perm], wts[perm]), y[perm], rtol=1e-2, atol=4e-3)


def test_moe_zero_weight_slot_contributes_nothing():
    x, w_gu, w_d, ids, wts = _tiny(3)
    w0 = wts.clone()
    w0[:, 0] = 0
    y = O.moe(x, w_gu, w_d, ids, w0)
    y2 = O.moe(x, w_gu, w_d, ids[:, 1:], w0[:, 1:])
    _close(y, y2, rtol=1e-2, atol=4e-3)


def test_moe_int8_equals_dequantised_weights_and_reference_fallback():
    x, w_gu, w_d, ids, wts = _tiny(4)
    q_gu, s_gu = O.quantize_rows_int8(w_gu, torch.bfloat16)
    q_d, s_d = O.quantize_rows_int8(w_d, torch.bfloat16)
    y8 = O.moe(x, q_gu, q_d, ids, wts, s_gu, s_d)
    deq_gu = q_gu.float() * s_gu.float()[:, :, None]  # exact in fp32: 8-bit q times a bf16 scale
    deq_d = q_d.float() * s_d.float()[:, :, None]
    # same math, rounding points met at slightly different fp32 values: a bf16 ulp of the outputs (~3 here)
    _close(y8, O.moe(x, deq_gu, deq_d, ids, wts), rtol=2e-2, atol=3e-2)
    _close(y8, O.moe_int8_fallback(x, q_gu, q_d, s_gu, s_d, ids, wts), rtol=2e-2, atol=3e-2)
    _close(y8, O.moe(x, w_gu, w_d, ids, wts), rtol=5e-2, atol=3e-2)


def test_moe_residual_is_a_second_bf16_add():
    x, w_gu, w_d, ids, wts = _tiny(5)
    r = torch.randn(x.shape).to(BF)
    y = O.moe(x, w_gu, w_d, ids, wts)
    assert torch.equal(O.moe(x, w_gu, w_d, ids, wts, residual=r), (y.float() + r.float()).to(BF))


def test_moe_dropped_ids_leave_no_contribution():
    x, w_gu, w_d, ids, wts = _tiny(6)
    bad = ids.clone()
    bad[:, 0] = 99
    y = O.moe(x, w_gu, w_d, bad, wts)
    _close(y, O.moe(x, w_gu, w_d, ids[:, 1:], wts[:, 1:]), rtol=1e-2, atol=4e-3)


# -------------------------------------------------------------------------------------------- small linear

@pytest.mark.parametrize("act", [0, 1, 2])
def test_small_linear_matches_library(act):
    g = torch.Generator().manual_seed(8)
    M, K, N = 3, 256, 96
    x = torch.randn(M, K, generator=g).to(BF)
    w = (torch.randn(N, K, generator=g) * 0.05).to(BF)
    b = torch.randn(N, generator=g).to(BF)
    r = torch.randn(M, N, generator=g).to(BF)
    got = O.small_linear(x, w, b, act, r)
    ref = F.linear(x.float(), w.float(), b.float())
    ref = {0: ref, 1: F.gelu(ref, approximate="tanh"), 2: F.silu(ref)}[act] + r.float()
    _close(got, ref)


def test_small_linear_norm_prologue_matches_library():
    g = torch.Generator().manual_seed(9)
    x = (torch.randn(2, 512, generator=g) * 2).to(BF)
    w = (torch.randn(64, 512, generator=g) * 0.05).to(BF)
    gam = (1 + 0.1 * torch.randn(512, generator=g)).to(BF)
    got = O.small_linear(x, w, norm=(gam, 1e-6))
    ref = F.linear(F.rms_norm(x.float(), (512,), gam.float(), 1e-6), w.float())
    _close(got, ref)


@pytest.mark.parametrize("act", [0, 1, 2])
def test_small_linear_torch_branch_equals_bf16_library_ops(act):
    """More than 16 rows follow the reference's torch path (fastlinear.py:151-160). Torch's own bf16 CPU ops
    (F.rms_norm, F.linear, F.gelu / F.silu and the residual add on bf16 tensors) round where the branch says;
    they may differ in the GEMM's summation order, i.e. by an output ulp here and there."""
    g = torch.Generator().manual_seed(10)
    M, K, N = 40, 512, 96
    x = (torch.randn(M, K, generator=g) * 2).to(BF)
    w = (torch.randn(N, K, generator=g) * 0.05).to(BF)
    b = torch.randn(N, generator=g).to(BF)
    r = torch.randn(M, N, generator=g).to(BF)
    gam = (1 + 0.1 * torch.randn(K, generator=g)).to(BF)
    got = O.small_linear(x, w, b, act, r, norm=(gam, 1e-6))
    y = F.linear(F.rms_norm(x, (K,), gam, 1e-6), w, b)
    y = {0: y, 1: F.gelu(y, approximate="tanh"), 2: F.silu(y)}[act] + r
    assert got.dtype == BF and got.shape == (M, N)
    diff = (got.float() - y.float()).abs()
    ulp = y.float().abs().clamp_min(2 ** -6) * 2 ** -7  # one or two bf16 ulps
    assert (diff <= ulp).float().mean() > 0.97 and (diff <= 4 * ulp).all()


def test_small_linear_torch_branch_agrees_with_the_kernel_formula():
    """Both branches round at the same points after the GEMM (bf16 before the activation and before the
    residual); the norm rounds once on the torch branch and twice in the kernel formula, an ulp of the
    normalised row at most. So 20 rows through the torch branch equal 16 + 4 rows through the M <= 16 formula
    within the bf16 tolerance, most outputs within an ulp; a planted mistake (the residual added before the activation) is caught, and the
    branch's norm is the single-rounded one (bit-equal to F.rms_norm on bf16, unlike the two-step form)."""
    g = torch.Generator().manual_seed(11)
    M, K, N = 20, 256, 64
    x = torch.randn(M, K, generator=g).to(BF)
    w = (torch.randn(N, K, generator=g) * 0.05).to(BF)
    b = torch.randn(N, generator=g).to(BF)
    r = torch.randn(M, N, generator=g).to(BF)
    gam = (1 + 0.1 * torch.randn(K, generator=g)).to(BF)
    for act in (0, 1, 2):  # no residual here: one that cancels the output would magnify a one-ulp difference
        whole = O.small_linear(x, w, b, act, norm=(gam, 1e-6))
        parts = torch.cat([O.small_linear(x[:16], w, b, act, norm=(gam, 1e-6)),
                           O.small_linear(x[16:], w, b, act, norm=(gam, 1e-6))])
        _close(whole, parts, rtol=2e-2, atol=1e-2)
        d = (whole.float() - parts.float()).abs()
        assert (d <= parts.float().abs().clamp_min(2 ** -6) * 2 ** -7).float().mean() > 0.8
    planted = F.gelu(O.small_linear(x, w, b, 0, r, norm=(gam, 1e-6)).float(), approximate="tanh")
    assert not torch.allclose(planted, O.small_linear(x, w, b, 1, r, norm=(gam, 1e-6)).float(), rtol=2e-2, atol=1e-2)
    xn1 = O.small_linear(x, torch.eye(K).to(BF), norm=(gam, 1e-6))  # 20 rows: the torch branch's norm, exactly
    assert torch.equal(xn1, F.rms_norm(x, (K,), gam, 1e-6))
    assert not torch.equal(O.small_linear(x[:16], torch.eye(K).to(BF), norm=(gam, 1e-6)), xn1[:16])


def test_reference_loop_equals_the_kernel_formula():
    """O.moe_reference_loop (dev/test_moe_prefill.py:24-38, the CPU baseline) rounds where the kernels do (bf16 g
    and u from the bf16 GEMM, bf16 silu, bf16 a, bf16 part) and sums the slots in fp32 in expert order: equal to
    O.moe up to the order of that sum and an ulp of bf16 GEMM output. A planted mistake in the pair -> token
    map (order % NK instead of order // NK) is caught."""
    x, w_gu, w_d, ids, wts = _tiny(7)
    y = O.moe_reference_loop(x, w_gu, w_d, ids, wts)
    assert y.dtype == torch.float32
    _close(y.to(BF), O.moe(x, w_gu, w_d, ids, wts), rtol=1e-2, atol=4e-3)
    perm = torch.arange(x.shape[0]).flip(0)
    bad = O.moe_reference_loop(x[perm], w_gu, w_d, ids, wts)  # tokens no longer match their ids
    assert not torch.allclose(bad.to(BF).float(), O.moe(x, w_gu, w_d, ids, wts).float(), rtol=1e-2, atol=4e-3)
