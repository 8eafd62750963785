"""GPU parity of the HIP kernels against the CPU oracle, on the seeded synthetic thinker-MoE inputs.

Integer results (router ids given the same logits, align output, int8 codes) must be bit-exact; bf16
outputs must match within rtol 2e-2 / atol 1e-2 (fp32 accumulation on both sides, different order).
Full-size cases use the benchmarked shapes (hidden 2048, 64 + 1 experts of 1408, top-6)."""
import numpy as np
import pytest
import torch

import _mingmoe
import fastlinear
import fused_moe
import fused_ops
import workloads as W
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16
RTOL, ATOL = 2e-2, 1e-2


def close(got, want, rtol=RTOL, atol=ATOL):
    torch.testing.assert_close(got.float().cpu(), want.float().cpu(), rtol=rtol, atol=atol)


@pytest.fixture(scope="module")
def blk():
    """The benchmarked block on the GPU (bf16 + int8/bf16-scale experts) and its CPU copy."""
    b = W.block(seed=0, device=DEV)
    W.quantize_block(b, torch.bfloat16)
    torch.cuda.synchronize()
    cpu = {k: v.cpu() for k, v in b.items()}
    return b, cpu


def test_native_library_is_loaded():
    lib = _mingmoe.load()
    assert lib.mm_version() == _mingmoe.ABI_VERSION
    maps = open("/proc/self/maps").read()
    assert "libmingmoe.so" in maps


# ---------------------------------------------------------------------------------------------- RMSNorm

@pytest.mark.parametrize("rows", [1, 7, 512])
@pytest.mark.parametrize("wdt", [torch.bfloat16, torch.float32])
def test_rms_norm(rows, wdt):
    x = (W.normal((rows, 2048), 3.0, 5 + rows) ).to(DEV)
    w = W.normal((2048,), 0.02, 6, mean=1.0, dtype=wdt).to(DEV)
    y = fused_ops.rms_norm(x, w, 1e-6)
    ref = O.rms_norm(x.cpu(), w.cpu(), 1e-6)
    assert y.dtype == ref.dtype and y.shape == x.shape
    close(y, ref, rtol=1e-2, atol=1e-2)
    exact = (y.cpu().float() == ref.float()).float().mean().item()
    assert exact > 0.99, exact


def test_rms_norm_3d_noncontiguous():
    x = W.normal((4, 3, 4096), 1.0, 9).to(DEV)[..., ::2]
    w = W.normal((2048,), 0.02, 6, mean=1.0).to(DEV)
    close(fused_ops.rms_norm(x, w, 1e-6), O.rms_norm(x.cpu(), w.cpu(), 1e-6))


# ----------------------------------------------------------------------------------------------- router

def _check_selection(ids, wts, logits, bias, **kw):
    """ids must equal the oracle's selection on the GPU's own logits (bit-exact); weights to fp32 rounding."""
    ref_ids, ref_w = O.router_select(logits.cpu(), bias.cpu() if bias is not None else None, **kw)
    assert torch.equal(ids.cpu().long(), ref_ids), (ids.cpu()[:4], ref_ids[:4])
    torch.testing.assert_close(wts.cpu(), ref_w, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("n", [1, 3, 8, 512, 2048])
def test_router_softmax(blk, n):
    b, cpu = blk
    x = W.tokens(n, seed=20 + n, device=DEV)
    xn = fused_ops.rms_norm(x, b["norm_w"], W.EPS)
    bias = W.ragged_bias(device=DEV) if n >= 512 else None
    ids, wts, logits = fused_ops.route(xn, b["w32"], bias, top_k=6, scoring="softmax")
    close(logits, O.router_logits(xn.cpu(), cpu["w32"]), rtol=1e-4, atol=1e-4)
    _check_selection(ids, wts, logits, bias, scoring="softmax", top_k=6)
    assert torch.all(ids[:, 6] == 64) and torch.all(wts[:, 6] == 1.0)


@pytest.mark.parametrize("n", [1, 40])
def test_router_sigmoid_group_thinker_shape(n):
    E, H = 128, 1536  # the Ming thinker router: 8 groups, top 4 groups, top 8 experts, scale 2.5
    w32 = W.normal((E, H), 0.02, 30, DEV, dtype=torch.float32)
    bias = W.normal((E,), 0.05, 31, DEV, dtype=torch.float32)
    x = W.tokens(n, seed=32, device=DEV, hidden=H)
    logits = torch.empty(n, E, device=DEV)
    ids = torch.empty(n, 9, device=DEV, dtype=torch.long)
    wts = torch.empty(n, 9, device=DEV)
    fused_ops.moe_route(x, w32, bias, 8, 4, 8, 2.5, logits, ids, wts)
    close(logits, O.router_logits(x.cpu(), w32.cpu()), rtol=1e-4, atol=1e-4)
    # selection uses sigmoid scores; the GPU exp may differ from the CPU's in the last ulp, so a mismatch
    # is only accepted where the oracle's keys are tied within a few ulps
    ref_ids, ref_w = O.router_select(logits.cpu(), bias.cpu(), scoring="sigmoid", n_group=8, topk_group=4, top_k=8,
                                     scale=2.5)
    if not torch.equal(ids.cpu(), ref_ids):
        r = torch.sigmoid(logits.cpu()) + bias.cpu()
        for t in range(n):
            if ids[t].tolist() != ref_ids[t].tolist():
                got_set, ref_set = set(ids[t].tolist()), set(ref_ids[t].tolist())
                diff = [e for e in got_set ^ ref_set if e < E]
                gap = (r[t, diff].max() - r[t, diff].min()).item() if diff else 0.0
                assert gap < 1e-6, (t, ids[t].tolist(), ref_ids[t].tolist(), gap)
    else:
        torch.testing.assert_close(wts.cpu(), ref_w, rtol=1e-5, atol=1e-6)


def test_router_ties_pick_lowest_index():
    w32 = torch.zeros(64, 256, device=DEV)
    x = torch.ones(2, 256, device=DEV, dtype=BF)
    ids, wts, _ = fused_ops.route(x, w32, None, top_k=6, scoring="softmax")
    assert ids.cpu().tolist() == [[0, 1, 2, 3, 4, 5, 64]] * 2
    ids, wts, _ = fused_ops.route(x, w32, None, top_k=8, scoring="sigmoid", n_group=8, topk_group=4, scale=1.0)
    assert ids.cpu().tolist() == [[0, 1, 2, 3, 4, 5, 6, 7, 64]] * 2


# ------------------------------------------------------------------------------------------------ align

@pytest.mark.parametrize("P,E1,dtype", [(0, 65, torch.int64), (7, 65, torch.int64), (3584, 65, torch.int32),
                                        (14336, 65, torch.int64), (5000, 256, torch.int64), (33, 1, torch.int32),
                                        (49152, 256, torch.int32), (50001, 65, torch.int64)])
def test_align_bit_exact(P, E1, dtype):
    """Pairs up to 48 K keep their expert ids in LDS between the counting and scatter passes; above that the
    scatter re-reads them (P = 49152 and 50001 straddle the switch)."""
    g = torch.Generator().manual_seed(P + E1)
    flat = torch.randint(0, E1, (P,), generator=g).to(dtype)
    if P > 100:
        flat[::97] = 0  # a hot expert
    off = torch.empty(E1 + 1, dtype=torch.int32, device=DEV)
    s, bexp, nb = fused_moe._align_blocks(flat.to(DEV), E1, 64, expert_offsets=off)
    rs, rb, rnb, roff = O.align_blocks(flat.numpy(), E1, 64)
    assert nb == rnb
    assert np.array_equal(s.cpu().numpy(), rs) and np.array_equal(bexp.cpu().numpy(), rb)
    assert np.array_equal(off.cpu().numpy(), roff)


def test_align_drops_out_of_range_ids():
    flat = torch.tensor([3, -1, 70, 3, 64, 0], dtype=torch.long)
    s, bexp, nb = fused_moe._align_blocks(flat.to(DEV), 65, 4)
    rs, rb, _, _ = O.align_blocks(flat.numpy(), 65, 4)
    assert np.array_equal(s.cpu().numpy(), rs) and np.array_equal(bexp.cpu().numpy(), rb)


# --------------------------------------------------------------------------------------------- quantise

@pytest.mark.parametrize("sdt", [torch.float32, torch.bfloat16])
def test_quantize_bit_exact(blk, sdt):
    b, cpu = blk
    w = b["w_gu"][:3]
    q, s = fused_moe.quantize_rows_int8(w, scale_dtype=sdt)
    rq, rsc = O.quantize_rows_int8(cpu["w_gu"][:3], sdt)
    assert torch.equal(q.cpu(), rq) and torch.equal(s.cpu(), rsc)
    z = torch.zeros(2, 64, device=DEV, dtype=BF)
    q, s = fused_moe.quantize_rows_int8(z)
    assert torch.count_nonzero(q) == 0 and torch.allclose(s.cpu(), torch.full((2,), 1e-8 / 127))


# ------------------------------------------------------------------------------------------------ MoE

def _route_tokens(b, x, bias=None):
    xn = fused_ops.rms_norm(x, b["norm_w"], W.EPS)
    ids, wts, _ = fused_ops.route(xn, b["w32"], bias, top_k=6, scoring="softmax")
    return xn, ids, wts


def _oracle_moe(cpu, xn, ids, wts, int8=False, residual=None, return_a=False):
    if int8:
        return O.moe(xn.cpu(), cpu["q_gu"], cpu["q_d"], ids.cpu(), wts.cpu(), cpu["s_gu"], cpu["s_d"],
                     residual=residual, return_a=return_a)
    return O.moe(xn.cpu(), cpu["w_gu"], cpu["w_d"], ids.cpu(), wts.cpu(), residual=residual, return_a=return_a)


def test_decode_bf16_one_token(blk):
    b, cpu = blk
    x = W.tokens(1, seed=40, device=DEV)
    xn, ids, wts = _route_tokens(b, x)
    a_buf = torch.empty(7, 1408, device=DEV, dtype=BF)
    y = fused_moe.fused_moe_decode(xn, b["w_gu"], b["w_d"], ids[0], wts[0], a_buf=a_buf)
    ref, ref_a = _oracle_moe(cpu, xn, ids, wts, return_a=True)
    close(a_buf, ref_a)
    close(y, ref)
    yr = fused_moe.fused_moe_decode(xn, b["w_gu"], b["w_d"], ids[0], wts[0], residual=x)
    close(yr, _oracle_moe(cpu, xn, ids, wts, residual=x.cpu()))


@pytest.mark.parametrize("n", [1, 2, 4, 8])
@pytest.mark.parametrize("sdt", [torch.bfloat16, torch.float32])
def test_decode_int8_batches(blk, n, sdt):
    b, cpu = blk
    if sdt == torch.float32:
        q_gu, s_gu = fused_moe.quantize_rows_int8(b["w_gu"], scale_dtype=sdt)
        q_d, s_d = fused_moe.quantize_rows_int8(b["w_d"], scale_dtype=sdt)
        c = {"q_gu": q_gu.cpu(), "q_d": q_d.cpu(), "s_gu": s_gu.cpu(), "s_d": s_d.cpu()}
    else:
        q_gu, s_gu, q_d, s_d, c = b["q_gu"], b["s_gu"], b["q_d"], b["s_d"], cpu
    x = W.tokens(n, seed=50 + n, device=DEV)
    xn, ids, wts = _route_tokens(b, x)
    y = fused_moe.fused_moe_decode(xn, q_gu, q_d, ids, wts, s_gu=s_gu, s_d=s_d)
    close(y, _oracle_moe(c, xn, ids, wts, int8=True))


@pytest.mark.parametrize("n", [1, 2, 4, 8])
@pytest.mark.parametrize("int8", [False, True])
def test_decode_dropped_pairs_contribute_nothing(blk, n, int8):
    """Pairs whose id lies outside the stack (-1, or the slot count 65) contribute nothing, as the oracle's zero
    rows, in every form of the down kernel: one token, batches that reload the expert rows per pair and batches
    that hold them, one or two rows per lane group; one slot of every token dropped, and a whole token's slots."""
    b, cpu = blk
    x = W.tokens(n, seed=70 + n, device=DEV)
    xn, ids, wts = _route_tokens(b, x)
    ids = ids.clone()
    ids[:, 1] = -1
    ids[:, 4] = 65
    if n > 1:
        ids[n - 1, :] = -1
    if int8:
        y = fused_moe.fused_moe_decode(xn, b["q_gu"], b["q_d"], ids, wts, s_gu=b["s_gu"], s_d=b["s_d"], residual=x)
    else:
        y = fused_moe.fused_moe_decode(xn, b["w_gu"], b["w_d"], ids, wts, residual=x)
    ref = _oracle_moe(cpu, xn, ids, wts, int8=int8, residual=x.cpu())
    close(y, ref)
    if n > 1:  # the token with every slot dropped keeps its residual alone: bf16(0) + x
        assert torch.equal(y[n - 1].cpu(), x[n - 1].cpu())


@pytest.mark.parametrize("n,int8", [(1, False), (3, False), (1, True), (2, True), (4, True), (8, True)])
def test_moe_block_decode_matches_unfused_and_oracle(blk, n, int8):
    """The three-kernel decode block equals rms_norm -> moe_route -> fused_moe_decode(residual=x) bit for bit
    (same rstd reduction, same logits order, same picks), and the oracle within tolerance."""
    b, cpu = blk
    x = W.tokens(n, seed=140 + n, device=DEV)
    wg, wd = (b["q_gu"], b["q_d"]) if int8 else (b["w_gu"], b["w_d"])
    sg, sd = (b["s_gu"], b["s_d"]) if int8 else (None, None)
    y, ids, wts, logits = fused_moe.moe_block_decode(x, b["norm_w"], W.EPS, b["w32"], wg, wd, top_k=6, s_gu=sg, s_d=sd)
    xn = fused_ops.rms_norm(x, b["norm_w"], W.EPS)
    l2 = torch.empty(n, 64, device=DEV)
    i2 = torch.empty(n, 7, device=DEV, dtype=torch.long)
    w2 = torch.empty(n, 7, device=DEV)
    fused_ops.moe_route(xn, b["w32"], None, 1, 1, 6, 1.0, l2, i2, w2, scoring="softmax")
    y2 = fused_moe.fused_moe_decode(xn, wg, wd, i2, w2, s_gu=sg, s_d=sd, residual=x)
    assert torch.equal(logits, l2) and torch.equal(ids, i2) and torch.equal(wts, w2)
    assert torch.equal(y, y2)
    close(y, _oracle_moe(cpu, xn, ids, wts, int8=int8, residual=x.cpu()))


def test_moe_block_decode_sigmoid_group_thinker_router():
    """The Ming thinker's router (128 experts, 8 groups, top 4 groups, top 8, scale 2.5) on the fused path."""
    H, I, E = 1536, 512, 128
    w_gu = W.normal((E + 1, 2 * I, H), 0.02, 150, DEV)
    w_d = W.normal((E + 1, H, I), 0.02, 151, DEV)
    w32 = W.normal((E, H), 0.02, 152, DEV, dtype=torch.float32)
    bias = W.normal((E,), 0.05, 153, DEV, dtype=torch.float32)
    nw = W.normal((H,), 0.02, 154, DEV, mean=1.0)
    x = W.tokens(1, seed=155, device=DEV, hidden=H)
    y, ids, wts, logits = fused_moe.moe_block_decode(x, nw, 1e-6, w32, w_gu, w_d, top_k=8, bias=bias, scoring="sigmoid",
                                                     n_group=8, topk_group=4, scale=2.5)
    ref_ids, ref_w = O.router_select(logits.cpu(), bias.cpu(), scoring="sigmoid", n_group=8, topk_group=4, top_k=8,
                                     scale=2.5)
    assert torch.equal(ids.cpu(), ref_ids)
    torch.testing.assert_close(wts.cpu(), ref_w, rtol=1e-5, atol=1e-6)
    xn = O.rms_norm(x.cpu(), nw.cpu(), 1e-6)
    close(y, O.moe(xn, w_gu.cpu(), w_d.cpu(), ids.cpu(), wts.cpu(), residual=x.cpu()))


@pytest.mark.parametrize("E", [48, 64])
@pytest.mark.parametrize("scoring", ["sigmoid", "softmax"])
def test_moe_block_decode_selecting_gate_up(E, scoring):
    """One bf16 token with at most 64 experts and no groups: the gate/up kernel ranks the logits itself (lanes past E
    masked). With a bias, sigmoid or softmax scoring and E below and at 64, every output equals the unfused chain
    rms_norm -> moe_route -> fused_moe_decode bit for bit, and the ids the oracle's selection."""
    H, I = 1024, 384
    w_gu = W.normal((E + 1, 2 * I, H), 0.02, 160 + E, DEV)
    w_d = W.normal((E + 1, H, I), 0.02, 161 + E, DEV)
    w32 = W.normal((E, H), 0.02, 162 + E, DEV, dtype=torch.float32)
    bias = W.normal((E,), 0.5, 163 + E, DEV, dtype=torch.float32)
    nw = W.normal((H,), 0.02, 164 + E, DEV, mean=1.0)
    x = W.tokens(1, seed=165 + E, device=DEV, hidden=H)
    scale = 2.5 if scoring == "sigmoid" else 1.0
    y, ids, wts, logits = fused_moe.moe_block_decode(x, nw, 1e-6, w32, w_gu, w_d, top_k=6, bias=bias, scoring=scoring,
                                                     scale=scale)
    xn = fused_ops.rms_norm(x, nw, 1e-6)
    l2 = torch.empty(1, E, device=DEV)
    i2 = torch.empty(1, 7, device=DEV, dtype=torch.long)
    w2 = torch.empty(1, 7, device=DEV)
    fused_ops.moe_route(xn, w32, bias, 1, 1, 6, scale, l2, i2, w2, scoring=scoring)
    y2 = fused_moe.fused_moe_decode(xn, w_gu, w_d, i2, w2, residual=x)
    assert torch.equal(logits, l2) and torch.equal(ids, i2) and torch.equal(wts, w2)
    assert torch.equal(y, y2)
    ref_ids, _ = O.router_select(logits.cpu(), bias.cpu(), scoring=scoring, top_k=6, scale=scale)
    assert torch.equal(ids.cpu(), ref_ids)
    assert int(ids[0, -1]) == E and float(wts[0, -1]) == 1.0


@pytest.mark.parametrize("n", [2, 5, 8])
def test_decode_bf16_batches_and_repeated_experts(blk, n):
    b, cpu = blk
    x = W.tokens(n, seed=60 + n, device=DEV)
    xn, ids, wts = _route_tokens(b, x)
    ids = ids.clone()
    ids[:, 0] = 3  # every token shares expert 3
    y = fused_moe.fused_moe_prefill(xn, b["w_gu"], b["w_d"], ids, wts)  # N <= 8 takes the decode kernels
    close(y, _oracle_moe(cpu, xn, ids, wts))


def test_prefill_bf16_ragged_512(blk):
    b, cpu = blk
    x = W.tokens(512, seed=70, device=DEV)
    xn, ids, wts = _route_tokens(b, x, W.ragged_bias(device=DEV))
    y = fused_moe.fused_moe_prefill(xn, b["w_gu"], b["w_d"], ids, wts, residual=x)
    close(y, _oracle_moe(cpu, xn, ids, wts, residual=x.cpu()))


@pytest.mark.parametrize("n", [9, 100])
def test_prefill_int8(blk, n):
    b, cpu = blk
    x = W.tokens(n, seed=80 + n, device=DEV)
    xn, ids, wts = _route_tokens(b, x, W.ragged_bias(device=DEV))
    y = fused_moe.fused_moe_prefill(xn, b["q_gu"], b["q_d"], ids, wts, s_gu=b["s_gu"], s_d=b["s_d"])
    close(y, _oracle_moe(cpu, xn, ids, wts, int8=True))


@pytest.mark.parametrize("n,int8", [(512, False), (100, True), (20, False), (5, False)])
def test_moe_block_prefill_matches_unfused_and_oracle(blk, n, int8):
    """The prefill block (norm fused into the router GEMM) equals rms_norm -> route -> fused_moe_prefill
    (residual=x) bit for bit above the decode sizes, and the oracle within tolerance."""
    b, cpu = blk
    bias = W.ragged_bias(device=DEV)
    x = W.tokens(n, seed=160 + n, device=DEV)
    wg, wd = (b["q_gu"], b["q_d"]) if int8 else (b["w_gu"], b["w_d"])
    sg, sd = (b["s_gu"], b["s_d"]) if int8 else (None, None)
    sc = fused_moe.PrefillScratch(n, 7, 65, W.HIDDEN, W.INTER, DEV, block=True, w_dtype=wg.dtype)
    y, ids, wts, logits = fused_moe.moe_block_prefill(x, b["norm_w"], W.EPS, b["w32"], wg, wd, top_k=6, bias=bias,
                                                      s_gu=sg, s_d=sd, scratch=sc)
    xn = fused_ops.rms_norm(x, b["norm_w"], W.EPS)
    assert torch.equal(sc.xn, xn)
    i2, w2, l2 = fused_ops.route(xn, b["w32"], bias, top_k=6, scoring="softmax")
    assert torch.equal(logits, l2) and torch.equal(ids, i2.long()) and torch.equal(wts, w2)
    if n > fused_moe.MAX_DECODE_TOKENS:  # the unfused call takes the same prefill kernels
        y2 = fused_moe.fused_moe_prefill(xn, wg, wd, i2, w2, s_gu=sg, s_d=sd, residual=x)
        assert torch.equal(y, y2)
    close(y, _oracle_moe(cpu, xn, ids, wts, int8=int8, residual=x.cpu()))


@pytest.mark.parametrize("H,E,n,scoring,groups,top_k", [(1536, 48, 37, "softmax", (1, 1), 6),
                                                         (2048, 64, 40, "sigmoid", (8, 4), 6),
                                                         (1024, 64, 9, "softmax", (1, 1), 8),
                                                         (2560, 64, 20, "softmax", (1, 1), 6)])
def test_block_prefill_router_front_shapes(H, E, n, scoring, groups, top_k):
    """The router front of the prefill block at other shapes: normalised rows, logits, ids and weights equal
    rms_norm -> route bit for bit with a partial 16-token group, an expert count that is not a multiple of
    16, rows wider than 2048 and the sigmoid group router; the block output equals fused_moe_prefill."""
    I = 128
    w_gu = W.normal((E + 1, 2 * I, H), 0.02, 170, DEV)
    w_d = W.normal((E + 1, H, I), 0.02, 171, DEV)
    w32 = W.normal((E, H), 0.02, 172, DEV, dtype=torch.float32)
    bias = W.normal((E,), 0.05, 173, DEV, dtype=torch.float32)
    nw = W.normal((H,), 0.02, 174, DEV, mean=1.0)
    x = W.tokens(n, seed=175, device=DEV, hidden=H)
    ng, tg = groups
    y, ids, wts, logits = fused_moe.moe_block_prefill(x, nw, 1e-6, w32, w_gu, w_d, top_k=top_k, bias=bias,
                                                      scoring=scoring, n_group=ng, topk_group=tg, scale=1.5)
    xn = fused_ops.rms_norm(x, nw, 1e-6)
    i2, w2, l2 = fused_ops.route(xn, w32, bias, top_k=top_k, scoring=scoring, n_group=ng, topk_group=tg, scale=1.5)
    assert torch.equal(logits, l2) and torch.equal(ids, i2.long()) and torch.equal(wts, w2)
    y2 = fused_moe.fused_moe_prefill(xn, w_gu, w_d, i2, w2, residual=x)
    assert torch.equal(y, y2)
    ref_ids, _ = O.router_select(logits.cpu(), bias.cpu(), scoring=scoring, n_group=ng, topk_group=tg, top_k=top_k,
                                 scale=1.5)
    assert torch.equal(ids.cpu(), ref_ids)


def test_moe_block_prefill_zipf_2048_128_row_blocks(blk):
    """2048 Zipf-routed tokens average 220 pairs per expert, so bf16 experts take 128-row blocks: the block
    equals the unfused chain bit for bit, and a seeded subset matches the oracle."""
    b, cpu = blk
    bias = W.zipf_bias(device=DEV)
    x = W.tokens(2048, seed=92, device=DEV)
    assert fused_moe.prefill_block_m(2048, 7, 65) == 128 and fused_moe.prefill_block_m(512, 7, 65) == 64
    assert fused_moe.prefill_block_m(2048, 7, 65, torch.int8) == 64
    y, ids, wts, _ = fused_moe.moe_block_prefill(x, b["norm_w"], W.EPS, b["w32"], b["w_gu"], b["w_d"], top_k=6,
                                                 bias=bias)
    xn = fused_ops.rms_norm(x, b["norm_w"], W.EPS)
    y2 = fused_moe.fused_moe_prefill(xn, b["w_gu"], b["w_d"], ids, wts, residual=x)
    assert torch.equal(y, y2)
    sub = torch.randperm(2048, generator=torch.Generator().manual_seed(2))[:128]
    close(y.cpu()[sub], _oracle_moe(cpu, xn[sub.to(DEV)], ids[sub.to(DEV)], wts[sub.to(DEV)],
                                    residual=x.cpu()[sub]))


def test_prefill_zipf_2048_int8_subset(blk):
    """Hot experts of the Zipf batch on the int8 path (64-row blocks, many per hot expert)."""
    b, cpu = blk
    x = W.tokens(2048, seed=91, device=DEV)
    xn, ids, wts = _route_tokens(b, x, W.zipf_bias(device=DEV))
    y = fused_moe.fused_moe_prefill(xn, b["q_gu"], b["q_d"], ids, wts, s_gu=b["s_gu"], s_d=b["s_d"])
    sub = torch.randperm(2048, generator=torch.Generator().manual_seed(1))[:160]
    close(y.cpu()[sub], _oracle_moe(cpu, xn[sub.to(DEV)], ids[sub.to(DEV)], wts[sub.to(DEV)], int8=True))


def test_prefill_zipf_2048_subset_and_histogram(blk):
    b, cpu = blk
    x = W.tokens(2048, seed=90, device=DEV)
    xn, ids, wts = _route_tokens(b, x, W.zipf_bias(device=DEV))
    counts = torch.bincount(ids.reshape(-1).cpu(), minlength=65)[:64].sort(descending=True).values
    assert counts[:3].sum().item() / ids.numel() > 0.30 or counts[:2].sum().item() / ids.numel() > 0.30
    y = fused_moe.fused_moe_prefill(xn, b["w_gu"], b["w_d"], ids, wts)
    # each token's output depends on that token only: check a seeded subset against the oracle
    sub = torch.randperm(2048, generator=torch.Generator().manual_seed(0))[:192]
    close(y.cpu()[sub], _oracle_moe(cpu, xn[sub.to(DEV)], ids[sub.to(DEV)], wts[sub.to(DEV)]))


@pytest.mark.parametrize("int8", [False, True])
def test_prefill_and_decode_ragged_shapes(int8):
    """Tails on every tiled dim: hidden 1536 (6 column tiles of 256), inter 208 (partial 128-column tile and a
    partial 64-wide k slab), 129 expert slots (the Ming thinker's 128 + shared), top-8. 1100 tokens put
    about 69 pairs on each routed expert (64-pair blocks, several per expert, odd last blocks)."""
    H, I, E, K = 1536, 208, 128, 8
    w_gu = W.normal((E + 1, 2 * I, H), 0.02, 130, DEV)
    w_d = W.normal((E + 1, H, I), 0.02, 131, DEV)
    g = torch.Generator().manual_seed(132)
    for n in (3, 77, 1100):
        sel = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(n)])
        ids = torch.cat([sel, torch.full((n, 1), E)], 1).to(DEV)
        wts = torch.cat([torch.rand(n, K, generator=g), torch.ones(n, 1)], 1).to(DEV)
        x = W.normal((n, H), 1.0, 133 + n, DEV)
        if int8:
            q_gu, s_gu = fused_moe.quantize_rows_int8(w_gu, scale_dtype=torch.bfloat16)
            q_d, s_d = fused_moe.quantize_rows_int8(w_d, scale_dtype=torch.bfloat16)
            y = fused_moe.fused_moe_prefill(x, q_gu, q_d, ids, wts, s_gu=s_gu, s_d=s_d)
            ref = O.moe(x.cpu(), q_gu.cpu(), q_d.cpu(), ids.cpu(), wts.cpu(), s_gu.cpu(), s_d.cpu())
        else:
            y = fused_moe.fused_moe_prefill(x, w_gu, w_d, ids, wts)
            ref = O.moe(x.cpu(), w_gu.cpu(), w_d.cpu(), ids.cpu(), wts.cpu())
        close(y, ref)


@pytest.mark.parametrize("int8", [False, True])
def test_prefill_dropped_pairs_contribute_nothing(blk, int8):
    """Prefill pairs whose id lies outside the stack (-1, 65) contribute nothing (align leaves them out of every
    expert block), as the oracle's zero rows; tokens with every slot dropped keep their residual alone."""
    b, cpu = blk
    n = 100
    x = W.tokens(n, seed=80, device=DEV)
    xn, ids, wts = _route_tokens(b, x)
    ids = ids.clone()
    ids[::3, 2] = -1
    ids[1::4, 5] = 65
    ids[7, :] = 65
    ids[50, :] = -1
    if int8:
        y = fused_moe.fused_moe_prefill(xn, b["q_gu"], b["q_d"], ids, wts, s_gu=b["s_gu"], s_d=b["s_d"], residual=x)
    else:
        y = fused_moe.fused_moe_prefill(xn, b["w_gu"], b["w_d"], ids, wts, residual=x)
    close(y, _oracle_moe(cpu, xn, ids, wts, int8=int8, residual=x.cpu()))
    assert torch.equal(y[7].cpu(), x[7].cpu()) and torch.equal(y[50].cpu(), x[50].cpu())


@pytest.mark.parametrize("int8", [False, True])
def test_prefill_phases_and_block_slab_layout(int8):
    """The prefill run as its three phases on one scratch (gate/up, then down, then combine, each a call of its own)
    equals the one call bit for bit; and the gated activations sit in the scratch in 64-column slabs per expert
    block, [nb][ceil(I/64)][block_m][64] with row r of block b holding pair sorted_ids[b * block_m + r]: rebuilt in
    pair order they match the oracle's, on ragged dims (inter 208: a partial last slab, a partial column tile)."""
    H, I, E, K, n = 1536, 208, 32, 6, 90
    w_gu = W.normal((E + 1, 2 * I, H), 0.02, 140, DEV)
    w_d = W.normal((E + 1, H, I), 0.02, 141, DEV)
    g = torch.Generator().manual_seed(142)
    sel = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(n)])
    ids = torch.cat([sel, torch.full((n, 1), E)], 1).to(DEV)
    wts = torch.cat([torch.rand(n, K, generator=g), torch.ones(n, 1)], 1).to(DEV)
    x = W.normal((n, H), 1.0, 143, DEV)
    kw = {}
    if int8:
        w_gu, kw["s_gu"] = fused_moe.quantize_rows_int8(w_gu, scale_dtype=torch.float32)
        w_d, kw["s_d"] = fused_moe.quantize_rows_int8(w_d, scale_dtype=torch.float32)
    sc1 = fused_moe.PrefillScratch(n, K + 1, E + 1, H, I, DEV, w_dtype=w_gu.dtype)
    y1 = fused_moe.fused_moe_prefill(x, w_gu, w_d, ids, wts, scratch=sc1, **kw).clone()
    sc2 = fused_moe.PrefillScratch(n, K + 1, E + 1, H, I, DEV, w_dtype=w_gu.dtype)
    for ph, al in ((_mingmoe.MM_PHASE_GATE_UP, True), (_mingmoe.MM_PHASE_DOWN, False),
                   (_mingmoe.MM_PHASE_COMBINE, False)):
        y2 = fused_moe.fused_moe_prefill(x, w_gu, w_d, ids, wts, scratch=sc2, phases=ph, align=al, **kw)
    assert torch.equal(y1, y2)
    P, BM, nb, nsl = n * (K + 1), sc1.block_m, sc1.nb, (I + 63) // 64
    assert sc1.a.shape == (nb * BM, nsl * 64)
    rows = sc1.a.view(nb, nsl, BM, 64).permute(0, 2, 1, 3).reshape(nb * BM, nsl * 64)[:, :I]
    sid = sc1.sorted_ids.long()
    valid = sid < P
    assert int(valid.sum()) == P  # every pair has one row
    a = torch.zeros(P, I, dtype=BF, device=DEV)
    a[sid[valid]] = rows[valid]
    s_gu, s_d = (kw["s_gu"].cpu(), kw["s_d"].cpu()) if int8 else (None, None)
    _, a_ref = O.moe(x.cpu(), w_gu.cpu(), w_d.cpu(), ids.cpu(), wts.cpu(), s_gu, s_d, return_a=True)
    close(a, a_ref)


def test_prefill_ragged_shapes_128_pair_blocks():
    """The 128-pair blocks (bf16 experts averaging at least 128 pairs: 700 tokens x 7 slots over 33 slots) on
    ragged dims: hidden 1536, inter 208 (a partial 128-column tile and a partial 64-wide k slab), so the
    two-row-wave layout of those tiles meets padding rows, partial column tiles and the k tail."""
    H, I, E, K = 1536, 208, 32, 6
    n = 700
    assert fused_moe.prefill_block_m(n, K + 1, E + 1) == 128
    w_gu = W.normal((E + 1, 2 * I, H), 0.02, 135, DEV)
    w_d = W.normal((E + 1, H, I), 0.02, 136, DEV)
    g = torch.Generator().manual_seed(137)
    sel = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(n)])
    sel[: n // 3, 0] = 5  # one hot expert: several full 128-pair blocks
    ids = torch.cat([sel, torch.full((n, 1), E)], 1).to(DEV)
    wts = torch.cat([torch.rand(n, K, generator=g), torch.ones(n, 1)], 1).to(DEV)
    x = W.normal((n, H), 1.0, 138, DEV)
    y = fused_moe.fused_moe_prefill(x, w_gu, w_d, ids, wts)
    close(y, O.moe(x.cpu(), w_gu.cpu(), w_d.cpu(), ids.cpu(), wts.cpu()))


def test_gate_up_slabs_copy_layout():
    """gate_up_slabs writes out[e, q, t, j, c] = w_gu[e, 8 q + j, 64 t + c], from a contiguous stack and from a
    strided view (rows 384 apart, 8 spare rows per expert)."""
    w = W.normal((5, 192, 320), 1.0, 140, DEV)
    q = fused_moe.gate_up_slabs(w)
    assert torch.equal(q, w.reshape(5, 24, 8, 5, 64).permute(0, 1, 3, 2, 4).contiguous())
    big = W.normal((5, 200, 384), 1.0, 141, DEV)
    view = big[:, :192, :320]
    assert view.stride(1) == 384 and view.stride(0) == 200 * 384
    q2 = fused_moe.gate_up_slabs(view)
    assert torch.equal(q2, view.contiguous().reshape(5, 24, 8, 5, 64).permute(0, 1, 3, 2, 4).contiguous())
    with pytest.raises(ValueError, match="multiple of 64"):
        fused_moe.gate_up_slabs(W.normal((2, 8, 96), 1.0, 142, DEV))


def test_down_slabs_copy_layout():
    """down_slabs writes out[e, q, t, j, c] = w_d[e, 8 q + j, 64 t + c], from a contiguous stack and from a strided
    view (rows 384 apart, 8 spare rows per expert)."""
    w = W.normal((5, 24, 320), 1.0, 147, DEV)
    q = fused_moe.down_slabs(w)
    assert torch.equal(q, w.reshape(5, 3, 8, 5, 64).permute(0, 1, 3, 2, 4).contiguous())
    big = W.normal((5, 32, 384), 1.0, 148, DEV)
    view = big[:, :24, :320]
    assert view.stride(1) == 384 and view.stride(0) == 32 * 384
    q2 = fused_moe.down_slabs(view)
    assert torch.equal(q2, view.contiguous().reshape(5, 3, 8, 5, 64).permute(0, 1, 3, 2, 4).contiguous())
    with pytest.raises(ValueError, match="multiple of 64"):
        fused_moe.down_slabs(W.normal((2, 8, 96), 1.0, 149, DEV))


def test_int8_slab_copies_layout():
    """int8 stacks take 16-row pieces: out[e, q, t, j, c] = w[e, 16 q + j, 64 t + c] (gate/up and down copies, from a
    contiguous stack and from a strided view)."""
    g = torch.Generator().manual_seed(155)
    w = torch.randint(-127, 128, (3, 64, 320), generator=g, dtype=torch.int8).to(DEV)
    want = w.reshape(3, 4, 16, 5, 64).permute(0, 1, 3, 2, 4).contiguous()
    assert torch.equal(fused_moe.gate_up_slabs(w), want) and torch.equal(fused_moe.down_slabs(w), want)
    big = torch.randint(-127, 128, (3, 80, 384), generator=g, dtype=torch.int8).to(DEV)
    view = big[:, :64, :320]
    assert torch.equal(fused_moe.gate_up_slabs(view),
                       view.contiguous().reshape(3, 4, 16, 5, 64).permute(0, 1, 3, 2, 4).contiguous())
    with pytest.raises(ValueError, match="multiple of 16"):
        fused_moe.down_slabs(torch.zeros(2, 24, 64, dtype=torch.int8, device=DEV))


@pytest.mark.parametrize("n,sdt", [(100, torch.bfloat16), (512, torch.float32)])
def test_int8_prefill_reads_the_slab_copy_bit_for_bit(blk, n, sdt):
    """int8 experts (bf16 or fp32 row scales) with prefill copies of q_gu and q_d: the block and fused_moe_prefill give
    the row layout's outputs bit for bit, and the oracle's within tolerance."""
    b, cpu = blk
    if sdt == torch.float32:
        q_gu, s_gu = fused_moe.quantize_rows_int8(b["w_gu"], scale_dtype=sdt)
        q_d, s_d = fused_moe.quantize_rows_int8(b["w_d"], scale_dtype=sdt)
    else:
        q_gu, s_gu, q_d, s_d = b["q_gu"], b["s_gu"], b["q_d"], b["s_d"]
    gq, dq = fused_moe.gate_up_slabs(q_gu), fused_moe.down_slabs(q_d)
    bias = W.ragged_bias(device=DEV)
    x = W.tokens(n, seed=190 + n, device=DEV)
    args = (x, b["norm_w"], W.EPS, b["w32"], q_gu, q_d)
    y, ids, wts, _ = fused_moe.moe_block_prefill(*args, top_k=6, bias=bias, s_gu=s_gu, s_d=s_d)
    for g_, d_ in ((gq, None), (None, dq), (gq, dq)):
        yq, idq, _, _ = fused_moe.moe_block_prefill(*args, top_k=6, bias=bias, s_gu=s_gu, s_d=s_d, w_gu_slabs=g_,
                                                    w_d_slabs=d_)
        assert torch.equal(idq, ids) and torch.equal(yq, y)
    xn = fused_ops.rms_norm(x, b["norm_w"], W.EPS)
    y2 = fused_moe.fused_moe_prefill(xn, q_gu, q_d, ids, wts, s_gu=s_gu, s_d=s_d, residual=x, w_gu_slabs=gq,
                                     w_d_slabs=dq)
    assert torch.equal(y2, y)
    c = {"q_gu": q_gu.cpu(), "q_d": q_d.cpu(), "s_gu": s_gu.cpu(), "s_d": s_d.cpu()}
    close(y, _oracle_moe(c, xn, ids, wts, int8=True, residual=x.cpu()))


@pytest.mark.parametrize("n,kind", [(100, "ragged"), (512, "ragged"), (2048, "zipf")])
def test_prefill_reads_the_slab_copy_bit_for_bit(blk, n, kind):
    """With the slab copies of w_gu and w_d (each alone and both) the prefill block and fused_moe_prefill give the
    row layout's outputs bit for bit: 64-pair blocks at 100 and 512 tokens, 128-pair blocks for the 2048 Zipf
    tokens (the GEMMs only read the weights at other addresses)."""
    b, _ = blk
    wq = fused_moe.gate_up_slabs(b["w_gu"])
    wd = fused_moe.down_slabs(b["w_d"])
    bias = W.zipf_bias(device=DEV) if kind == "zipf" else W.ragged_bias(device=DEV)
    x = W.tokens(n, seed=170 + n, device=DEV)
    y, ids, wts, _ = fused_moe.moe_block_prefill(x, b["norm_w"], W.EPS, b["w32"], b["w_gu"], b["w_d"], top_k=6,
                                                 bias=bias)
    for gq, dq in ((wq, None), (wq, wd)):
        yq, idq, _, _ = fused_moe.moe_block_prefill(x, b["norm_w"], W.EPS, b["w32"], b["w_gu"], b["w_d"], top_k=6,
                                                    bias=bias, w_gu_slabs=gq, w_d_slabs=dq)
        assert torch.equal(idq, ids) and torch.equal(yq, y)
    xn = fused_ops.rms_norm(x, b["norm_w"], W.EPS)
    for gq, dq in ((wq, None), (None, wd), (wq, wd)):
        y2 = fused_moe.fused_moe_prefill(xn, b["w_gu"], b["w_d"], ids, wts, residual=x, w_gu_slabs=gq, w_d_slabs=dq)
        assert torch.equal(y2, y)


def test_prefill_slab_copy_on_ragged_shapes():
    """The slab copy with a partial column tile (inter 208) on hidden 1536, 64- and 128-pair blocks."""
    H, I, E, K = 1536, 208, 32, 6
    w_gu = W.normal((E + 1, 2 * I, H), 0.02, 143, DEV)
    w_d = W.normal((E + 1, H, I), 0.02, 144, DEV)
    wq = fused_moe.gate_up_slabs(w_gu)
    g = torch.Generator().manual_seed(145)
    for n in (60, 700):
        sel = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(n)])
        ids = torch.cat([sel, torch.full((n, 1), E)], 1).to(DEV)
        wts = torch.cat([torch.rand(n, K, generator=g), torch.ones(n, 1)], 1).to(DEV)
        x = W.normal((n, H), 1.0, 146 + n, DEV)
        y = fused_moe.fused_moe_prefill(x, w_gu, w_d, ids, wts)
        assert torch.equal(fused_moe.fused_moe_prefill(x, w_gu, w_d, ids, wts, w_gu_slabs=wq), y), n


def test_prefill_down_slab_copy_on_ragged_shapes():
    """The down slab copy with a partial row tile of W_d (hidden 1544 = 12 x 128 + 8; hidden is not a multiple
    of 64, so w_gu has no copy) at inter 192, 64- and 128-pair blocks."""
    H, I, E, K = 1544, 192, 32, 6
    w_gu = W.normal((E + 1, 2 * I, H), 0.02, 150, DEV)
    w_d = W.normal((E + 1, H, I), 0.02, 151, DEV)
    wd = fused_moe.down_slabs(w_d)
    g = torch.Generator().manual_seed(152)
    for n in (60, 700):
        sel = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(n)])
        ids = torch.cat([sel, torch.full((n, 1), E)], 1).to(DEV)
        wts = torch.cat([torch.rand(n, K, generator=g), torch.ones(n, 1)], 1).to(DEV)
        x = W.normal((n, H), 1.0, 153 + n, DEV)
        y = fused_moe.fused_moe_prefill(x, w_gu, w_d, ids, wts)
        assert torch.equal(fused_moe.fused_moe_prefill(x, w_gu, w_d, ids, wts, w_d_slabs=wd), y), n
    close(y, O.moe(x.cpu(), w_gu.cpu(), w_d.cpu(), ids.cpu(), wts.cpu()))


def test_prefill_equals_per_token_decode(blk):
    b, _ = blk
    x = W.tokens(24, seed=95, device=DEV)
    xn, ids, wts = _route_tokens(b, x)
    y = fused_moe.fused_moe_prefill(xn, b["w_gu"], b["w_d"], ids, wts)
    for t in range(0, 24, 5):
        yt = fused_moe.fused_moe_decode(xn[t:t + 1], b["w_gu"], b["w_d"], ids[t], wts[t])
        close(yt, y[t:t + 1], rtol=1e-2, atol=8e-3)


def test_moe_block_forward(blk):
    b, cpu = blk
    for n, bias in ((1, None), (512, W.ragged_bias(device=DEV))):
        x = W.tokens(n, seed=99, device=DEV)
        y = W.moe_block_forward(x, b, bias)
        xn, ids, wts = _route_tokens(b, x, bias)
        close(y, _oracle_moe(cpu, xn, ids, wts, residual=x.cpu()))


# ------------------------------------------------------------- the reference's torch int8 path (engine.py)

@pytest.fixture(scope="module")
def fallback_weights(blk):
    """The int8 experts dequantised as the reference's unfused int8 prefill does it (engine.py:478-479:
    (q.half() * s.half()).to(bf16)), once, on the CPU."""
    _, cpu = blk
    d_gu = (cpu["q_gu"].half() * cpu["s_gu"][:, :, None].half()).to(BF)
    d_d = (cpu["q_d"].half() * cpu["s_d"][:, :, None].half()).to(BF)
    return d_gu, d_d


@pytest.mark.parametrize("n", [1, 2, 4, 8, 100, 512])
def test_int8_matches_the_reference_torch_int8_path(blk, fallback_weights, n):
    """int8 decode (1..8 tokens: the decode kernels) and int8 prefill (100, 512 tokens: align + grouped MFMA)
    against the reference's own torch int8 path (engine.py:455-486, restated by O.moe_int8_fallback): experts
    dequantised with fp16 rounding, per-expert bf16 products, fp32 sum over slots. The HIP kernels apply the
    row scale to the fp32 accumulator instead, so the two differ by weight rounding only (bf16 tolerance)."""
    b, cpu = blk
    x = W.tokens(n, seed=160 + n, device=DEV)
    xn, ids, wts = _route_tokens(b, x, W.ragged_bias(device=DEV) if n == 512 else None)
    y = fused_moe.fused_moe_prefill(xn, b["q_gu"], b["q_d"], ids, wts, s_gu=b["s_gu"], s_d=b["s_d"])
    d_gu, d_d = fallback_weights
    ref = O.moe(xn.cpu(), d_gu, d_d, ids.cpu(), wts.cpu())  # = O.moe_int8_fallback, dequantised once
    close(y, ref)
    if n == 100:
        torch.testing.assert_close(ref, O.moe_int8_fallback(xn.cpu(), cpu["q_gu"], cpu["q_d"], cpu["s_gu"], cpu["s_d"],
                                                            ids.cpu(), wts.cpu()), rtol=0, atol=0)


# -------------------------------------------------------------------------------------------- small linear

@pytest.mark.parametrize("M", [1, 2, 6, 16, 20, 64])
@pytest.mark.parametrize("KN", [(2048, 2048), (2048, 256), (896, 1152), (4864, 896), (256, 77), (1024, 130),
                                (6144, 64), (8192, 33), (9216, 40)])
def test_small_linear(M, KN):
    """Every launch shape: one pass per row with 16 / 32 / 64 lanes per row and 4..16 chunks per lane (K up to
    8192, norm fused), and the multi-pass kernel with its separate norm kernel (K = 9216). More than 16 rows
    (20, 64) are checked against the reference's torch path for that case (fastlinear.py:151-160: the norm
    rounded once), the others against its Triton kernel's rounding."""
    K, N = KN
    x = W.normal((M, K), 1.0, 100 + M, DEV)
    w = W.normal((N, K), 0.02, 101, DEV)
    bias = W.normal((N,), 1.0, 102, DEV)
    r = W.normal((M, N), 1.0, 103, DEV)
    for act in (0, 1, 2):
        y = fastlinear.small_linear(x, w, bias, act=act, residual=r)
        close(y, O.small_linear(x.cpu(), w.cpu(), bias.cpu(), act, r.cpu()))
    g = W.normal((K,), 0.02, 104, DEV, mean=1.0)
    y = fastlinear.small_linear(x, w, norm=(g, 1e-6))
    close(y, O.small_linear(x.cpu(), w.cpu(), norm=(g.cpu(), 1e-6)))


def test_small_linear_lm_head_shape():
    x = W.normal((1, 2048), 1.0, 110, DEV)
    w = W.normal((126464, 2048), 0.02, 111, DEV)
    y = fastlinear.small_linear(x, w)
    close(y, O.small_linear(x.cpu(), w.cpu()))


# --------------------------------------------------------------------------------------------- hipGraph

def test_decode_step_graph_replays_match_eager(blk):
    b, _ = blk
    x = W.tokens(1, seed=120, device=DEV)
    logits = torch.empty(64, device=DEV)
    ids = torch.empty(7, device=DEV, dtype=torch.long)
    wts = torch.empty(7, device=DEV)
    a_buf = torch.empty(7, 1408, device=DEV, dtype=BF)
    out = torch.empty(1, 2048, device=DEV, dtype=BF)

    def step():
        xn = fused_ops.rms_norm(x, b["norm_w"], W.EPS)
        fused_ops.moe_route(xn, b["w32"], None, 1, 1, 6, 1.0, logits, ids, wts, scoring="softmax")
        fused_moe.fused_moe_decode(xn, b["w_gu"], b["w_d"], ids, wts, a_buf=a_buf, out=out, residual=x)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step()
    for i in range(4):
        out.zero_()
        x.add_(0)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
    x.copy_(W.tokens(1, seed=121, device=DEV))  # new input through the same graph
    g.replay()
    torch.cuda.synchronize()
    from_graph = out.clone()
    step()
    torch.cuda.synchronize()
    assert torch.equal(out, from_graph) and not torch.equal(from_graph, eager)


def test_gpu_argument_errors():
    x = torch.zeros(1, 64, device=DEV, dtype=BF)
    with pytest.raises(ValueError, match="M=17"):
        _mingmoe.check(_mingmoe.load().mm_small_linear(_mingmoe.ptr(x), 17, 64, 64, _mingmoe.ptr(x), 64, 64, None, 0,
                                                       None, 0, None, 0.0, None, _mingmoe.ptr(x), 64,
                                                       _mingmoe.stream_of(x)), "small_linear")
    with pytest.raises(ValueError, match="pairs"):
        fused_moe.fused_moe_decode(torch.zeros(9, 2048, device=DEV, dtype=BF), torch.zeros(2, 16, 2048, device=DEV,
                                   dtype=BF), torch.zeros(2, 2048, 8, device=DEV, dtype=BF),
                                   torch.zeros(9, 8, device=DEV, dtype=torch.long), torch.zeros(9, 8, device=DEV))


def test_block_decode_graph_replays_follow_new_inputs(blk):
    """The fused decode block captured once and replayed on new token rows: every replay equals an eager
    call on the same rows."""
    b, _ = blk
    x = W.tokens(2, seed=130, device=DEV)
    logits = torch.empty(2, 64, device=DEV)
    ids = torch.empty(2, 7, device=DEV, dtype=torch.long)
    wts = torch.empty(2, 7, device=DEV)
    a_buf = torch.empty(14, 1408, device=DEV, dtype=BF)
    out = torch.empty(2, 2048, device=DEV, dtype=BF)
    ws = torch.empty(2, 2048, device=DEV, dtype=BF)

    def step():
        fused_moe.moe_block_decode(x, b["norm_w"], W.EPS, b["w32"], b["w_gu"], b["w_d"], top_k=6, logits=logits,
                                   ids=ids, wts=wts, a_buf=a_buf, out=out, workspace=ws)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step()
    for i in range(4):
        x.copy_(W.tokens(2, seed=131 + i, device=DEV))
        want, want_ids, _, _ = fused_moe.moe_block_decode(x, b["norm_w"], W.EPS, b["w32"], b["w_gu"], b["w_d"],
                                                          top_k=6)
        torch.cuda.synchronize()
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(ids, want_ids) and torch.equal(out, want), f"replay {i}"
