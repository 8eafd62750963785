"""The HIP kernels against the committed golden vectors (tests/golden/moe_small.npz): block alignment and
int8 quantisation bit for bit, softmax selection (ids exact), and one MoE block (H=64, I=32, 4 routed
experts + shared, top-2 + shared) through the decode and prefill paths. The vectors come from a scalar
brute force that shares no code with the kernels or the oracle."""
import ctypes
import os

import numpy as np
import pytest
import torch

import _mingmoe as mm
import fused_moe

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16
FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "moe_small.npz")


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX) as z:
        return {k: torch.from_numpy(z[k]) for k in z.files}


def _close(got, want):
    torch.testing.assert_close(got.float().cpu(), want.float(), rtol=2e-2, atol=1e-2)


@pytest.mark.parametrize("bm", [4, 64])
def test_align_golden(fx, bm):
    off = torch.empty(10, dtype=torch.int32, device=DEV)
    s, b, nb = fused_moe._align_blocks(fx["align_flat"].to(DEV), 9, bm, expert_offsets=off)
    assert nb == fx[f"align_bexp_bm{bm}"].numel()
    assert torch.equal(s.cpu(), fx[f"align_sorted_bm{bm}"]) and torch.equal(b.cpu(), fx[f"align_bexp_bm{bm}"])
    assert torch.equal(off.cpu(), fx[f"align_offsets_bm{bm}"])


def test_quantize_golden(fx):
    q, s = fused_moe.quantize_rows_int8(fx["quant_w"].to(BF).to(DEV), scale_dtype=torch.float32)
    assert torch.equal(q.cpu(), fx["quant_q"]) and torch.equal(s.cpu(), fx["quant_s"])


def test_softmax_select_golden(fx):
    logits = fx["sel_logits"].to(DEV)
    bias = fx["sel_bias"].to(DEV)
    N, E = logits.shape
    ids = torch.empty(N, 4, dtype=torch.int64, device=DEV)
    wts = torch.empty(N, 4, dtype=torch.float32, device=DEV)
    lib = mm.load()
    mm.check(lib.mm_router_select(mm.ptr(logits), N, E, mm.ptr(bias), mm.MM_SCORE_SOFTMAX, 1, 1, 3,
                                  ctypes.c_float(1.0), 1, mm.ptr(ids), mm.MM_INT64, mm.ptr(wts), 4,
                                  mm.stream_of(logits)), "router_select")
    torch.cuda.synchronize()
    assert torch.equal(ids.cpu(), fx["sel_ids"])
    torch.testing.assert_close(wts.cpu(), fx["sel_wts"], rtol=1e-5, atol=1e-6)


def test_decode_golden(fx):
    x = fx["moe_x"].to(BF).to(DEV)
    w_gu, w_d = fx["moe_w_gu"].to(BF).to(DEV), fx["moe_w_d"].to(BF).to(DEV)
    ids, wts = fx["moe_ids"].to(DEV), fx["moe_wts"].to(DEV)
    a_buf = torch.empty(ids.numel(), w_d.shape[-1], device=DEV, dtype=BF)
    y = fused_moe.fused_moe_decode(x, w_gu, w_d, ids, wts, a_buf=a_buf, residual=x)
    _close(a_buf, fx["moe_a"])
    _close(y, fx["moe_y"])
    y1 = fused_moe.fused_moe_decode(x[1:2], w_gu, w_d, ids[1], wts[1], residual=x[1:2])
    _close(y1, fx["moe_y"][1:2])


@pytest.mark.parametrize("reps", [1, 4])
def test_prefill_golden(fx, reps):
    x = fx["moe_x"].to(BF).repeat(reps, 1).to(DEV)
    w_gu, w_d = fx["moe_w_gu"].to(BF).to(DEV), fx["moe_w_d"].to(BF).to(DEV)
    ids, wts = fx["moe_ids"].repeat(reps, 1).to(DEV), fx["moe_wts"].repeat(reps, 1).to(DEV)
    y = fused_moe.fused_moe_prefill(x, w_gu, w_d, ids, wts, residual=x)
    _close(y, fx["moe_y"].repeat(reps, 1))


def _int8_block(fx):
    return (fx["moe_q_gu"].to(DEV), fx["moe_s_gu"].to(BF).to(DEV), fx["moe_q_d"].to(DEV),
            fx["moe_s_d"].to(BF).to(DEV))


def test_quantize_bf16_scales_golden(fx):
    q, s = fused_moe.quantize_rows_int8(fx["moe_w_gu"].to(BF).to(DEV), scale_dtype=BF)
    assert torch.equal(q.cpu(), fx["moe_q_gu"]) and torch.equal(s.float().cpu(), fx["moe_s_gu"])


def test_decode_int8_golden(fx):
    x = fx["moe_x"].to(BF).to(DEV)
    q_gu, s_gu, q_d, s_d = _int8_block(fx)
    ids, wts = fx["moe_ids"].to(DEV), fx["moe_wts"].to(DEV)
    a_buf = torch.empty(ids.numel(), q_d.shape[-1], device=DEV, dtype=BF)
    y = fused_moe.fused_moe_decode(x, q_gu, q_d, ids, wts, a_buf=a_buf, s_gu=s_gu, s_d=s_d, residual=x)
    _close(a_buf, fx["moe_a_i8"])
    _close(y, fx["moe_y_i8"])


@pytest.mark.parametrize("reps", [1, 4])
def test_prefill_int8_golden(fx, reps):
    x = fx["moe_x"].to(BF).repeat(reps, 1).to(DEV)
    q_gu, s_gu, q_d, s_d = _int8_block(fx)
    ids, wts = fx["moe_ids"].repeat(reps, 1).to(DEV), fx["moe_wts"].repeat(reps, 1).to(DEV)
    y = fused_moe.fused_moe_prefill(x, q_gu, q_d, ids, wts, s_gu=s_gu, s_d=s_d, residual=x)
    _close(y, fx["moe_y_i8"].repeat(reps, 1))
