"""The oracle against committed golden vectors (tests/golden/moe_small.npz, written by
tests/golden/make_fixtures.py from a scalar Python / float64 brute force that shares no code with the
oracle). Each check fails on the plausible oracle mistakes: a wrong pad or block count (align), a wrong
scale or rounding mode (quantize), a wrong tie order or normaliser (select), a dropped rounding point,
swapped gate/up halves or a missing residual (moe)."""
import os

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "moe_small.npz")
BF = torch.bfloat16


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX) as z:
        return {k: z[k] for k in z.files}


def test_fixture_inputs_are_bf16_values(fx):
    for k in ("quant_w", "moe_x", "moe_w_gu", "moe_w_d"):
        v = torch.from_numpy(fx[k])
        assert torch.equal(v.to(BF).float(), v), k


@pytest.mark.parametrize("bm", [4, 64])
def test_align_matches_golden(fx, bm):
    s, b, nb, off = O.align_blocks(fx["align_flat"], 9, bm)
    assert np.array_equal(s, fx[f"align_sorted_bm{bm}"])
    assert np.array_equal(b, fx[f"align_bexp_bm{bm}"])
    assert nb == fx[f"align_bexp_bm{bm}"].size
    assert np.array_equal(off, fx[f"align_offsets_bm{bm}"])


def test_quantize_matches_golden(fx):
    q, s = O.quantize_rows_int8(torch.from_numpy(fx["quant_w"]).to(BF))
    assert torch.equal(q, torch.from_numpy(fx["quant_q"]))
    assert torch.equal(s, torch.from_numpy(fx["quant_s"]))
    assert fx["quant_q"][4, :4].tolist() == [127, 2, -4, 0]  # the half-to-even row


def test_softmax_select_matches_golden(fx):
    ids, wts = O.router_select(torch.from_numpy(fx["sel_logits"]), torch.from_numpy(fx["sel_bias"]),
                               scoring="softmax", top_k=3)
    assert torch.equal(ids, torch.from_numpy(fx["sel_ids"]))
    torch.testing.assert_close(wts, torch.from_numpy(fx["sel_wts"]), rtol=1e-6, atol=1e-6)


def test_moe_matches_golden(fx):
    x = torch.from_numpy(fx["moe_x"]).to(BF)
    y, a = O.moe(x, torch.from_numpy(fx["moe_w_gu"]).to(BF), torch.from_numpy(fx["moe_w_d"]).to(BF),
                 torch.from_numpy(fx["moe_ids"]), torch.from_numpy(fx["moe_wts"]), residual=x, return_a=True)
    torch.testing.assert_close(a.float(), torch.from_numpy(fx["moe_a"]), rtol=2e-2, atol=1e-2)
    torch.testing.assert_close(y.float(), torch.from_numpy(fx["moe_y"]), rtol=2e-2, atol=1e-2)
    # most outputs agree to the bit: a dropped rounding point would move far more than a few of them
    assert (a.float() == torch.from_numpy(fx["moe_a"])).float().mean() > 0.9
    assert (y.float() == torch.from_numpy(fx["moe_y"])).float().mean() > 0.9


def test_int8_block_matches_golden(fx):
    """The same block on int8 experts with bf16 row scales: the quantiser and the int8 MoE restated by the
    oracle reproduce the brute force's codes, scales and outputs."""
    w_gu = torch.from_numpy(fx["moe_w_gu"]).to(BF)
    w_d = torch.from_numpy(fx["moe_w_d"]).to(BF)
    q_gu, s_gu = O.quantize_rows_int8(w_gu, scale_dtype=BF)
    q_d, s_d = O.quantize_rows_int8(w_d, scale_dtype=BF)
    assert torch.equal(q_gu, torch.from_numpy(fx["moe_q_gu"])) and torch.equal(q_d, torch.from_numpy(fx["moe_q_d"]))
    assert torch.equal(s_gu.float(), torch.from_numpy(fx["moe_s_gu"]))
    assert torch.equal(s_d.float(), torch.from_numpy(fx["moe_s_d"]))
    x = torch.from_numpy(fx["moe_x"]).to(BF)
    y, a = O.moe(x, q_gu, q_d, torch.from_numpy(fx["moe_ids"]), torch.from_numpy(fx["moe_wts"]), s_gu, s_d,
                 residual=x, return_a=True)
    torch.testing.assert_close(a.float(), torch.from_numpy(fx["moe_a_i8"]), rtol=2e-2, atol=1e-2)
    torch.testing.assert_close(y.float(), torch.from_numpy(fx["moe_y_i8"]), rtol=2e-2, atol=1e-2)
    assert (y.float() == torch.from_numpy(fx["moe_y_i8"])).float().mean() > 0.9
