"""The prefill copies of the expert stacks bound to their stacks (fused_moe.prefill_copies, PREFILL_COPIES = "auto").

The reference's engine calls fused_moe_prefill(x, w_gu, w_d, ids, wts) on its stacks (engine.py:300-310) and its
loader writes checkpoint tensors into views of those stacks (engine.py:150-188, direct_load.py:109-132). These tests
check that the unchanged call finds or makes the copies, that outputs equal the row layout's bit for bit, and that a
copy never outlives a write into its stack: passed explicitly it is refused, found in the registry it is remade
(eagerly) or refused (under graph capture)."""
import pytest
import torch

import fused_moe
import workloads as W
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
H, I, E, K = 1024, 384, 16, 4


def _stacks(seed):
    return W.normal((E + 1, 2 * I, H), 0.02, seed, DEV), W.normal((E + 1, H, I), 0.02, seed + 1, DEV)


def _pairs(n, seed):
    g = torch.Generator().manual_seed(seed)
    sel = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(n)])
    ids = torch.cat([sel, torch.full((n, 1), E)], 1).to(DEV)
    wts = torch.cat([torch.rand(n, K, generator=g), torch.ones(n, 1)], 1).to(DEV)
    return W.normal((n, H), 1.0, seed + 2, DEV), ids, wts


def _rows(x, w_gu, w_d, ids, wts):
    """The same call on the row layout (the registry switched off for it)."""
    prev, fused_moe.PREFILL_COPIES = fused_moe.PREFILL_COPIES, "off"
    try:
        return fused_moe.fused_moe_prefill(x, w_gu, w_d, ids, wts)
    finally:
        fused_moe.PREFILL_COPIES = prev


def test_engine_call_makes_and_reuses_the_copies(monkeypatch):
    print("[prefill copies] engine call, auto", flush=True)
    w_gu, w_d = _stacks(200)
    x, ids, wts = _pairs(300, 203)
    monkeypatch.setattr(fused_moe, "PREFILL_COPIES", "auto")
    want = _rows(x, w_gu, w_d, ids, wts)
    n0 = len(fused_moe._registry)
    y = fused_moe.fused_moe_prefill(x, w_gu, w_d, ids, wts)  # the reference's call, unchanged
    assert len(fused_moe._registry) == n0 + 2
    gq, dq = fused_moe._copies_for(w_gu, w_d)
    assert gq._mm_source[4] == w_gu._version and dq._mm_source[4] == w_d._version
    assert torch.equal(y, want)
    y2 = fused_moe.fused_moe_prefill(x, w_gu, w_d, ids, wts)
    assert torch.equal(y2, want) and fused_moe._copies_for(w_gu, w_d)[0] is gq  # found, not made again
    torch.testing.assert_close(y.float().cpu(), O.moe(x.cpu(), w_gu.cpu(), w_d.cpu(), ids.cpu(), wts.cpu()).float(),
                               rtol=2e-2, atol=1e-2)
    del w_gu, w_d, gq, dq
    assert len(fused_moe._registry) == n0  # the copies go with their stacks


@pytest.mark.parametrize("write", ["loader_copy", "in_place_op"])
def test_write_into_the_stack_after_the_copy(monkeypatch, write):
    """A write into w_gu after the copies were made: the explicit copy is refused, the registered one is remade on the
    next eager call, and the outputs follow the new weights (equal to the row layout on them)."""
    print(f"[prefill copies] write {write}", flush=True)
    monkeypatch.setattr(fused_moe, "PREFILL_COPIES", "registered")
    w_gu, w_d = _stacks(210)
    x, ids, wts = _pairs(200, 213)
    gq, dq = fused_moe.prefill_copies(w_gu, w_d)
    y0 = fused_moe.fused_moe_prefill(x, w_gu, w_d, ids, wts)
    assert torch.equal(y0, _rows(x, w_gu, w_d, ids, wts))
    with torch.no_grad():
        if write == "loader_copy":  # what direct_load does with a checkpoint tensor: copy_ into a view of the stack
            w_gu[3, :I].copy_(W.normal((I, H), 0.05, 214, DEV))
        else:
            w_gu[E].mul_(2.0)
    with pytest.raises(ValueError, match="stale"):
        fused_moe.fused_moe_prefill(x, w_gu, w_d, ids, wts, w_gu_slabs=gq, w_d_slabs=dq)
    y1 = fused_moe.fused_moe_prefill(x, w_gu, w_d, ids, wts)
    assert gq._mm_source[4] == w_gu._version  # remade in place
    assert torch.equal(y1, _rows(x, w_gu, w_d, ids, wts))
    assert not torch.equal(y1, y0)
    assert torch.equal(gq, fused_moe.gate_up_slabs(w_gu))


def test_stale_copy_under_capture_is_refused(monkeypatch):
    print("[prefill copies] stale under capture", flush=True)
    monkeypatch.setattr(fused_moe, "PREFILL_COPIES", "auto")
    w_gu, w_d = _stacks(220)
    x, ids, wts = _pairs(100, 223)
    sc = fused_moe.PrefillScratch(100, K + 1, E + 1, H, I, DEV)
    fused_moe.fused_moe_prefill(x, w_gu, w_d, ids, wts, scratch=sc)  # eager: copies made
    with torch.no_grad():
        w_d[0].add_(1.0)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="prefill_copies"):
        with torch.cuda.graph(g, stream=s):
            fused_moe.fused_moe_prefill(x, w_gu, w_d, ids, wts, scratch=sc)
    torch.cuda.synchronize()
    fused_moe.prefill_copies(w_gu, w_d)  # remade: capture now takes the copies
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=s):
        y = fused_moe.fused_moe_prefill(x, w_gu, w_d, ids, wts, scratch=sc)
    want = _rows(x, w_gu, w_d, ids, wts).clone()
    for _ in range(2):
        y.zero_()
        g2.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want)


def test_copy_of_another_stack_is_refused():
    w_gu, w_d = _stacks(230)
    other, _ = _stacks(232)
    x, ids, wts = _pairs(50, 233)
    with pytest.raises(ValueError, match="another stack"):
        fused_moe.fused_moe_prefill(x, w_gu, w_d, ids, wts, w_gu_slabs=fused_moe.gate_up_slabs(other))
    plain = torch.empty_like(fused_moe.gate_up_slabs(w_gu))
    with pytest.raises(ValueError, match="must be made by"):
        fused_moe.fused_moe_prefill(x, w_gu, w_d, ids, wts, w_gu_slabs=plain)
