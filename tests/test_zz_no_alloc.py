"""GPU check of mm_moe_block_decode_noalloc, the decode MoE block whose scratch lives in a static device array.

Called through the C ABI, it must give exactly what mm_moe_block_decode gives with caller scratch (same
kernels): logits, ids, weights and outputs bit for bit, on two calls in a row, the second with fewer tokens
(the array keeps the first call's contents), for bf16 and int8 experts at the benchmarked block shape."""
import ctypes

import pytest
import torch

import _mingmoe as mm
import workloads as W

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def blk():
    b = W.block(seed=0, device=DEV)
    W.quantize_block(b, torch.bfloat16)
    torch.cuda.synchronize()
    return b


def _outputs(n, E, NK, H):
    return (torch.full((n, E), float("nan"), device=DEV), torch.full((n, NK), -7, device=DEV, dtype=torch.int64),
            torch.full((n, NK), float("nan"), device=DEV), torch.zeros(n, H, device=DEV, dtype=torch.bfloat16))


def _call(lib, noalloc, x, b, ex, top_k, outs, int8):
    n, H = x.shape
    E, NK = b["w32"].shape[0], top_k + 1
    logits, ids, wts, y = outs
    common = (mm.ptr(x), n, H, mm.ptr(b["norm_w"]), W.EPS, mm.ptr(b["w32"]), E, None, mm.MM_SCORE_SOFTMAX, 1, 1,
              top_k, 1.0, ctypes.byref(ex), mm.ptr(logits), mm.ptr(ids), mm.MM_INT64, mm.ptr(wts))
    stream = mm.stream_of(x)
    if noalloc:
        print(f"[no_alloc] noalloc n={n} int8={int8}", flush=True)
        rc = lib.mm_moe_block_decode_noalloc(*common, 1, mm.ptr(y), H, stream)
    else:
        print(f"[no_alloc] caller-scratch n={n} int8={int8}", flush=True)
        a_buf = torch.empty(n * NK, ex.inter, device=DEV, dtype=torch.bfloat16)
        ws = torch.empty(n, H, device=DEV, dtype=torch.bfloat16)
        rc = lib.mm_moe_block_decode(*common, mm.ptr(a_buf), mm.ptr(ws), 1, mm.ptr(y), H, stream)
    mm.check(rc, "moe_block_decode" + ("_noalloc" if noalloc else ""))
    torch.cuda.synchronize()


@pytest.mark.parametrize("int8", [False, True])
def test_noalloc_matches_caller_scratch_twice(blk, int8):
    lib = mm.load()
    ex = mm.experts(blk["q_gu"], blk["q_d"], blk["s_gu"], blk["s_d"]) if int8 else mm.experts(blk["w_gu"], blk["w_d"])
    E, H, top_k = W.EXPERTS, W.HIDDEN, W.TOP_K
    assert lib.mm_moe_block_decode_noalloc_bytes(8, top_k, H, W.INTER) <= 2 * 1024 * 1024
    for n, seed in ((8, 901), (1, 902)):  # the second call is smaller: it must not see the first call's rows
        x = W.tokens(n, seed=seed + (10 if int8 else 0), device=DEV)
        want = _outputs(n, E, top_k + 1, H)
        got = _outputs(n, E, top_k + 1, H)
        _call(lib, False, x, blk, ex, top_k, want, int8)
        _call(lib, True, x, blk, ex, top_k, got, int8)
        for name, g, w in zip(("logits", "ids", "wts", "y"), got, want):
            assert torch.equal(g, w), (name, n, int8)
        assert torch.isfinite(got[3].float()).all()


_CAPTURE_FIRST = r"""
import ctypes, sys
sys.path[:0] = [sys.argv[1], sys.argv[2]]
import torch
import _mingmoe as mm
import workloads as W
lib = mm.load()
dev = "cuda"
H, I, E, K = 512, 256, 16, 4
b = W.block(seed=5, device=dev, hidden=H, inter=I, experts=E)
ex = mm.experts(b["w_gu"], b["w_d"])
x = W.tokens(2, seed=6, device=dev, hidden=H)
def bufs():
    return (torch.empty(2, E, device=dev), torch.empty(2, K + 1, device=dev, dtype=torch.int64),
            torch.empty(2, K + 1, device=dev), torch.zeros(2, H, device=dev, dtype=torch.bfloat16))
def common(o):
    return (mm.ptr(x), 2, H, mm.ptr(b["norm_w"]), W.EPS, mm.ptr(b["w32"]), E, None, mm.MM_SCORE_SOFTMAX, 1, 1, K, 1.0,
            ctypes.byref(ex), mm.ptr(o[0]), mm.ptr(o[1]), mm.MM_INT64, mm.ptr(o[2]))
got, want = bufs(), bufs()
s = torch.cuda.Stream()
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
print("[capture-first] capturing the first noalloc call of this process", flush=True)
with torch.cuda.graph(g, stream=s):
    mm.check(lib.mm_moe_block_decode_noalloc(*common(got), 1, mm.ptr(got[3]), H, mm.stream_of(x)), "noalloc")
a_buf = torch.empty(2 * (K + 1), I, device=dev, dtype=torch.bfloat16)
ws = torch.empty(2, H, device=dev, dtype=torch.bfloat16)
mm.check(lib.mm_moe_block_decode(*common(want), mm.ptr(a_buf), mm.ptr(ws), 1, mm.ptr(want[3]), H, mm.stream_of(x)),
         "caller scratch")
torch.cuda.synchronize()
for rep in range(3):
    for t in got:
        t.zero_()
    g.replay()
    torch.cuda.synchronize()
    for name, a, w in zip(("logits", "ids", "wts", "y"), got, want):
        assert torch.equal(a, w), (rep, name)
    z = (x.float() * 2).sum()  # eager work between the replays
    torch.cuda.synchronize()
print("[capture-first] ok", flush=True)
"""


def test_noalloc_first_call_under_graph_capture():
    """A process whose first call of the entry point is made under hipGraph capture (the scratch address is looked up
    on that call): the graph's replays equal the caller-scratch entry point's eager result, every replay."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _CAPTURE_FIRST, os.path.join(root, "ming-voice_amd"), root],
                       capture_output=True, text=True, timeout=240)
    print(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0 and "[capture-first] ok" in r.stdout


def test_noalloc_rejects_oversize_shape(blk):
    lib = mm.load()
    ex = mm.experts(blk["w_gu"], blk["w_d"])
    ex.inter = 1 << 15  # 8 tokens x 7 slots x 32768 x 2 bytes > the 2 MiB array (checked before any launch)
    P = ctypes.c_void_p(16)
    rc = lib.mm_moe_block_decode_noalloc(P, 8, W.HIDDEN, P, W.EPS, P, W.EXPERTS, None, mm.MM_SCORE_SOFTMAX, 1, 1,
                                         W.TOP_K, 1.0, ctypes.byref(ex), P, P, mm.MM_INT64, P, 1, P, W.HIDDEN, None)
    assert rc == mm.MM_ERR_ARG and "maximum" in mm.last_error()
