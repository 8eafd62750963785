"""Small-M linear on a hand-written gfx950 HIP kernel (drop-in for the reference fastlinear.py):
y = act(norm?(x) @ W^T + b) + residual, bandwidth-bound GEMV for decode-sized activations.

The reference tunes Triton block configs per shape and caches them in CACHE_FILE; the HIP kernel picks
its launch shape from (M, K) alone, so nothing is tuned: `_best` stays empty, `save_cache()` has nothing
to write, and shapes never need tuning before graph capture. More than 16 rows run as 16-row pieces of the
same kernel with the rounding points of the reference's torch path for that case (fastlinear.py:151-160):
the same as the kernel's except the RMSNorm prologue, which F.rms_norm rounds once, bf16(x * rstd * g),
where the Triton kernel rounds twice, bf16(bf16(x * rstd) * g).
"""
import json
import os
import time

import torch

import _mingmoe as _mm

__all__ = ["small_linear", "save_cache", "CACHE_FILE"]

CACHE_FILE = os.path.join(os.environ.get("MING_DATA_DIR") or os.path.dirname(os.path.abspath(__file__)),
                          ".fastlinear_tuning.json")
MAX_M = 16
ACT_NONE, ACT_GELU_TANH, ACT_SILU = 0, 1, 2

_best: dict = {}
_dirty = False


def save_cache():
    """Writes tuned configs to CACHE_FILE when there are new ones (never, for the HIP kernel)."""
    global _dirty
    if not _dirty:
        return
    try:
        with open(CACHE_FILE, "w") as f:
            json.dump({json.dumps(list(k)): v for k, v in _best.items()}, f, indent=0)
        _dirty = False
    except OSError:
        pass


def _graph_time(fn, reps=20, inner=40):
    """Seconds per call of fn, captured `inner` times in one hipGraph and replayed `reps` times."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for _ in range(inner):
                fn()
        g.replay()
        s.synchronize()
        t = time.perf_counter()
        for _ in range(reps):
            g.replay()
        s.synchronize()
    torch.cuda.current_stream().wait_stream(s)
    return (time.perf_counter() - t) / reps / inner


def _launch(lib, x2, w, b, r2, act, norm, y, xn):
    M, K = x2.shape
    N = w.shape[0]
    g, eps = norm if norm is not None else (None, 0.0)
    _mm.check(lib.mm_small_linear(_mm.ptr(x2), M, K, x2.stride(0), _mm.ptr(w), N, w.stride(0), _mm.ptr(b), int(act),
                                  _mm.ptr(r2), r2.stride(0) if r2 is not None else 0, _mm.ptr(g), float(eps or 0.0),
                                  _mm.ptr(xn), _mm.ptr(y), y.stride(0), _mm.stream_of(x2)), "small_linear")


def small_linear(x, w, b=None, act=0, residual=None, out=None, norm=None):
    """x: [..., K] bf16; w: [N, K] contiguous; act: 0 none, 1 gelu-tanh, 2 silu;
    residual: tensor broadcastable as [..., N] added after the activation;
    norm: (gamma, eps) applies RMSNorm to x first (fused)."""
    g = norm[0] if norm is not None else None
    _mm.require_gpu(x, w, b, residual, out, g)
    shape = x.shape
    K = shape[-1]
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:  # rows strided by a 16-byte multiple pass as is
        x2 = x2.contiguous()
    M, N = x2.shape[0], w.shape[0]
    for name, t in (("x", x2), ("w", w), ("b", b), ("residual", residual), ("norm gamma", g)):
        if t is not None and t.dtype != torch.bfloat16:
            raise ValueError(f"small_linear: {name} must be bf16 (got {t.dtype})")
    if w.dim() != 2 or w.shape[1] != K or w.stride(1) != 1:
        raise ValueError(f"small_linear: w must be [N, {K}] with a contiguous last dim")
    if b is not None and not b.is_contiguous():
        b = b.contiguous()
    if g is not None and not g.is_contiguous():
        g = g.contiguous()
        norm = (g, norm[1])
    r2 = None
    if residual is not None:
        r2 = residual.reshape(-1, N)
        if r2.shape[0] != M:
            r2 = residual.expand(*shape[:-1], N).reshape(M, N)
        if not r2.is_contiguous():
            r2 = r2.contiguous()
    y = torch.empty(M, N, device=x.device, dtype=x.dtype) if out is None else out.view(M, N)
    # the library fuses the norm into the GEMV for K <= 8192 and needs the scratch row only beyond that
    xn = torch.empty(min(M, MAX_M), K, device=x.device, dtype=torch.bfloat16) if norm is not None and K > 8192 else None
    if M > MAX_M and norm is not None:
        act = int(act) | _mm.MM_NORM_ROUND_ONCE  # F.rms_norm's single rounding (fastlinear.py:151-153)
    lib = _mm.load()
    with _mm.on_device(x):
        for m0 in range(0, M, MAX_M):
            m1 = min(M, m0 + MAX_M)
            _launch(lib, x2[m0:m1], w, b, r2[m0:m1] if r2 is not None else None, act, norm, y[m0:m1], xn)
    return y.reshape(*shape[:-1], N)
