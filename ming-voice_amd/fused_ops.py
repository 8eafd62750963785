"""RMSNorm and the MoE router on hand-written gfx950 HIP kernels (drop-in for the reference fused_ops.py).

  rms_norm(x, w, eps)            BailingMoeV3RMSNorm in one kernel (fused_ops.py:16-37)
  moe_route(x, w32, bias, ...)   the MoE router for one token, writing into caller buffers
                                 (fused_ops.py:40-103); the shared expert is appended after the top_k
  route(x, w32, ...)             the same router for any number of tokens, returning new tensors
                                 (the multi-token gate of engine.py:326-333)

Scoring modes: "sigmoid" (the thinker router: sigmoid + bias, group-limited top-k, weights from the
unbiased sigmoid scores times `scale`) and "softmax" (softmax over logits + bias, plain top-k, weights
renormalised over the selected experts). Ties pick the lowest expert index.
"""
import torch

import _mingmoe as _mm

__all__ = ["rms_norm", "moe_route", "route"]

_SCORING = {"sigmoid": _mm.MM_SCORE_SIGMOID_GROUP, "softmax": _mm.MM_SCORE_SOFTMAX}


def rms_norm(x, w, eps):
    """y = w * bf16(x * rsqrt(mean(x^2) + eps)) over the last dim, in promote(w.dtype, x.dtype)."""
    _mm.require_gpu(x, w)
    N = x.shape[-1]
    if w.dim() != 1 or w.shape[0] != N:
        raise ValueError(f"rms_norm: weight shape {tuple(w.shape)} does not match the last dim {N}")
    w = w if w.is_contiguous() else w.contiguous()
    x2 = x.reshape(-1, N)
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    out_dtype = torch.promote_types(w.dtype, x.dtype)
    y = torch.empty(x2.shape, dtype=out_dtype, device=x.device)
    lib = _mm.load()
    with _mm.on_device(x):
        _mm.check(lib.mm_rms_norm(_mm.ptr(x2), _mm.dtype_code(x2), x2.shape[0], N, x2.stride(0), _mm.ptr(w),
                                  _mm.dtype_code(w), float(eps), _mm.ptr(y), _mm.dtype_code(y), N, _mm.stream_of(x)),
                  "rms_norm")
    return y.view(x.shape)


def _route_into(x2, w32, bias, n_group, topk_group, top_k, scale, logits, ids, wts, scoring, append_shared, out_stride):
    E, H = w32.shape
    if x2.shape[-1] != H:
        raise ValueError(f"router: x hidden {x2.shape[-1]} does not match w32 {tuple(w32.shape)}")
    if w32.dtype != torch.float32 or not w32.is_contiguous():
        raise ValueError("router: w32 must be a contiguous fp32 [E, H] tensor")
    if bias is not None and (bias.dtype != torch.float32 or bias.numel() != E or not bias.is_contiguous()):
        raise ValueError("router: bias must be a contiguous fp32 [E] tensor")
    if logits.dtype != torch.float32 or logits.numel() < x2.shape[0] * E or not logits.is_contiguous():
        raise ValueError("router: logits buffer must be contiguous fp32 with n_tokens * E elements")
    if wts.dtype != torch.float32:
        raise ValueError("router: weights buffer must be fp32")
    if scoring not in _SCORING:
        raise ValueError(f"router: scoring must be one of {sorted(_SCORING)}")
    lib = _mm.load()
    with _mm.on_device(x2):
        _mm.check(lib.mm_router(_mm.ptr(x2), _mm.dtype_code(x2), x2.shape[0], H, x2.stride(0), _mm.ptr(w32), E,
                                _mm.ptr(bias), _SCORING[scoring], int(n_group), int(topk_group), int(top_k),
                                float(scale), 1 if append_shared else 0, _mm.ptr(logits), _mm.ptr(ids),
                                _mm.dtype_code(ids), _mm.ptr(wts), out_stride, _mm.stream_of(x2)), "moe_route")


def moe_route(x, w32, bias, n_group, topk_group, top_k, scale, logits_buf, ids_out, wts_out, *, scoring="sigmoid",
              append_shared=True):
    """x: [1, H] (one token; [N, H] also accepted). Writes logits_buf [E] (or [N, E]) fp32, ids_out [top_k+1]
    (shared expert id E last) and wts_out [top_k+1] fp32 in place and returns (ids_out, wts_out, logits_buf)."""
    _mm.require_gpu(x, w32, bias, logits_buf, ids_out, wts_out)
    x2 = x.reshape(-1, x.shape[-1])
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    n = x2.shape[0]
    width = top_k + (1 if append_shared else 0)
    if not ids_out.is_contiguous() or not wts_out.is_contiguous():
        raise ValueError("moe_route: ids_out and wts_out must be contiguous")
    if ids_out.numel() != n * width or wts_out.numel() != n * width:
        raise ValueError(f"moe_route: ids_out/wts_out need {n}x{width} elements")
    _route_into(x2, w32, bias, n_group, topk_group, top_k, scale, logits_buf, ids_out, wts_out, scoring,
                append_shared, width)
    return ids_out, wts_out, logits_buf


def route(x, w32, bias=None, *, top_k, n_group=1, topk_group=1, scale=1.0, scoring="softmax", append_shared=True,
          ids_dtype=torch.int64):
    """Router for N tokens: returns (ids [N, top_k(+1)], wts [N, top_k(+1)] fp32, logits [N, E] fp32)."""
    _mm.require_gpu(x, w32, bias)
    x2 = x.reshape(-1, x.shape[-1])
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    n, E = x2.shape[0], w32.shape[0]
    width = top_k + (1 if append_shared else 0)
    logits = torch.empty(n, E, device=x.device, dtype=torch.float32)
    ids = torch.empty(n, width, device=x.device, dtype=ids_dtype)
    wts = torch.empty(n, width, device=x.device, dtype=torch.float32)
    _route_into(x2, w32, bias, n_group, topk_group, top_k, scale, logits, ids, wts, scoring, append_shared, width)
    return ids, wts, logits
