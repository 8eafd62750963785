"""Fused MoE for the Ming thinker on hand-written gfx950 HIP kernels (drop-in for the reference fused_moe.py).

Experts (plus the shared expert, stored as expert index E) live in stacked tensors w_gu [E+1, 2I, H]
(gate rows, then up rows) and w_d [E+1, H, I], bf16 or int8 with per-output-row scales.

  fused_moe_decode   1..8 tokens: expert-gathered GEMV pair streaming each distinct expert once
                     (fused_moe.py:67-83)
  fused_moe_prefill  N tokens: on-GPU align into 64-row expert blocks, grouped MFMA gate/up and down GEMMs,
                     ordered per-token combine (fused_moe.py:176-196); N <= 8 takes the decode kernels
  _align_blocks      the stable counting sort behind prefill, bit-exact with the reference (fused_moe.py:154-173)
  quantize_rows_int8 symmetric per-row int8 (fused_moe.py:199-204)
  gate_up_slabs      the prefill copy of a bf16 w_gu (each 64-k slab of 8 rows one 1 KB piece), made once at
                     load; passed as w_gu_slabs, the prefill gate/up GEMM reads it instead of w_gu (same results)
  down_slabs         the same for w_d, passed as w_d_slabs and read by the prefill down GEMM
  prefill_copies     makes and registers both copies of a stack pair; fused_moe_prefill and moe_block_prefill then
                     find them by themselves (PREFILL_COPIES = "auto" also makes them on the first eager call)

A copy is bound to the stack it was made from: it records the stack's address, shape, strides and torch's
write counter, and a copy whose stack was written to since (the loader's copy_ into it, any in-place op) is
refused when passed explicitly and remade when found in the registry.

CFG and GCFG are kept for callers that read or tune them; the HIP kernels choose their own tiles, so the
values are advisory.
"""
import time
import weakref

import torch

import _mingmoe as _mm

__all__ = ["fused_moe_decode", "fused_moe_prefill", "quantize_rows_int8", "gate_up_slabs", "down_slabs",
           "prefill_copies", "release_prefill_copies", "CFG", "GCFG"]

CFG = dict(A=dict(BN=16, BK=256, num_warps=4), B=dict(BN=16, BK=256, num_warps=4))
GCFG = dict(A=dict(BM=64, BN=64, BK=64, num_warps=4), B=dict(BM=64, BN=128, BK=64, num_warps=4))

BLOCK_M = 64        # rows per expert block of the reference's grouped kernels (_align_blocks default)
MAX_DECODE_TOKENS = 8
_MAX_PAIRS = 64


def _flat_ids(ids):
    if ids.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"ids must be int32 or int64 (got {ids.dtype})")
    return ids if ids.is_contiguous() else ids.contiguous()


def fused_moe_decode(x, w_gu, w_d, ids, weights, a_buf=None, out=None, s_gu=None, s_d=None, *, residual=None,
                     phases=_mm.MM_PHASE_ALL):
    """x: [1, H] bf16 ([N, H] with N <= 8 also accepted); ids: [NK] (or [N, NK]) expert ids, shared expert
    included; weights: same shape, fp32. w_gu/w_d are bf16, or int8 with row scales s_gu [E+1, 2I] /
    s_d [E+1, H] (fp32 or bf16). Returns y [N, H] bf16 = sum_k weights[k] * expert_k(x) (+ residual).
    phases (default all) selects the gate/up and/or down kernel, for timing one of them."""
    _mm.require_gpu(x, w_gu, w_d, ids, weights, a_buf, out, s_gu, s_d, residual)
    H = x.shape[-1]
    x2 = x.reshape(-1, H)
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    N = x2.shape[0]
    ids2 = _flat_ids(ids).reshape(N, -1)
    NK = ids2.shape[1]
    if weights.dtype != torch.float32:
        weights = weights.float()
    wts2 = weights.reshape(N, NK)
    if not wts2.is_contiguous():
        wts2 = wts2.contiguous()
    if x.dtype != torch.bfloat16:
        raise ValueError(f"fused_moe_decode: x must be bf16 (got {x.dtype})")
    if N * NK > _MAX_PAIRS:
        raise ValueError(f"fused_moe_decode: {N} tokens x {NK} slots exceeds {_MAX_PAIRS} pairs")
    ex = _mm.experts(w_gu, w_d, s_gu, s_d)
    I = ex.inter
    a = torch.empty(N * NK, I, device=x.device, dtype=torch.bfloat16) if a_buf is None else a_buf
    if a.dtype != torch.bfloat16 or a.numel() < N * NK * I or not a.is_contiguous():
        raise ValueError(f"fused_moe_decode: a_buf must be a contiguous bf16 buffer of {N * NK}x{I}")
    y = torch.empty(N, H, device=x.device, dtype=torch.bfloat16) if out is None else out
    if y.dtype != torch.bfloat16 or y.numel() != N * H or not y.is_contiguous():
        raise ValueError(f"fused_moe_decode: out must be a contiguous bf16 [{N}, {H}] tensor")
    r2 = None
    if residual is not None:
        r2 = residual.reshape(N, H)
        if r2.dtype != torch.bfloat16:
            raise ValueError("fused_moe_decode: residual must be bf16")
        if not r2.is_contiguous():
            r2 = r2.contiguous()
    lib = _mm.load()
    with _mm.on_device(x):
        _mm.check(lib.mm_moe_decode(_mm.ptr(x2), N, x2.stride(0), ex, _mm.ptr(ids2), _mm.dtype_code(ids2), NK,
                                    ids2.stride(0), _mm.ptr(wts2), wts2.stride(0), _mm.ptr(r2),
                                    r2.stride(0) if r2 is not None else 0, _mm.ptr(a), _mm.ptr(y), H, phases,
                                    _mm.stream_of(x)), "fused_moe_decode")
    return y.view(N, H)


_SCORING = {"sigmoid": _mm.MM_SCORE_SIGMOID_GROUP, "softmax": _mm.MM_SCORE_SOFTMAX}


def moe_block_decode(x, norm_w, eps, w32, w_gu, w_d, *, top_k, bias=None, scoring="softmax", n_group=1,
                     topk_group=1, scale=1.0, s_gu=None, s_d=None, residual=True, logits=None, ids=None, wts=None,
                     a_buf=None, out=None, workspace=None):
    """One decode MoE block for 1..8 bf16 tokens in four kernels: the router GEMV with the RMSNorm (norm_w, eps)
    applied on the fly (the normalised rows go to `workspace`, bf16 [N, H]); the expert selection (shared
    expert appended); the gate/up GEMV; the down GEMV with the combine and the residual add of x.
    Same results as rms_norm -> moe_route -> fused_moe_decode(residual=x). Returns (y [N, H], ids, wts,
    logits); the optional buffers make the call allocation-free."""
    _mm.require_gpu(x, norm_w, w32, w_gu, w_d, bias, s_gu, s_d, logits, ids, wts, a_buf, out, workspace)
    H = x.shape[-1]
    x2 = x.reshape(-1, H)
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    N, E = x2.shape[0], w32.shape[0]
    NK = top_k + 1
    for name, t, dt in (("x", x2, torch.bfloat16), ("norm_w", norm_w, torch.bfloat16), ("w32", w32, torch.float32)):
        if t.dtype != dt or not t.is_contiguous():
            raise ValueError(f"moe_block_decode: {name} must be contiguous {dt}")
    if bias is not None and (bias.dtype != torch.float32 or bias.numel() != E or not bias.is_contiguous()):
        raise ValueError("moe_block_decode: bias must be a contiguous fp32 [E] tensor")
    if scoring not in _SCORING:
        raise ValueError(f"moe_block_decode: scoring must be one of {sorted(_SCORING)}")
    ex = _mm.experts(w_gu, w_d, s_gu, s_d)
    dev = x.device
    logits = torch.empty(N, E, device=dev, dtype=torch.float32) if logits is None else logits
    ids = torch.empty(N, NK, device=dev, dtype=torch.int64) if ids is None else ids
    wts = torch.empty(N, NK, device=dev, dtype=torch.float32) if wts is None else wts
    a = torch.empty(N * NK, ex.inter, device=dev, dtype=torch.bfloat16) if a_buf is None else a_buf
    y = torch.empty(N, H, device=dev, dtype=torch.bfloat16) if out is None else out
    for name, t, n, dt in (("logits", logits, N * E, torch.float32), ("wts", wts, N * NK, torch.float32),
                           ("a_buf", a, N * NK * ex.inter, torch.bfloat16), ("out", y, N * H, torch.bfloat16)):
        if t.dtype != dt or t.numel() < n or not t.is_contiguous():
            raise ValueError(f"moe_block_decode: {name} must be a contiguous {dt} buffer of {n} elements")
    if ids.dtype not in (torch.int32, torch.int64) or ids.numel() != N * NK or not ids.is_contiguous():
        raise ValueError(f"moe_block_decode: ids must be a contiguous int32/int64 [{N}, {NK}] tensor")
    ws = torch.empty(N, H, device=dev, dtype=torch.bfloat16) if workspace is None else workspace
    if ws.numel() * ws.element_size() < N * H * 2 or not ws.is_contiguous():
        raise ValueError(f"moe_block_decode: workspace must be a contiguous buffer of at least {N * H * 2} bytes")
    lib = _mm.load()
    with _mm.on_device(x):
        _mm.check(lib.mm_moe_block_decode(_mm.ptr(x2), N, x2.stride(0), _mm.ptr(norm_w), float(eps), _mm.ptr(w32), E,
                                          _mm.ptr(bias), _SCORING[scoring], int(n_group), int(topk_group), int(top_k),
                                          float(scale), ex, _mm.ptr(logits), _mm.ptr(ids), _mm.dtype_code(ids),
                                          _mm.ptr(wts), _mm.ptr(a), _mm.ptr(ws), 1 if residual else 0, _mm.ptr(y),
                                          H, _mm.stream_of(x)), "moe_block_decode")
    return y.view(N, H), ids.view(N, NK), wts.view(N, NK), logits.view(N, E)


def _num_blocks(P, E1, BM):
    return (P + E1 * (BM - 1) + BM - 1) // BM


def _align_blocks(flat, E1, BM, expert_offsets=None, out=None):
    """Sort pair indices by expert, padding each expert's run to a multiple of BM (GPU only, no sync).
    Returns sorted pair ids (P = padding) and the expert of each BM block (-1 = unused), and nb.
    expert_offsets (int32 [E1+1]) receives each expert's padded start row and the used row count;
    out = (sorted_ids, bexp) reuses caller buffers."""
    _mm.require_gpu(flat)
    flat = _flat_ids(flat).reshape(-1)
    P = flat.numel()
    nb = _num_blocks(P, E1, BM)
    if out is not None:
        sorted_ids, bexp = out
        if sorted_ids.numel() != nb * BM or bexp.numel() != nb or sorted_ids.dtype != torch.int32 \
                or bexp.dtype != torch.int32:
            raise ValueError("_align_blocks: out buffers do not match the block count")
    else:
        sorted_ids = torch.empty(nb * BM, dtype=torch.int32, device=flat.device)
        bexp = torch.empty(nb, dtype=torch.int32, device=flat.device)
    if expert_offsets is not None and (expert_offsets.dtype != torch.int32 or expert_offsets.numel() != E1 + 1):
        raise ValueError("_align_blocks: expert_offsets must be int32 with E1 + 1 elements")
    lib = _mm.load()
    with _mm.on_device(flat):
        _mm.check(lib.mm_align_blocks(_mm.ptr(flat), _mm.dtype_code(flat), P, int(E1), int(BM), _mm.ptr(sorted_ids),
                                      _mm.ptr(bexp), nb, _mm.ptr(expert_offsets), _mm.stream_of(flat)),
                  "_align_blocks")
    return sorted_ids, bexp, nb


def prefill_block_m(n_tokens, kp1, n_slots, w_dtype=torch.bfloat16):
    """Rows per expert block the prefill kernels take for this shape (the align padding): 128 for bf16 experts
    averaging at least 128 pairs, else 64."""
    code = _mm.MM_INT8 if w_dtype == torch.int8 else _mm.MM_BF16
    return int(_mm.load().mm_prefill_block_m(int(n_tokens), int(kp1), int(n_slots), code))


def _a_cols(I):
    return 64 * ((I + 63) // 64)


class PrefillScratch:
    """Device buffers of one prefill call (align output and intermediates), reusable across calls of the
    same shape and expert dtype so that a caller can keep them outside the timed or captured region."""

    def __init__(self, N, KP1, E1, H, I, device, block=False, w_dtype=torch.bfloat16):
        P = N * KP1
        self.block_m = prefill_block_m(N, KP1, E1, w_dtype)
        self.nb = _num_blocks(P, E1, self.block_m)
        self.sorted_ids = torch.empty(self.nb * self.block_m, dtype=torch.int32, device=device)
        self.bexp = torch.empty(self.nb, dtype=torch.int32, device=device)
        self.offsets = torch.empty(E1 + 1, dtype=torch.int32, device=device)
        # the gated activations in 64-column slabs per expert block: [nb][ceil(I/64)][block_m][64]
        self.a = torch.empty(self.nb * self.block_m, _a_cols(I), device=device, dtype=torch.bfloat16)
        self.part = torch.empty(P, H, device=device, dtype=torch.bfloat16)
        self.y = torch.empty(N, H, device=device, dtype=torch.bfloat16)
        if block:  # router outputs and normalised rows of moe_block_prefill
            self.logits = torch.empty(N, E1 - 1, device=device, dtype=torch.float32)
            self.ids = torch.empty(N, KP1, device=device, dtype=torch.int64)
            self.wts = torch.empty(N, KP1, device=device, dtype=torch.float32)
            self.xn = torch.empty(N, H, device=device, dtype=torch.bfloat16)


def fused_moe_prefill(x, w_gu, w_d, ids, weights, s_gu=None, s_d=None, *, residual=None, scratch=None,
                      phases=_mm.MM_PHASE_ALL, align=True, w_gu_slabs=None, w_d_slabs=None):
    """x: [N, H] bf16; ids: [N, K+1] expert ids per token (shared expert included); weights: [N, K+1] fp32.
    Returns [N, H] bf16 = sum_k weights[:, k] * expert_k(x) (+ residual). w_gu_slabs: gate_up_slabs(w_gu), read by
    the gate/up GEMM instead of w_gu; w_d_slabs: down_slabs(w_d), read by the down GEMM instead of w_d (same
    results). When neither is passed, the copies registered for w_gu / w_d are used (prefill_copies; with
    PREFILL_COPIES = "auto" an eager call makes them when the device has room), so the reference's call
    fused_moe_prefill(x, w_gu, w_d, ids, wts) reads the prefill layout without a change.
    scratch (a PrefillScratch) supplies the buffers; phases / align=False run part of the pipeline on
    scratch left by an earlier call, for timing one kernel."""
    _mm.require_gpu(x, w_gu, w_d, ids, weights, s_gu, s_d, residual)
    N, H = x.shape
    KP1 = ids.shape[-1]
    if N == 0:
        return torch.empty(0, H, device=x.device, dtype=x.dtype)
    if N <= MAX_DECODE_TOKENS and N * KP1 <= _MAX_PAIRS:  # decode-sized batches stream each expert once
        return fused_moe_decode(x, w_gu, w_d, ids, weights, s_gu=s_gu, s_d=s_d, residual=residual,
                                phases=phases & (_mm.MM_PHASE_GATE_UP | _mm.MM_PHASE_DOWN))
    if x.dtype != torch.bfloat16:
        raise ValueError(f"fused_moe_prefill: x must be bf16 (got {x.dtype})")
    if w_gu_slabs is None and w_d_slabs is None:
        w_gu_slabs, w_d_slabs = _copies_for(w_gu, w_d)
    ex = _mm.experts(w_gu, w_d, s_gu, s_d, w_gu_slabs, w_d_slabs)
    E1, I = ex.n_slots, ex.inter
    x2 = x if x.is_contiguous() else x.contiguous()
    flat = _flat_ids(ids).reshape(-1)
    P = flat.numel()
    if P != N * KP1:
        raise ValueError("fused_moe_prefill: ids must be [N, K+1]")
    wts = weights.reshape(-1).float().contiguous()
    sc = scratch if scratch is not None else PrefillScratch(N, KP1, E1, H, I, x.device, w_dtype=w_gu.dtype)
    if sc.a.shape != (sc.nb * sc.block_m, _a_cols(I)) or sc.y.shape != (N, H) or sc.offsets.numel() != E1 + 1:
        raise ValueError("fused_moe_prefill: scratch was made for another shape")
    if sc.block_m != prefill_block_m(N, KP1, E1, w_gu.dtype):
        raise ValueError("fused_moe_prefill: scratch was made for another expert dtype (PrefillScratch w_dtype)")
    nb = sc.nb
    if align:
        _align_blocks(flat, E1, sc.block_m, expert_offsets=sc.offsets, out=(sc.sorted_ids, sc.bexp))
    sorted_ids, bexp, a, part, y = sc.sorted_ids, sc.bexp, sc.a, sc.part, sc.y
    r2 = None
    if residual is not None:
        r2 = residual.reshape(N, H)
        if r2.dtype != torch.bfloat16:
            raise ValueError("fused_moe_prefill: residual must be bf16")
        if not r2.is_contiguous():
            r2 = r2.contiguous()
    lib = _mm.load()
    with _mm.on_device(x):
        _mm.check(lib.mm_moe_prefill(_mm.ptr(x2), N, x2.stride(0), ex, KP1, _mm.ptr(flat), _mm.dtype_code(flat),
                                     _mm.ptr(wts), _mm.ptr(sorted_ids), _mm.ptr(bexp), _mm.ptr(sc.offsets), nb,
                                     sc.block_m, _mm.ptr(r2), r2.stride(0) if r2 is not None else 0, _mm.ptr(a),
                                     _mm.ptr(part), _mm.ptr(y), H,
                                     phases, _mm.stream_of(x)), "fused_moe_prefill")
    return y


def moe_block_prefill(x, norm_w, eps, w32, w_gu, w_d, *, top_k, bias=None, scoring="softmax", n_group=1,
                      topk_group=1, scale=1.0, s_gu=None, s_d=None, residual=True, scratch=None, w_gu_slabs=None,
                      w_d_slabs=None):
    """One prefill MoE block: RMSNorm (norm_w, eps; normalised rows kept in the scratch), router, expert
    selection (shared expert appended), align, gate/up, down, combine (+ x).
    Same results as rms_norm -> route -> fused_moe_prefill(residual=x). Returns (y [N, H], ids, wts,
    logits), views of `scratch` (a PrefillScratch made with block=True; allocated when None). w_gu_slabs,
    w_d_slabs: as in fused_moe_prefill (registered copies are found the same way)."""
    _mm.require_gpu(x, norm_w, w32, w_gu, w_d, bias, s_gu, s_d)
    H = x.shape[-1]
    x2 = x.reshape(-1, H)
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    N, E = x2.shape[0], w32.shape[0]
    NK = top_k + 1
    for name, t, dt in (("x", x2, torch.bfloat16), ("norm_w", norm_w, torch.bfloat16), ("w32", w32, torch.float32)):
        if t.dtype != dt or not t.is_contiguous():
            raise ValueError(f"moe_block_prefill: {name} must be contiguous {dt}")
    if bias is not None and (bias.dtype != torch.float32 or bias.numel() != E or not bias.is_contiguous()):
        raise ValueError("moe_block_prefill: bias must be a contiguous fp32 [E] tensor")
    if scoring not in _SCORING:
        raise ValueError(f"moe_block_prefill: scoring must be one of {sorted(_SCORING)}")
    if w_gu_slabs is None and w_d_slabs is None:
        w_gu_slabs, w_d_slabs = _copies_for(w_gu, w_d)
    ex = _mm.experts(w_gu, w_d, s_gu, s_d, w_gu_slabs, w_d_slabs)
    sc = scratch if scratch is not None else PrefillScratch(N, NK, ex.n_slots, H, ex.inter, x.device, block=True,
                                                             w_dtype=w_gu.dtype)
    if sc.block_m != prefill_block_m(N, NK, ex.n_slots, w_gu.dtype):
        raise ValueError("moe_block_prefill: scratch was made for another expert dtype (PrefillScratch w_dtype)")
    if not hasattr(sc, "xn") or sc.xn.shape != (N, H) or sc.ids.shape != (N, NK) or sc.logits.shape != (N, E) \
            or sc.a.shape != (sc.nb * sc.block_m, _a_cols(ex.inter)) or sc.offsets.numel() != ex.n_slots + 1:
        raise ValueError("moe_block_prefill: scratch was made for another shape (or without block=True)")
    if N == 0:
        return sc.y, sc.ids, sc.wts, sc.logits
    lib = _mm.load()
    with _mm.on_device(x):
        _mm.check(lib.mm_moe_block_prefill(_mm.ptr(x2), N, x2.stride(0), _mm.ptr(norm_w), float(eps), _mm.ptr(w32), E,
                                           _mm.ptr(bias), _SCORING[scoring], int(n_group), int(topk_group),
                                           int(top_k), float(scale), ex, _mm.ptr(sc.logits), _mm.ptr(sc.ids),
                                           _mm.dtype_code(sc.ids), _mm.ptr(sc.wts), _mm.ptr(sc.xn),
                                           _mm.ptr(sc.sorted_ids), _mm.ptr(sc.bexp), _mm.ptr(sc.offsets), sc.nb,
                                           _mm.ptr(sc.a), _mm.ptr(sc.part), 1 if residual else 0, _mm.ptr(sc.y), H,
                                           _mm.stream_of(x)), "moe_block_prefill")
    return sc.y, sc.ids, sc.wts, sc.logits


def _piece_rows(w):
    """Rows per 1 KB piece of the prefill layout: 8 for bf16 weights (128 bytes of a 64-k slab each), 16 for int8."""
    return 8 if w.dtype == torch.bfloat16 else 16


def gate_up_slabs(w_gu, out=None):
    """The prefill copy of a gate/up stack w_gu [E1, 2I, H], bf16 or int8 (H a multiple of 64; 2I of R, R = 8 for
    bf16 and 16 for int8): out[e, q, t, j, c] = w_gu[e, R q + j, 64 t + c], a contiguous [E1, 2I / R, H / 64, R, 64]
    tensor of w_gu's dtype, so that each 64-wide k-slab of R consecutive rows is one 1 KB piece. A load-time step: it
    costs a second gate/up stack and lets the prefill gate/up GEMM read a tile's k-slab as 1 KB pieces (one per
    direct-load instruction) instead of 128- (bf16) or 64-byte (int8) row slices. Pass the result as w_gu_slabs, or register it with prefill_copies. The result
    records w_gu's stamp (_mingmoe.source_stamp); once w_gu is written to, the copy is refused until made again."""
    _mm.require_gpu(w_gu, out)
    if w_gu.dim() != 3 or w_gu.dtype not in (torch.bfloat16, torch.int8) or w_gu.stride(2) != 1:
        raise ValueError("gate_up_slabs: w_gu must be a bf16 or int8 [E1, 2I, H] stack with a contiguous last dim")
    E1, two_i, H = w_gu.shape
    R = _piece_rows(w_gu)
    if H % 64 or two_i % R:
        raise ValueError(f"gate_up_slabs: hidden ({H}) must be a multiple of 64 and 2I ({two_i}) a multiple of {R}")
    ex = _mm.Experts()  # only w_gu is read
    ex.w_gu, ex.w_dtype, ex.s_dtype = w_gu.data_ptr(), _mm.dtype_code(w_gu), _mm.MM_FP32
    ex.n_slots, ex.hidden, ex.inter = E1, H, two_i // 2
    ex.gu_stride_e, ex.gu_stride_n = w_gu.stride(0), w_gu.stride(1)
    shape = (E1, two_i // R, H // 64, R, 64)
    q = torch.empty(shape, device=w_gu.device, dtype=w_gu.dtype) if out is None else out
    if q.dtype != w_gu.dtype or not q.is_contiguous() or tuple(q.shape) != shape:
        raise ValueError(f"gate_up_slabs: out must be a contiguous {w_gu.dtype} {shape} tensor")
    lib = _mm.load()
    with _mm.on_device(w_gu):
        _mm.check(lib.mm_gate_up_slabs(ex, _mm.ptr(q), _mm.stream_of(w_gu)), "gate_up_slabs")
    q._mm_source = _mm.source_stamp(w_gu)  # what the copy is current for (checked by _mingmoe.experts)
    return q


def down_slabs(w_d, out=None):
    """The prefill copy of a down stack w_d [E1, H, I], bf16 or int8 (I a multiple of 64, H of R):
    out[e, q, t, j, c] = w_d[e, R q + j, 64 t + c], a contiguous [E1, H / R, I / 64, R, 64] tensor, laid out as
    gate_up_slabs lays out w_gu. A load-time step: it costs a second down stack and lets the prefill down GEMM
    read each k-slab of a weight tile as 1 KB pieces. Pass the result as w_d_slabs."""
    _mm.require_gpu(w_d, out)
    if w_d.dim() != 3 or w_d.dtype not in (torch.bfloat16, torch.int8) or w_d.stride(2) != 1:
        raise ValueError("down_slabs: w_d must be a bf16 or int8 [E1, H, I] stack with a contiguous last dim")
    E1, H, I = w_d.shape
    R = _piece_rows(w_d)
    if I % 64 or H % R:
        raise ValueError(f"down_slabs: inter ({I}) must be a multiple of 64 and hidden ({H}) a multiple of {R}")
    ex = _mm.Experts()  # only w_d is read
    ex.w_d, ex.w_dtype, ex.s_dtype = w_d.data_ptr(), _mm.dtype_code(w_d), _mm.MM_FP32
    ex.n_slots, ex.hidden, ex.inter = E1, H, I
    ex.d_stride_e, ex.d_stride_n = w_d.stride(0), w_d.stride(1)
    shape = (E1, H // R, I // 64, R, 64)
    q = torch.empty(shape, device=w_d.device, dtype=w_d.dtype) if out is None else out
    if q.dtype != w_d.dtype or not q.is_contiguous() or tuple(q.shape) != shape:
        raise ValueError(f"down_slabs: out must be a contiguous {w_d.dtype} {shape} tensor")
    lib = _mm.load()
    with _mm.on_device(w_d):
        _mm.check(lib.mm_down_slabs(ex, _mm.ptr(q), _mm.stream_of(w_d)), "down_slabs")
    q._mm_source = _mm.source_stamp(w_d)
    return q


# ------------------------------------------------------------------------- prefill copies bound to their stacks

# "auto": an eager prefill call on a stack without a registered copy makes one (if the device keeps at
# least COPY_FREE_FRACTION of its memory free afterwards) and registers it; "registered": only the copies made by
# prefill_copies are used; "off": the prefill GEMMs read the stacks themselves (the row layout).
PREFILL_COPIES = "auto"
COPY_FREE_FRACTION = 0.10


class _Entry:
    """A registered prefill copy: the copy, a weak reference to its stack's base tensor (the entry goes when the
    stack goes) and whether it was registered explicitly (trusted for stacks that keep no write counter)."""
    __slots__ = ("copy", "ref", "explicit", "__weakref__")


_registry = {}  # stack key (device, address, shape, strides) -> _Entry


def _base(w):
    return w._base if w._base is not None else w


def _slab_shape_ok(w):
    # gate/up copy [E1, 2I, H]: H a multiple of 64, 2I of R; down copy [E1, H, I]: I a multiple of 64, H of R
    return w.dtype in (torch.bfloat16, torch.int8) and w.dim() == 3 and w.stride(2) == 1 and \
        w.shape[2] % 64 == 0 and w.shape[1] % _piece_rows(w) == 0


def _register(w, copy, explicit):
    key = _mm.source_stamp(w)[:4]
    e = _Entry()
    e.copy, e.explicit = copy, explicit

    def gone(_ref, key=key, e=e, reg=_registry):  # reg bound now: module globals are gone at interpreter exit
        if reg.get(key) is e:
            del reg[key]
    e.ref = weakref.ref(_base(w), gone)
    _registry[key] = e


def _registered(w, make):
    """The current registered copy of stack w, made or remade here when allowed; None for the stack itself."""
    if PREFILL_COPIES == "off" or not _slab_shape_ok(w):
        return None
    key = _mm.source_stamp(w)[:4]
    e = _registry.get(key)
    if e is not None and e.ref() is not _base(w):  # another tensor now lives at that address
        del _registry[key]
        e = None
    ver = _mm.version_of(w)
    if e is not None and ((ver is not None and e.copy._mm_source[4] == ver) or (ver is None and e.explicit)):
        return e.copy
    capturing = torch.cuda.is_current_stream_capturing()
    if e is not None:  # the stack was written to after its copy was made
        if capturing:
            raise RuntimeError("fused_moe: an expert stack changed after its prefill copy was made; call "
                               "fused_moe.prefill_copies(w_gu, w_d) again before capturing")
        make(w, out=e.copy)
        return e.copy
    if capturing or PREFILL_COPIES != "auto" or ver is None:
        return None
    free, total = torch.cuda.mem_get_info(w.device)
    if free - w.numel() * w.element_size() < COPY_FREE_FRACTION * total:
        return None
    copy = make(w)
    _register(w, copy, False)
    return copy


def _copies_for(w_gu, w_d):
    return _registered(w_gu, gate_up_slabs), _registered(w_d, down_slabs)


def prefill_copies(w_gu, w_d):
    """Makes (or remakes) the prefill copies of a stack pair (bf16, or int8 without their scales) and registers them: every later
    fused_moe_prefill / moe_block_prefill on these stacks reads them, with no argument passed. A copy follows its
    stack: once the stack is written to (torch's write counter moves), the next eager call remakes the copy in
    place and a call under graph capture raises. Stacks made under torch.inference_mode keep no write counter:
    their copies are trusted until prefill_copies is called again. Returns (w_gu copy, w_d copy), either None for a
    shape the layout does not take. Costs a second copy of both stacks (per layer of hidden 2048, 64 + 1 experts of
    1408: 1.125 GB in bf16, 563 MB in int8)."""
    _mm.require_gpu(w_gu, w_d)
    out = []
    for w, make in ((w_gu, gate_up_slabs), (w_d, down_slabs)):
        if not _slab_shape_ok(w):
            out.append(None)
            continue
        e = _registry.get(_mm.source_stamp(w)[:4])
        copy = make(w, out=e.copy if e is not None and e.ref() is _base(w) else None)
        _register(w, copy, True)
        out.append(copy)
    return tuple(out)


def release_prefill_copies(*stacks):
    """Drops the registered copies of the given stacks (of every stack when none is given)."""
    if not stacks:
        _registry.clear()
        return
    for w in stacks:
        _registry.pop(_mm.source_stamp(w)[:4], None)


def quantize_rows_int8(w, *, scale_dtype=torch.float32):
    """Symmetric per-output-row int8: w [..., N, K] -> (int8 [..., N, K], scales [..., N]).
    scale_dtype torch.float32 (the reference) or torch.bfloat16 (q then divides by the rounded scale)."""
    _mm.require_gpu(w)
    if scale_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("quantize_rows_int8: scale_dtype must be torch.float32 or torch.bfloat16")
    K = w.shape[-1]
    w2 = w.reshape(-1, K)
    if not w2.is_contiguous():
        w2 = w2.contiguous()
    rows = w2.shape[0]
    q = torch.empty(w.shape, dtype=torch.int8, device=w.device)
    s = torch.empty(w.shape[:-1], dtype=scale_dtype, device=w.device)
    lib = _mm.load()
    with _mm.on_device(w):
        _mm.check(lib.mm_quantize_rows_int8(_mm.ptr(w2), _mm.dtype_code(w2), rows, K, w2.stride(0), _mm.ptr(q), K,
                                            _mm.ptr(s), _mm.dtype_code(s), _mm.stream_of(w)), "quantize_rows_int8")
    return q, s


def _graph_us(fn, reps=50, inner=20):
    """Microseconds per call of fn, captured `inner` times in one hipGraph and replayed `reps` times."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
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
    return (time.perf_counter() - t) / reps / inner * 1e6
