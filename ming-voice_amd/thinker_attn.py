"""The thinker's attention mixers on hand-written gfx950 HIP kernels: the KDA (Kimi delta attention) layers'
recurrent core, short convolutions and gated output norm, and the MLA layers' attention over the static cache (one
decode token, or a prompt's tokens).

  fused_recurrent_kda   drop-in for fla.ops.kda.fused_recurrent_kda (fla-core 0.5.2; engine.py:242-262): same
                        keywords, B = 1; the state is fp32 [1, H, K, V], updated in place with inplace=True
  short_conv            the step form of fla's ShortConvolution (a [1, C, W] cache of the last inputs, SiLU)
  rms_norm_gated        fla's FusedRMSNormGated with a sigmoid gate (a KDA layer's o_norm)
  kda_decode_step       one decode token of a KDA layer's core (convolutions, the f / g LoRA up-projections, the
                        recurrence, the gated norm) in one kernel instead of the five calls above
  mla_decode_attn       one token of an MLA layer: the StaticHybridCache update at pos (engine.py:537-548) and the
                        masked softmax attention over positions 0..pos
  mla_prefill_attn      the T tokens of a prompt through an MLA layer: the update at pos .. pos + T - 1 and the
                        causal attention, token t over positions 0..pos+t (engine.py:938-972)
  embed_rows            word_embeddings(tok_buf), the input row of a decode step (engine.py:686)
  argmax_rows           logits.argmax(-1), the greedy pick a decode step writes back (engine.py:688)
Every call enqueues on torch's current stream and can be captured in a hipGraph (the workspace and outputs can be
passed in); there is no CPU path.
"""
import ctypes

import torch

import _mingmoe as _mm

__all__ = ["fused_recurrent_kda", "kda_workspace", "short_conv", "short_conv_many", "rms_norm_gated", "kda_decode_step", "mla_decode_attn",
           "mla_attn_workspace", "mla_prefill_attn", "embed_rows", "argmax_rows", "argmax_workspace"]


def _f32_or_bf16(t, name):
    if t.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"{name} must be fp32 or bf16 (got {t.dtype})")
    return _mm.MM_FP32 if t.dtype == torch.float32 else _mm.MM_BF16


def _tokens(t, name, H, D):
    """[1, T, H, D] or [T, H, D] with contiguous heads -> (tensor, T, token stride in elements)."""
    if t.dim() == 4:
        if t.shape[0] != 1:
            raise ValueError(f"{name}: batch {t.shape[0]} (B = 1 only)")
        t = t[0]
    if t.dim() != 3 or t.shape[1] != H or t.shape[2] != D:
        raise ValueError(f"{name}: expected [1, T, {H}, {D}], got {tuple(t.shape)}")
    if t.stride(2) != 1 or t.stride(1) != D:
        t = t.contiguous()
    return t, t.shape[0], t.stride(0)


def kda_workspace(T, H, K, device):
    """The fp32 workspace fused_recurrent_kda needs for T tokens of H heads of key dim K."""
    n = _mm.load().mm_kda_recurrent_workspace(T, H, K)
    if n < 0:
        raise ValueError(f"kda_workspace: bad T={T}, H={H} or K={K}")
    return torch.empty(max(n, 16) // 4, device=device, dtype=torch.float32)


def kda_chunk_workspace(T, H, K, device):
    """The fp32 workspace chunk_kda needs for T tokens of H heads of key dim K."""
    n = _mm.load().mm_kda_chunk_workspace(T, H, K)
    if n < 0:
        raise ValueError(f"kda_chunk_workspace: bad T={T}, H={H} or K={K}")
    return torch.empty(max(n, 16) // 4, device=device, dtype=torch.float32)


def fused_recurrent_kda(q, k, v, g, beta, A_log=None, dt_bias=None, scale=None, initial_state=None,
                        output_final_state=False, use_qk_l2norm_in_kernel=False, use_gate_in_kernel=False,
                        lower_bound=None, inplace=False, out=None, beta_is_logits=False, workspace=None, n_valid=None,
                        **unused):
    """q, k [1, T, H, K] bf16; v [1, T, H, V] bf16; g [1, T, H, K] (bf16 / fp32; the raw gate projection when
    use_gate_in_kernel, else a log decay); beta [1, T, H] (fp32 / bf16); A_log [H], dt_bias [H * K] (or [H, K]);
    initial_state [1, H, K, V] fp32 (zeros when None). Returns (o [1, T, H, V] bf16, final_state or None).
    scale defaults to K ** -0.5. inplace=True updates initial_state itself (final_state is then that tensor);
    beta_is_logits=True takes the beta projection itself and applies the sigmoid in the kernel. workspace: from
    kda_workspace(T, H, K) (allocated when None). n_valid: a one-element int64 device tensor n, or None: tokens
    n .. T - 1 are padding and leave the state exactly unchanged (the engine's padded prefill, engine.py:252-253)."""
    return _kda("fused_recurrent_kda", False, q, k, v, g, beta, A_log, dt_bias, scale, initial_state,
                output_final_state, use_qk_l2norm_in_kernel, use_gate_in_kernel, lower_bound, inplace, out,
                beta_is_logits, workspace, n_valid)


def chunk_kda(q, k, v, g, beta, A_log=None, dt_bias=None, scale=None, initial_state=None, output_final_state=False,
              use_qk_l2norm_in_kernel=False, use_gate_in_kernel=False, lower_bound=None, inplace=False, out=None,
              beta_is_logits=False, workspace=None, n_valid=None, **unused):
    """fla's chunk_kda (the form the engine's eager prefill selects past 192 tokens, engine.py:946-949): the
    arguments, outputs and state update of fused_recurrent_kda, computed 16 tokens at a time in closed form (the
    same values up to the order of fp32 sums). workspace: from kda_chunk_workspace(T, H, K) (allocated when None)."""
    return _kda("chunk_kda", True, q, k, v, g, beta, A_log, dt_bias, scale, initial_state, output_final_state,
                use_qk_l2norm_in_kernel, use_gate_in_kernel, lower_bound, inplace, out, beta_is_logits, workspace,
                n_valid)


def _kda(name, chunked, q, k, v, g, beta, A_log, dt_bias, scale, initial_state, output_final_state,
         use_qk_l2norm_in_kernel, use_gate_in_kernel, lower_bound, inplace, out, beta_is_logits, workspace, n_valid):
    _mm.require_gpu(q, k, v, g, beta, A_log, dt_bias, initial_state, out, workspace, n_valid)
    _check_count(n_valid, name)
    if q.dim() != 4 or q.shape[0] != 1:
        raise ValueError(f"{name}: q must be [1, T, H, K] (got {tuple(q.shape)})")
    _, T, H, K = q.shape
    V = v.shape[-1]
    for nm, t in (("q", q), ("k", k), ("v", v)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{name}: {nm} must be bf16 (got {t.dtype})")
    q2, _, qts = _tokens(q, "q", H, K)
    k2, _, kts = _tokens(k, "k", H, K)
    v2, _, vts = _tokens(v, "v", H, V)
    g2, _, gts = _tokens(g, "g", H, K)
    gdt = _f32_or_bf16(g2, "g")
    b2 = beta[0] if beta.dim() == 3 else beta
    if tuple(b2.shape) != (T, H):
        raise ValueError(f"{name}: beta must be [1, T, H] (got {tuple(beta.shape)})")
    if b2.stride(1) != 1:
        b2 = b2.contiguous()
    bdt = _f32_or_bf16(b2, "beta")
    use_gate = bool(use_gate_in_kernel)
    if use_gate:
        if A_log is None or dt_bias is None:
            raise ValueError(f"{name}: use_gate_in_kernel needs A_log and dt_bias")
        A_log = A_log.float().reshape(H).contiguous()
        dt_bias = dt_bias.float().reshape(H * K).contiguous()
    if initial_state is None:
        state = torch.zeros(H, K, V, device=q.device, dtype=torch.float32)
    else:
        if initial_state.dtype != torch.float32 or tuple(initial_state.shape[-3:]) != (H, K, V):
            raise ValueError(f"{name}: initial_state must be fp32 [1, {H}, {K}, {V}]")
        if inplace:
            if not initial_state.is_contiguous():
                raise ValueError(f"{name}: inplace needs a contiguous initial_state")
            state = initial_state
        else:
            state = initial_state.reshape(H, K, V).clone()
    o = torch.empty(T, H, V, device=q.device, dtype=torch.bfloat16) if out is None else out.view(T, H, V)
    if o.dtype != torch.bfloat16 or o.stride(2) != 1 or o.stride(1) != V:
        raise ValueError(f"{name}: out must be bf16 [1, T, H, V] with contiguous heads")
    sc = float(scale) if scale is not None else K ** -0.5
    lb = float("nan") if lower_bound is None else float(lower_bound)
    lib = _mm.load()
    ws = workspace
    if ws is None and (lib.mm_kda_chunk_workspace if chunked else lib.mm_kda_recurrent_workspace)(T, H, K) > 0:
        ws = (kda_chunk_workspace if chunked else kda_workspace)(T, H, K, q.device)
    fn = lib.mm_kda_chunk if chunked else lib.mm_kda_recurrent
    with _mm.on_device(q):
        _mm.check(fn(_mm.ptr(q2), qts, _mm.ptr(k2), kts, _mm.ptr(v2), vts, _mm.ptr(g2), gdt, gts, _mm.ptr(b2), bdt,
                     b2.stride(0), _mm.ptr(A_log), _mm.ptr(dt_bias), lb, 1 if use_qk_l2norm_in_kernel else 0,
                     1 if use_gate else 0, 1 if beta_is_logits else 0, sc, T, H, K, V, _mm.ptr(state), _mm.ptr(o),
                     o.stride(0), _mm.ptr(n_valid), _mm.ptr(ws), ws.numel() * 4 if ws is not None else 0,
                     _mm.stream_of(q)), name)
    final = None
    if output_final_state or inplace:
        final = state if (inplace and initial_state is not None) else state.reshape(1, H, K, V)
    return o.reshape(1, T, H, V), final


def _check_count(n, what):
    if n is not None and (n.dtype != torch.int64 or n.numel() != 1):
        raise ValueError(f"{what}: n_valid must be a one-element int64 device tensor")


def short_conv(x, cache, weight, bias=None, activation="silu", out=None, n_valid=None):
    """x [1, T, C] or [T, C] bf16; cache [1, C, W] bf16 (the last W inputs per channel, updated in place); weight
    [C, 1, W] or [C, W] bf16; bias [C] or None. Returns y with x's shape: act(conv over the window) per token.
    n_valid: a one-element int64 device tensor n, or None: the cache ends on the first n tokens' inputs."""
    _mm.require_gpu(x, cache, weight, bias, out, n_valid)
    _check_count(n_valid, "short_conv")
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    T, C = x2.shape
    W = cache.shape[-1]
    if cache.numel() != C * W or not cache.is_contiguous() or cache.dtype != torch.bfloat16:
        raise ValueError(f"short_conv: cache must be a contiguous bf16 [1, {C}, W] tensor")
    w2 = weight.reshape(C, -1)
    if w2.shape[1] != W or w2.dtype != torch.bfloat16:
        raise ValueError(f"short_conv: weight must be bf16 [{C}, 1, {W}]")
    w2 = w2.contiguous()
    if bias is not None:
        bias = bias.to(torch.bfloat16).contiguous()
    if activation not in ("silu", "swish", None):
        raise ValueError(f"short_conv: activation {activation!r} (silu or None)")
    y = torch.empty(T, C, device=x.device, dtype=torch.bfloat16) if out is None else out.view(T, C)
    lib = _mm.load()
    with _mm.on_device(x):
        _mm.check(lib.mm_short_conv(_mm.ptr(x2), x2.stride(0), T, C, _mm.ptr(cache), W, _mm.ptr(w2), _mm.ptr(bias),
                                    0 if activation is None else 1, _mm.ptr(y), y.stride(0), _mm.ptr(n_valid),
                                    _mm.stream_of(x)),
                  "short_conv")
    return y.reshape(x.shape)


def short_conv_many(xs, caches, weights, activation="silu", n_valid=None):
    """short_conv (no bias) on up to 4 inputs over the same tokens and window width in one launch, each with its own
    cache (updated in place) and weight: the q, k and v convolutions of a KDA layer's prompt. xs: [T, C_i] bf16 (unit
    last-dim stride); caches [1, C_i, W]; weights [C_i, 1, W]. Returns [y_i], each equal to short_conv(x_i, ...)."""
    n = len(xs)
    if not 1 <= n <= 4 or len(caches) != n or len(weights) != n:
        raise ValueError("short_conv_many: 1 to 4 inputs, with as many caches and weights")
    _mm.require_gpu(*xs, *caches, *weights, n_valid)
    _check_count(n_valid, "short_conv_many")
    if activation not in ("silu", "swish", None):
        raise ValueError(f"short_conv_many: activation {activation!r} (silu or None)")
    x2s, w2s, ys = [], [], []
    T, W = xs[0].reshape(-1, xs[0].shape[-1]).shape[0], caches[0].shape[-1]
    for x, cache, weight in zip(xs, caches, weights):
        x2 = x.reshape(-1, x.shape[-1])
        if x2.stride(-1) != 1:
            x2 = x2.contiguous()
        C = x2.shape[1]
        if x2.shape[0] != T or cache.shape[-1] != W:
            raise ValueError("short_conv_many: every input needs the same tokens and window width")
        if cache.numel() != C * W or not cache.is_contiguous() or cache.dtype != torch.bfloat16:
            raise ValueError(f"short_conv_many: cache must be a contiguous bf16 [1, {C}, W] tensor")
        w2 = weight.reshape(C, -1)
        if w2.shape[1] != W or w2.dtype != torch.bfloat16:
            raise ValueError(f"short_conv_many: weight must be bf16 [{C}, 1, {W}]")
        x2s.append(x2)
        w2s.append(w2.contiguous())
        ys.append(torch.empty(T, C, device=x.device, dtype=torch.bfloat16))

    def arr(ctype, vals):
        return (ctype * n)(*vals)
    lib = _mm.load()
    with _mm.on_device(xs[0]):
        _mm.check(lib.mm_short_conv_many(
            n, arr(ctypes.c_void_p, [_mm.ptr(t) for t in x2s]), arr(ctypes.c_int64, [t.stride(0) for t in x2s]),
            arr(ctypes.c_int64, [t.shape[1] for t in x2s]), arr(ctypes.c_void_p, [_mm.ptr(c) for c in caches]),
            arr(ctypes.c_void_p, [_mm.ptr(w) for w in w2s]), arr(ctypes.c_void_p, [_mm.ptr(y) for y in ys]),
            arr(ctypes.c_int64, [y.stride(0) for y in ys]), T, W, 0 if activation is None else 1, _mm.ptr(n_valid),
            _mm.stream_of(xs[0])), "short_conv_many")
    return [y.reshape(x.shape) for x, y in zip(xs, ys)]


def rms_norm_gated(x, g, weight, eps=1e-5, out=None):
    """bf16(x * rsqrt(mean(x^2) + eps) * weight * sigmoid(g)) over the last dim (<= 512); x, g bf16 of one shape."""
    _mm.require_gpu(x, g, weight, out)
    n = x.shape[-1]
    x2 = x.reshape(-1, n)
    g2 = g.reshape(-1, n)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    if g2.stride(-1) != 1:
        g2 = g2.contiguous()
    if x2.shape != g2.shape:
        raise ValueError("rms_norm_gated: x and g must have one shape")
    y = torch.empty(x2.shape, device=x.device, dtype=torch.bfloat16) if out is None else out.view(x2.shape)
    w = weight.to(torch.bfloat16).contiguous()
    lib = _mm.load()
    with _mm.on_device(x):
        _mm.check(lib.mm_rms_norm_gated(_mm.ptr(x2), x2.stride(0), _mm.ptr(g2), g2.stride(0), _mm.ptr(w), x2.shape[0], n,
                                        float(eps), _mm.ptr(y), y.stride(0), _mm.stream_of(x)), "rms_norm_gated")
    return y.reshape(x.shape)


def _three(t, sizes, name):
    """A (q, k, v) triple of tensors, or one tensor holding the three along dim -2 (split into views)."""
    if isinstance(t, (tuple, list)):
        if len(t) != 3:
            raise ValueError(f"kda_decode_step: {name} must hold q, k and v")
        return list(t)
    x = t.reshape(-1, t.shape[-1])
    if x.shape[0] != sum(sizes):
        raise ValueError(f"kda_decode_step: {name} must have {sum(sizes)} channels (got {x.shape[0]})")
    return list(torch.split(x, sizes, dim=0))


def kda_decode_step(pr, conv_w, conv_cache, f_b, g_b, A_log, dt_bias, state, o_norm, *, heads, eps=1e-5,
                    lower_bound=None, scale=None, out=None):
    """One decode token of a KDA layer's core in one kernel, on the layer's projection row
    pr = [q | k (heads * K each) | v (heads * V) | fa | ga (rank R each) | beta logits (heads)] ([1, len] or [len]
    bf16). conv_w and conv_cache: the q, k and v conv1d weights ([C, 1, 4]) and the layer's three conv caches
    ([1, C, 4], shifted in place), each a (q, k, v) tuple as the model and its cache hold them (engine.py:645-647),
    or one tensor of all 2 heads K + heads V channels in that order. Then f = f_b(fa), the recurrence of
    fused_recurrent_kda (l2-normed q and k, the in-kernel gate with A_log / dt_bias, beta = sigmoid of its logit;
    state [1, heads, K, V] fp32 in place), g = g_b(ga) and the gated RMSNorm with o_norm. Returns y [heads, V] bf16,
    the input of the layer's o projection. Same results as short_conv -> small_linear -> fused_recurrent_kda ->
    small_linear -> rms_norm_gated (engine.py:242-265) up to the last bf16 place of f and g. K = 128."""
    ws = conv_w if isinstance(conv_w, (tuple, list)) else [conv_w]
    cs = conv_cache if isinstance(conv_cache, (tuple, list)) else [conv_cache]
    _mm.require_gpu(pr, *ws, *cs, f_b, g_b, A_log, dt_bias, state, o_norm, out)
    H = int(heads)
    if state.dtype != torch.float32 or not state.is_contiguous() or state.dim() < 3:
        raise ValueError("kda_decode_step: state must be a contiguous fp32 [1, H, K, V] tensor")
    K, V = state.shape[-2:]
    R = f_b.shape[-1]
    if tuple(state.shape[-3:]) != (H, K, V):
        raise ValueError(f"kda_decode_step: state must be [1, {H}, K, V] (got {tuple(state.shape)})")
    sizes = [H * K, H * K, H * V]
    wq = _three(conv_w, sizes, "conv_w")
    cq = _three(conv_cache, sizes, "conv_cache")
    for name, group in (("conv_w", wq), ("conv_cache", cq)):
        for t, n in zip(group, sizes):
            if t.dtype != torch.bfloat16 or not t.is_contiguous() or t.numel() != n * 4:
                raise ValueError(f"kda_decode_step: each {name} part must be a contiguous bf16 [{n}, 4] tensor")
    for name, t, rows in (("f_b", f_b, H * K), ("g_b", g_b, H * V)):
        if t.dtype != torch.bfloat16 or not t.is_contiguous() or t.numel() != rows * R:
            raise ValueError(f"kda_decode_step: {name} must be a contiguous bf16 [{rows}, {R}] tensor")
    p = pr.reshape(-1)
    if p.dtype != torch.bfloat16 or p.stride(0) != 1:
        raise ValueError("kda_decode_step: pr must be a contiguous bf16 row")
    y = torch.empty(H, V, device=pr.device, dtype=torch.bfloat16) if out is None else out
    if y.dtype != torch.bfloat16 or not y.is_contiguous() or y.numel() != H * V:
        raise ValueError(f"kda_decode_step: out must be a contiguous bf16 [{H}, {V}] tensor")
    A = A_log.float().reshape(H).contiguous()
    dtb = dt_bias.float().reshape(H * K).contiguous()
    w = o_norm.to(torch.bfloat16).contiguous()
    fb, gb = _aligned16(f_b), _aligned16(g_b)
    sc = float(scale) if scale is not None else K ** -0.5
    lb = float("nan") if lower_bound is None else float(lower_bound)
    wp = (ctypes.c_void_p * 3)(*[t.data_ptr() for t in wq])
    cp = (ctypes.c_void_p * 3)(*[t.data_ptr() for t in cq])
    lib = _mm.load()
    with _mm.on_device(pr):
        _mm.check(lib.mm_kda_decode_step(_mm.ptr(p), p.numel(), wp, cp, 4, _mm.ptr(fb), _mm.ptr(gb), R, _mm.ptr(A),
                                         _mm.ptr(dtb), lb, sc, _mm.ptr(state), H, K, V, _mm.ptr(w), float(eps),
                                         _mm.ptr(y), _mm.stream_of(pr)), "kda_decode_step")
    return y.reshape(H, V)


def _aligned16(t):
    """t contiguous at a 16-byte aligned address (a copy when a view is not)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def mla_attn_workspace(nh, dv, max_len, device):
    n = int(_mm.load().mm_mla_attn_workspace(int(nh), int(dv), int(max_len)))
    return torch.empty(max(n // 4, 1), device=device, dtype=torch.float32)


def mla_decode_attn(q, k_new, v_new, k_cache, v_cache, pos, scale=None, out=None, workspace=None):
    """One token of an MLA layer. q, k_new [nh, dqk] (any leading shape with nh * dqk elements), v_new [nh, dv];
    k_cache [1, nh, max_len, dqk], v_cache [1, nh, max_len, dv] (bf16, the layer's StaticHybridCache buffers);
    pos: a device tensor holding the position (int64 / int32). Writes the new rows at pos and returns
    out [nh, dv] = softmax(scale * q . K[0..pos]^T) . V[0..pos] (scale defaults to dqk ** -0.5)."""
    _mm.require_gpu(q, k_new, v_new, k_cache, v_cache, pos, out, workspace)
    nh, max_len, dqk = k_cache.shape[-3:]
    dv = v_cache.shape[-1]
    if tuple(v_cache.shape[-3:-1]) != (nh, max_len) or not k_cache.is_contiguous() or not v_cache.is_contiguous():
        raise ValueError("mla_decode_attn: caches must be contiguous [1, nh, max_len, d]")
    qf, kf, vf = (_aligned16(t.reshape(nh, d)) for t, d in ((q, dqk), (k_new, dqk), (v_new, dv)))
    for name, t in (("q", qf), ("k_new", kf), ("v_new", vf), ("k_cache", k_cache), ("v_cache", v_cache)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"mla_decode_attn: {name} must be bf16")
    if pos.dtype not in (torch.int64, torch.int32) or pos.numel() != 1:
        raise ValueError("mla_decode_attn: pos must be a one-element int64 / int32 device tensor")
    y = torch.empty(nh, dv, device=q.device, dtype=torch.bfloat16) if out is None else out.view(nh, dv)
    ws = mla_attn_workspace(nh, dv, max_len, q.device) if workspace is None else workspace
    sc = float(scale) if scale is not None else dqk ** -0.5
    lib = _mm.load()
    with _mm.on_device(q):
        _mm.check(lib.mm_mla_decode_attn(_mm.ptr(qf), _mm.ptr(kf), _mm.ptr(vf), nh, dqk, dv, _mm.ptr(k_cache),
                                         _mm.ptr(v_cache), max_len, _mm.ptr(pos), _mm.dtype_code(pos), sc, _mm.ptr(y),
                                         _mm.ptr(ws), ws.numel() * ws.element_size(), _mm.stream_of(q)),
                  "mla_decode_attn")
    return y


def _token_rows(t, T, n, name):
    """[T, n] view of a tensor holding T tokens of n contiguous elements (e.g. [1, T, heads, d] or a column slice
    of a wider projection output) and its token stride; copied when its rows are not 16-byte aligned."""
    if t.dtype != torch.bfloat16:
        raise ValueError(f"mla_prefill_attn: {name} must be bf16")
    if t.numel() != T * n:
        raise ValueError(f"mla_prefill_attn: {name} must hold {T} tokens of {n} elements (got {tuple(t.shape)})")
    t2 = t.reshape(T, n)
    if t2.stride(1) != 1 or (T > 1 and t2.stride(0) % 8) or t2.data_ptr() % 16:
        t2 = t2.contiguous()
    return t2, t2.stride(0) if T > 1 else n


def mla_prefill_attn(q, k_new, v_new, k_cache, v_cache, pos, scale=None, out=None):
    """T prompt tokens of an MLA layer (the engine's prefill over the static cache, engine.py:938-972, 537-541,
    679-682). q, k_new: T tokens of [nh, dqk] ([T, nh * dqk], [1, T, nh, dqk], or column slices of a projection
    output); v_new: T tokens of [nh, dv]; k_cache [1, nh, max_len, dqk], v_cache [1, nh, max_len, dv] (bf16);
    pos: a one-element int64 / int32 device tensor, the first token's position. Writes the new rows at
    pos .. pos + T - 1 and returns out [T, nh * dv]: token t attends to positions 0 .. pos + t (scale defaults to
    dqk ** -0.5). A prompt that does not fit in the cache leaves it unchanged and returns NaN."""
    _mm.require_gpu(q, k_new, v_new, k_cache, v_cache, pos, out)
    nh, max_len, dqk = k_cache.shape[-3:]
    dv = v_cache.shape[-1]
    if tuple(v_cache.shape[-3:-1]) != (nh, max_len) or not k_cache.is_contiguous() or not v_cache.is_contiguous():
        raise ValueError("mla_prefill_attn: caches must be contiguous [1, nh, max_len, d]")
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"mla_prefill_attn: {name} must be bf16")
    if q.numel() % (nh * dqk):
        raise ValueError(f"mla_prefill_attn: q must hold tokens of [{nh}, {dqk}]")
    T = q.numel() // (nh * dqk)
    qf, qs = _token_rows(q, T, nh * dqk, "q")
    kf, ks = _token_rows(k_new, T, nh * dqk, "k_new")
    vf, vs = _token_rows(v_new, T, nh * dv, "v_new")
    if pos.dtype not in (torch.int64, torch.int32) or pos.numel() != 1:
        raise ValueError("mla_prefill_attn: pos must be a one-element int64 / int32 device tensor")
    y = torch.empty(T, nh * dv, device=q.device, dtype=torch.bfloat16) if out is None else out.view(T, nh * dv)
    if y.dtype != torch.bfloat16 or y.stride(1) != 1 or y.data_ptr() % 8 or (T > 1 and y.stride(0) % 4):
        raise ValueError("mla_prefill_attn: out must be bf16 [T, nh * dv] with 8-byte aligned rows")
    sc = float(scale) if scale is not None else dqk ** -0.5
    lib = _mm.load()
    with _mm.on_device(q):
        _mm.check(lib.mm_mla_prefill_attn(_mm.ptr(qf), qs, _mm.ptr(kf), ks, _mm.ptr(vf), vs, T, nh, dqk, dv,
                                          _mm.ptr(k_cache), _mm.ptr(v_cache), max_len, _mm.ptr(pos),
                                          _mm.dtype_code(pos), sc, _mm.ptr(y), y.stride(0) if T > 1 else nh * dv,
                                          _mm.stream_of(q)), "mla_prefill_attn")
    return y


def embed_rows(table, ids, *, out=None):
    """word_embeddings(ids) (engine.py:686) for a bf16 / fp16 / fp32 table [V, H] with 16-byte aligned rows and
    device ids (int64 / int32, any shape of n elements): returns out [*ids.shape, H], out[i] = table[ids[i]]. An id
    outside [0, V) gives a row of zeros, where torch's embedding stops on a device-side assert."""
    _mm.require_gpu(table, ids, out)
    if table.dim() != 2 or table.stride(1) != 1:
        raise ValueError("embed_rows: table must be [V, H] with contiguous rows")
    if table.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError("embed_rows: table must be bf16, fp16 or fp32")
    if ids.dtype not in (torch.int64, torch.int32):
        raise ValueError("embed_rows: ids must be int64 or int32")
    V, H = table.shape
    idf = ids.reshape(-1)
    if not idf.is_contiguous():
        idf = idf.contiguous()
    n = idf.numel()
    shape = (*ids.shape, H)
    y = torch.empty(shape, device=table.device, dtype=table.dtype) if out is None else out
    if tuple(y.shape) != shape or y.dtype != table.dtype or not y.is_contiguous():
        raise ValueError(f"embed_rows: out must be a contiguous {table.dtype} tensor of shape {shape}")
    lib = _mm.load()
    with _mm.on_device(table):
        _mm.check(lib.mm_embed_rows(_mm.ptr(table), _mm.dtype_code(table), V, H, table.stride(0), _mm.ptr(idf),
                                    _mm.dtype_code(idf), n, _mm.ptr(y), H, _mm.stream_of(table)), "embed_rows")
    return y


def argmax_workspace(rows, n, dtype=torch.bfloat16, device="cuda"):
    """Device workspace for argmax_rows over `rows` rows of n logits of `dtype` (the split form)."""
    nb = int(_mm.load().mm_argmax_rows_workspace_bytes(int(rows), int(n), _mm.dtype_code(torch.empty(0, dtype=dtype))))
    if nb < 0:
        raise ValueError("argmax_workspace: rows >= 0, n >= 1 and bf16 / fp32 logits")
    return torch.empty(max(nb, 16), dtype=torch.uint8, device=device)


def argmax_rows(logits, *, out=None, workspace=None):
    """logits.argmax(-1) (engine.py:688) over the last dim of bf16 / fp32 logits [..., n] (last dim contiguous):
    torch's order, the largest value, NaN above every number, the lowest index among equals. Returns int64
    [...]; out: an int64 device tensor with one element per row (e.g. the [1, 1] token buffer), written in place.
    workspace (from argmax_workspace): the row split over many workgroups, the same results (a long row drawn
    through one CU is slow); calls sharing a workspace must not overlap."""
    _mm.require_gpu(logits, out)
    if logits.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("argmax_rows: logits must be bf16 or fp32")
    n = logits.shape[-1]
    x2 = logits.reshape(-1, n)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    rows = x2.shape[0]
    y = torch.empty(logits.shape[:-1], device=logits.device, dtype=torch.int64) if out is None else out
    if y.dtype != torch.int64 or y.numel() != rows or not y.is_contiguous():
        raise ValueError(f"argmax_rows: out must be a contiguous int64 tensor of {rows} elements")
    lib = _mm.load()
    with _mm.on_device(logits):
        if workspace is None:
            _mm.check(lib.mm_argmax_rows(_mm.ptr(x2), _mm.dtype_code(x2), rows, n, x2.stride(0) if rows > 1 else n,
                                         _mm.ptr(y), _mm.stream_of(logits)), "argmax_rows")
        else:
            _mm.require_gpu(workspace)
            _mm.check(lib.mm_argmax_rows_ws(_mm.ptr(x2), _mm.dtype_code(x2), rows, n, x2.stride(0) if rows > 1 else n,
                                            _mm.ptr(y), _mm.ptr(workspace), workspace.numel() * workspace.element_size(),
                                            _mm.stream_of(logits)), "argmax_rows")
    return y
