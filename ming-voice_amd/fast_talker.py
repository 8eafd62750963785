"""The Talker's per-token work on hand-written gfx950 HIP kernels (drop-in for the reference fast_talker.py).

  rope_attn(qkv, cos, sin, heads)      interleaved-rotary attention over 2-3 tokens per (batch, head), the
                                       DiT / aggregator blocks' attention (fast_talker.py:34-79)
  qwen_decode_attn(qkv, k, v, pos, ...) single-token GQA decode attention over StaticQwen2's KV cache,
                                       writing this token's k / v at `pos` (fast_talker.py:165-212)
  silu_mul(gu, out=None)               bf16(bf16(silu(g)) * u) of the Qwen2 MLP (fast_talker.py:215-222)
  gate_up_silu(x, wgu, norm=None)      silu_mul(small_linear(x, wgu, norm=norm)) in one kernel, bit for bit
  FastQwen2Step                        the Talker LLM decode step built from small_linear and the kernels
                                       above (fast_talker.py:225-262)
  FastTail                             the per-latent flow-matching DiT loop, aggregator and stop head on
                                       small_linear and rope_attn (fast_talker.py:82-160)

Every op runs on torch's current stream, allocates only with torch (so it can be captured in a graph),
and raises if the HIP library is missing: there is no CPU or Triton path.
"""
import math

import torch
import torch.nn.functional as F

import _mingmoe as _mm
from fastlinear import small_linear

__all__ = ["rope_attn", "qwen_decode_attn", "silu_mul", "gate_up_silu", "cfg_update", "FastQwen2Step", "FastTail",
           "decode_attn_workspace"]


def rope_attn(qkv, cos, sin, heads):
    """qkv [B, S, 3D] bf16 (q | k | v); cos, sin [S, HD/2] fp32 (one angle per interleaved pair, as
    _rope_tables builds them). Returns the attention output [B, S, D] bf16 (fast_talker.py:72-79).
    S <= 8; HD = D / heads even and <= 256."""
    _mm.require_gpu(qkv, cos, sin)
    if qkv.dim() != 3 or qkv.shape[-1] % 3:
        raise ValueError(f"rope_attn: qkv must be [B, S, 3D] (got {tuple(qkv.shape)})")
    B, S, D3 = qkv.shape
    D = D3 // 3
    if D % heads:
        raise ValueError(f"rope_attn: dim {D} is not divisible by heads={heads}")
    P = D // heads // 2
    if qkv.dtype != torch.bfloat16:
        raise ValueError(f"rope_attn: qkv must be bf16 (got {qkv.dtype})")
    for name, t in (("cos", cos), ("sin", sin)):
        if t.dtype != torch.float32 or t.numel() != S * P:
            raise ValueError(f"rope_attn: {name} must be fp32 [S={S}, HD/2={P}] (got {t.dtype} {tuple(t.shape)})")
    qkv = qkv if qkv.is_contiguous() else qkv.contiguous()
    cos = cos if cos.is_contiguous() else cos.contiguous()
    sin = sin if sin.is_contiguous() else sin.contiguous()
    out = torch.empty(B, S, D, device=qkv.device, dtype=qkv.dtype)
    lib = _mm.load()
    with _mm.on_device(qkv):
        _mm.check(lib.mm_rope_attn(_mm.ptr(qkv), B, S, D, int(heads), _mm.ptr(cos), _mm.ptr(sin), _mm.ptr(out),
                                   _mm.stream_of(qkv)), "rope_attn")
    return out


def decode_attn_workspace(nh, hd, max_len, device):
    """The fp32 workspace qwen_decode_attn needs (no initialisation needed); reusable across calls and layers
    on one stream."""
    n = _mm.load().mm_decode_attn_workspace(int(nh), int(hd), int(max_len))
    if n <= 0:
        raise ValueError(f"decode_attn_workspace: bad shape nh={nh} hd={hd} max_len={max_len}")
    return torch.empty((n + 3) // 4, dtype=torch.float32, device=device)


def qwen_decode_attn(qkv, k_cache, v_cache, pos, inv_freq, out, max_len, scale, nh, nkv, hd, workspace=None):
    """One decode token of the Talker's Qwen2 attention (fast_talker.py:165-212, launched at :255-256).

    qkv: [1, (nh + 2 nkv) hd] bf16 (the fused q | k | v projection); k_cache, v_cache: one layer of
    StaticQwen2's cache, [1, nkv, max_len, hd] bf16, written at row pos; pos: [1] int64 (or int32) device
    tensor; inv_freq: [hd/2] fp32; out: [1, nh hd] bf16 or None (allocated). Returns out.
    A pos outside [0, max_len) leaves the caches untouched and gives NaN outputs."""
    _mm.require_gpu(qkv, k_cache, v_cache, pos, inv_freq, out, workspace)
    nh, nkv, hd, max_len = int(nh), int(nkv), int(hd), int(max_len)
    if qkv.dtype != torch.bfloat16 or qkv.numel() != (nh + 2 * nkv) * hd or not qkv.is_contiguous():
        raise ValueError(f"qwen_decode_attn: qkv must be contiguous bf16 with (nh + 2 nkv) hd = "
                         f"{(nh + 2 * nkv) * hd} elements (got {qkv.dtype} {tuple(qkv.shape)})")
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        if c.dtype != torch.bfloat16 or c.numel() != nkv * max_len * hd or not c.is_contiguous():
            raise ValueError(f"qwen_decode_attn: {name} must be contiguous bf16 [nkv, max_len, hd] = "
                             f"[{nkv}, {max_len}, {hd}] (got {c.dtype} {tuple(c.shape)})")
    if pos.numel() != 1 or pos.dtype not in (torch.int64, torch.int32):
        raise ValueError("qwen_decode_attn: pos must be a one-element int64 or int32 tensor")
    if inv_freq.dtype != torch.float32 or inv_freq.numel() != hd // 2 or not inv_freq.is_contiguous():
        raise ValueError(f"qwen_decode_attn: inv_freq must be contiguous fp32 [{hd // 2}]")
    if out is None:
        out = torch.empty(1, nh * hd, device=qkv.device, dtype=torch.bfloat16)
    elif out.dtype != torch.bfloat16 or out.numel() != nh * hd or not out.is_contiguous():
        raise ValueError(f"qwen_decode_attn: out must be contiguous bf16 with nh hd = {nh * hd} elements")
    if workspace is None:
        workspace = decode_attn_workspace(nh, hd, max_len, qkv.device)
    lib = _mm.load()
    with _mm.on_device(qkv):
        _mm.check(lib.mm_qwen_decode_attn(_mm.ptr(qkv), nh, nkv, hd, _mm.ptr(k_cache), _mm.ptr(v_cache), max_len,
                                          _mm.ptr(pos), _mm.dtype_code(pos), _mm.ptr(inv_freq), float(scale),
                                          _mm.ptr(out), _mm.ptr(workspace),
                                          workspace.numel() * workspace.element_size(), _mm.stream_of(qkv)),
                  "qwen_decode_attn")
    return out


def silu_mul(gu, out=None):
    """gu [..., 2I] bf16 = [g | u] -> bf16(bf16(silu(g)) * u) [..., I] (fast_talker.py:215-222)."""
    _mm.require_gpu(gu, out)
    if gu.dtype != torch.bfloat16 or gu.shape[-1] % 2:
        raise ValueError(f"silu_mul: gu must be bf16 with an even last dim (got {gu.dtype} {tuple(gu.shape)})")
    I = gu.shape[-1] // 2
    g2 = gu.reshape(-1, 2 * I)
    if g2.stride(-1) != 1:
        g2 = g2.contiguous()
    if out is None:
        out = torch.empty(*gu.shape[:-1], I, device=gu.device, dtype=gu.dtype)
    o2 = out.reshape(-1, I)
    if o2.shape[0] != g2.shape[0] or out.dtype != torch.bfloat16 or o2.stride(-1) != 1 or o2.data_ptr() != out.data_ptr():
        raise ValueError("silu_mul: out must be bf16 [..., I] with the rows of gu and a contiguous last dim")
    lib = _mm.load()
    with _mm.on_device(gu):
        _mm.check(lib.mm_silu_mul(_mm.ptr(g2), g2.shape[0], I, g2.stride(0), _mm.ptr(o2), o2.stride(0),
                                  _mm.stream_of(gu)), "silu_mul")
    return out


def cfg_update(y, pred_null, cfg, dt, out=None):
    """y + (pred + (pred - null) * cfg) * dt for bf16 y [1, L], pred_null [2, L] (rows pred, null) and a
    one-element dt tensor, rounded to bf16 after every operation exactly as the torch expression of
    fast_talker.py:151-152 is, in one kernel. Returns out (a new [1, L] tensor by default; may be y)."""
    _mm.require_gpu(y, pred_null, dt, out)
    L = y.shape[-1]
    if y.dtype != torch.bfloat16 or pred_null.dtype != torch.bfloat16 or y.numel() != L or not y.is_contiguous():
        raise ValueError("cfg_update: y must be a contiguous bf16 [1, L] row and pred_null bf16")
    if pred_null.dim() != 2 or pred_null.shape[0] != 2 or pred_null.shape[1] != L or pred_null.stride(1) != 1:
        raise ValueError(f"cfg_update: pred_null must be [2, {L}] with a contiguous last dim")
    # a bf16 dt (any one-element shape) or a 0-dim fp32 dt keep the expression in bf16; a [1] fp32 dt would
    # promote it to fp32 in torch, which this kernel does not reproduce
    if dt.numel() != 1 or not (dt.dtype == torch.bfloat16 or (dt.dtype == torch.float32 and dt.dim() == 0)):
        raise ValueError("cfg_update: dt must be a one-element bf16 tensor or a 0-dim fp32 tensor")
    out = torch.empty_like(y) if out is None else out
    lib = _mm.load()
    with _mm.on_device(y):
        _mm.check(lib.mm_cfg_update(_mm.ptr(y), _mm.ptr(pred_null), pred_null.stride(0), L, float(cfg), _mm.ptr(dt),
                                    _mm.dtype_code(dt), _mm.ptr(out), _mm.stream_of(y)), "cfg_update")
    return out


def gate_up_silu(x, wgu, norm=None, out=None):
    """x [..., K] bf16; wgu [2I, K] bf16 (gate rows, then up rows); norm: (gamma, eps) RMSNorm prologue.
    Returns bf16(bf16(silu(g)) * u) [..., I], equal bit for bit to silu_mul(small_linear(x, wgu, norm=norm))
    (fast_talker.py:258-260) without the [..., 2I] intermediate. At most 16 rows, K <= 8192."""
    g = norm[0] if norm is not None else None
    _mm.require_gpu(x, wgu, out, g)
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    for name, t in (("x", x2), ("wgu", wgu), ("norm gamma", g)):
        if t is not None and t.dtype != torch.bfloat16:
            raise ValueError(f"gate_up_silu: {name} must be bf16 (got {t.dtype})")
    if wgu.dim() != 2 or wgu.shape[1] != K or wgu.shape[0] % 2 or wgu.stride(1) != 1:
        raise ValueError(f"gate_up_silu: wgu must be [2I, {K}] with a contiguous last dim (got {tuple(wgu.shape)})")
    if g is not None and not g.is_contiguous():
        g = g.contiguous()
    I = wgu.shape[0] // 2
    M = x2.shape[0]
    y = torch.empty(M, I, device=x.device, dtype=torch.bfloat16) if out is None else out.view(M, I)
    lib = _mm.load()
    with _mm.on_device(x):
        _mm.check(lib.mm_small_linear_glu(_mm.ptr(x2), M, K, x2.stride(0), _mm.ptr(wgu), I, wgu.stride(0), _mm.ptr(g),
                                          float(norm[1]) if norm is not None else 0.0, _mm.ptr(y), y.stride(0),
                                          _mm.stream_of(x)), "gate_up_silu")
    return y.reshape(*x.shape[:-1], I)


def _fuse(mods, attr="weight"):
    """One contiguous tensor holding the `attr` of each Linear in mods, stacked along dim 0; each module's
    parameter becomes a view into it, so the weights are held once (fast_talker.py:21-31)."""
    parts = [getattr(m, attr) for m in mods]
    fused = torch.cat([p.detach() for p in parts], dim=0).contiguous()
    row = 0
    for p in parts:
        p.data = fused[row:row + p.shape[0]]
        row += p.shape[0]
    return fused


class _Block:
    """One DiT / aggregator transformer block on the fused kernels (fast_talker.py:82-102):
    h = h + to_out(rope_attn(q|k|v(RMSNorm1(h)))); h = h + W2(GELU_tanh(W1(RMSNorm2(h)))), every bias, norm,
    activation and residual in a small_linear prologue or epilogue."""

    def __init__(self, blk):
        at = blk.attn
        if at.q_norm is not None or at.pe_attn_head is not None:
            raise ValueError("DiT block with q/k norms or a positional attention head is not supported")
        ff = blk.mlp.ff
        if ff[0][1].approximate != "tanh":
            raise ValueError("DiT feed-forward must use GELU(approximate='tanh')")
        self.heads = at.heads
        self.wqkv = _fuse([at.to_q, at.to_k, at.to_v])
        self.bqkv = _fuse([at.to_q, at.to_k, at.to_v], "bias")
        self.wo, self.bo = at.to_out[0].weight, at.to_out[0].bias
        self.n1 = (blk.norm1.weight, blk.norm1.eps)
        self.n2 = (blk.norm2.weight, blk.norm2.eps)
        self.w1, self.b1 = ff[0][0].weight, ff[0][0].bias
        self.w2, self.b2 = ff[2].weight, ff[2].bias

    def __call__(self, h, cos, sin):
        att = rope_attn(small_linear(h, self.wqkv, self.bqkv, norm=self.n1), cos, sin, self.heads)
        h = small_linear(att, self.wo, self.bo, residual=h)
        f = small_linear(h, self.w1, self.b1, act=1, norm=self.n2)
        return small_linear(f, self.w2, self.b2, residual=h)


def _rope_tables(rotary, n):
    """cos / sin [n, hd/2] fp32 of the block's rotary embedding: forward_from_seq_len gives each pair's angle
    twice (interleaved), so every other column is taken (fast_talker.py:105-108)."""
    freqs, _ = rotary.forward_from_seq_len(n)
    ang = freqs[0, :, 0::2].float()
    return ang.cos().contiguous(), ang.sin().contiguous()


class FastTail:
    """y_latent, next_input_embedding, stop_prob = tail(hidden, history, noise) (fast_talker.py:111-160).

    Flow matching with classifier-free guidance at temperature 0: per step the DiT runs on a batch of two
    3-token sequences [condition + timestep, history, current latent] (conditioned and null rows), and
    y += (pred + (pred - null) * cfg) * dt. Then the aggregator maps [cls, latent] to the next LLM input and
    the stop head gives P(stop). Everything constant over the steps (timestep and condition embeddings,
    rotary tables, the cls token) is computed once here."""

    def __init__(self, talker, ts, dts, cfg_strength):
        t = talker.t
        dit, agg = t.cfm.model, t.aggregator
        if getattr(dit, "spk_embedder", None) is not None:
            raise ValueError("DiT with a speaker embedder is not supported")
        dev = t.stop_head.weight.device
        self.cfg = cfg_strength
        self.dts = [d.reshape(1) for d in dts]
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            self.t_emb = [dit.t_embedder(ts[i].reshape(1)).to(torch.bfloat16) for i in range(len(self.dts))]
            self.t_emb_all = torch.cat(self.t_emb, 0)  # [steps, D]
            self.cls = agg.word_embedder(torch.zeros(1, 1, dtype=torch.long, device=dev)).to(torch.bfloat16)
        self.c_w, self.c_b = dit.c_embedder.cond_embedder.weight, dit.c_embedder.cond_embedder.bias
        self.null_c = self.c_b.reshape(1, -1)  # the condition embedder of a zero condition is its bias
        self.x_w, self.x_b = dit.x_embedder.weight, dit.x_embedder.bias
        self.f_norm = (dit.final_layer.norm_final.weight, dit.final_layer.norm_final.eps)
        self.f_w, self.f_b = dit.final_layer.linear.weight, dit.final_layer.linear.bias
        self.blocks = [_Block(b) for b in dit.blocks]
        self.cos3, self.sin3 = _rope_tables(dit.rotary_embed, 3)
        self.a_x_w, self.a_x_b = agg.x_embedder.weight, agg.x_embedder.bias
        self.a_blocks = [_Block(b) for b in agg.blocks]
        self.cos2, self.sin2 = _rope_tables(agg.rotary_embed, 2)
        self.a_norm = (agg.final_layer.norm_final.weight, agg.final_layer.norm_final.eps)
        self.a_w, self.a_b = agg.final_layer.linear.weight, agg.final_layer.linear.bias
        self.s_w, self.s_b = t.stop_head.weight, t.stop_head.bias

    def __call__(self, hidden, hist, noise):
        D = self.x_w.shape[0]
        steps = len(self.dts)
        cond = torch.cat([small_linear(hidden.reshape(1, -1), self.c_w, self.c_b), self.null_c], 0)  # [2, D]
        # the DiT input of every step, [steps, 2, 3, D]: condition + timestep, history, current latent; the
        # first two are known now, the latent slot is written by the x_embedder at each step
        hs = torch.empty(steps, 2, 3, D, device=cond.device, dtype=cond.dtype)
        torch.add(cond[None], self.t_emb_all[:, None], out=hs[:, :, 0])
        hs[:, :, 1] = small_linear(hist.reshape(1, -1), self.x_w, self.x_b)
        y = noise.reshape(1, -1)
        for i, dt in enumerate(self.dts):
            small_linear(y.expand(2, -1), self.x_w, self.x_b, out=hs[i, :, 2])  # both rows at once
            h = hs[i]
            for blk in self.blocks:
                h = blk(h, self.cos3, self.sin3)
            out = small_linear(h[:, -1], self.f_w, self.f_b, norm=self.f_norm)  # [2, latent]: pred, null
            y = cfg_update(y, out, self.cfg, dt)  # y + (pred + (pred - null) * cfg) * dt
        Da = self.a_x_w.shape[0]
        a = torch.stack([self.cls.reshape(1, Da), small_linear(y, self.a_x_w, self.a_x_b)], 1)  # [1, 2, Da]
        for blk in self.a_blocks:
            a = blk(a, self.cos2, self.sin2)
        x_next = small_linear(a[:, 0], self.a_w, self.a_b, norm=self.a_norm).reshape(1, 1, -1)
        stop = small_linear(hidden.reshape(1, -1), self.s_w, self.s_b).float().softmax(-1)[0, 1]
        return y.reshape(1, 1, -1), x_next, stop


class FastQwen2Step:
    """Single-token decode of the Talker's Qwen2 over StaticQwen2's static KV cache (fast_talker.py:225-262).

    Per layer: small_linear(RMSNorm -> fused q|k|v + bias), qwen_decode_attn (rotary, cache write at pos,
    attention), small_linear(o_proj + residual), gate_up_silu(RMSNorm -> fused gate|up -> silu_mul, one
    kernel), small_linear(down_proj + residual); the final norm is torch's rms_norm as in the reference."""

    def __init__(self, static_llm):
        m = static_llm.m
        self.sl = static_llm
        self.nh, self.nkv, self.hd = static_llm.nh, static_llm.nkv, static_llm.hd
        self.scale = 1.0 / math.sqrt(self.hd)
        self.layers = []
        for layer in m.layers:
            at, mlp = layer.self_attn, layer.mlp
            self.layers.append({
                "wqkv": _fuse([at.q_proj, at.k_proj, at.v_proj]),
                "bqkv": _fuse([at.q_proj, at.k_proj, at.v_proj], "bias"),
                "wo": at.o_proj.weight,
                "wgu": _fuse([mlp.gate_proj, mlp.up_proj]),
                "wd": mlp.down_proj.weight,
                "n1": (layer.input_layernorm.weight, layer.input_layernorm.variance_epsilon),
                "n2": (layer.post_attention_layernorm.weight, layer.post_attention_layernorm.variance_epsilon),
            })
        self.norm = (m.norm.weight, m.norm.variance_epsilon)
        self._ws = {}

    def _workspace(self, device):
        ws = self._ws.get(device)
        if ws is None:
            ws = decode_attn_workspace(self.nh, self.hd, self.sl.max_len, device)
            self._ws[device] = ws
        return ws

    def __call__(self, x, pos):
        """x: [1, 1, H] input embedding; pos: [1] long device tensor (position of x).
        Returns the final-normed hidden state [1, 1, H]."""
        H = x.shape[-1]
        h = x.reshape(1, H)
        sl = self.sl
        ws = self._workspace(h.device)
        for i, L in enumerate(self.layers):
            qkv = small_linear(h, L["wqkv"], L["bqkv"], norm=L["n1"])
            a = qwen_decode_attn(qkv, sl.k[i], sl.v[i], pos, sl.inv_freq, None, sl.max_len, self.scale, self.nh,
                                 self.nkv, self.hd, workspace=ws)
            h = small_linear(a, L["wo"], None, residual=h)
            act = gate_up_silu(h, L["wgu"], norm=L["n2"])  # = silu_mul(small_linear(h, wgu, norm=n2))
            h = small_linear(act, L["wd"], None, residual=h)
        return F.rms_norm(h, (H,), self.norm[0], self.norm[1]).reshape(1, 1, H)
