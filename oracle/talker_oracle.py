"""CPU oracle of the Talker's three small kernels — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only to
check results against (or as the timed CPU baseline); the product path (ming-voice_amd/) never calls it.

It restates in plain torch (fp32 on the CPU) the algorithm of fast_talker.py's Triton kernels, with their
rounding points. How each function is pinned (closed forms, the unfused torch path of engine.py's
StaticQwen2, complex-number rotation, torch's scaled_dot_product_attention and silu) is in
tests/test_talker_oracle.py.
"""
import math

import torch
import torch.nn.functional as F

BF16 = torch.bfloat16


def _bf(t):
    """Round an fp32 tensor through bf16 (round to nearest even) and back to fp32."""
    return t.to(BF16).float()


def rope_attn(qkv, cos, sin, heads):
    """fast_talker.py:34-79. qkv [B, S, 3D] bf16; cos, sin [S, HD/2] fp32 (one angle per pair).
    Interleaved pairs (x[2p], x[2p+1]) -> (xe c - xo s, xo c + xe s), rounded to bf16 for q and k (:53-57);
    scores = (sum over pairs of qe'ke' + qo'ko') * HD^-1/2 (:58-59); softmax over the S keys (:60-63); p rounded
    to bf16 (:64); out = p . v rounded to bf16 (:65-69). Returns [B, S, D] bf16."""
    B, S, D3 = qkv.shape
    D = D3 // 3
    HD = D // heads
    P = HD // 2
    x = qkv.float().reshape(B, S, 3, heads, P, 2)
    c = cos.float()[None, :, None, :]
    s = sin.float()[None, :, None, :]

    def rot(t):
        e, o = t[..., 0], t[..., 1]
        return _bf(e * c - o * s), _bf(o * c + e * s)

    qe, qo = rot(x[:, :, 0])
    ke, ko = rot(x[:, :, 1])
    ve, vo = x[:, :, 2, ..., 0], x[:, :, 2, ..., 1]
    # [B, heads, S, P]
    qe, qo, ke, ko, ve, vo = (t.permute(0, 2, 1, 3) for t in (qe, qo, ke, ko, ve, vo))
    sc = (qe @ ke.transpose(-1, -2) + qo @ ko.transpose(-1, -2)) * (1.0 / math.sqrt(HD))
    p = torch.softmax(sc, dim=-1)
    p = _bf(p)
    oe, oo = p @ ve, p @ vo
    out = torch.stack([oe, oo], dim=-1)  # [B, heads, S, P, 2]
    return out.permute(0, 2, 1, 3, 4).reshape(B, S, D).to(BF16)


def _rotate_half_fused(x, c, s):
    """fast_talker.py:176-187: x'[d] = x[d] c[d] + sign(d) x[(d + HD/2) % HD] s[d], sign = -1 below HD/2."""
    HD = x.shape[-1]
    half = HD // 2
    partner = (torch.arange(HD) + half) % HD
    sign = torch.where(torch.arange(HD) < half, -1.0, 1.0)
    return x * c + sign * x[..., partner] * s


def qwen_decode_attn(qkv, k_cache, v_cache, pos, inv_freq, scale, nh, nkv, hd, block=64):
    """fast_talker.py:165-212 for one token. qkv [(nh + 2 nkv) hd] bf16; k_cache, v_cache [nkv, max_len, hd]
    bf16 (modified in place at row pos, :191-193); pos int; inv_freq [hd/2] fp32.
    Angles f = pos * inv_freq[d % (hd/2)] with cos / sin rounded to bf16 (:178-180); q and k rotated and
    rounded to bf16 (:184-187); online softmax in fp32 starting from the current position (m = q.k scale,
    l = 1, acc = v, :195-197) and walking the cached prefix [0, pos) in blocks of `block` (:199-211).
    Returns out [nh * hd] bf16."""
    G = nh // nkv
    half = hd // 2
    d = torch.arange(hd)
    f = torch.tensor(float(pos), dtype=torch.float32) * inv_freq.float()[d % half]
    c = _bf(torch.cos(f))
    s = _bf(torch.sin(f))
    x = qkv.float()
    q = _bf(_rotate_half_fused(x[: nh * hd].reshape(nh, hd), c, s))
    k = _bf(_rotate_half_fused(x[nh * hd:(nh + nkv) * hd].reshape(nkv, hd), c, s))
    v = x[(nh + nkv) * hd:(nh + 2 * nkv) * hd].reshape(nkv, hd)
    k_cache[:, pos] = k.to(BF16)
    v_cache[:, pos] = v.to(BF16)
    kvh = torch.arange(nh) // G
    kq, vq = k[kvh], v[kvh]  # [nh, hd]: each query head's own k / v
    m = (q * kq).sum(-1) * scale
    l = torch.ones(nh)
    acc = vq.clone()
    K = k_cache.float()[kvh]  # [nh, max_len, hd]
    V = v_cache.float()[kvh]
    for start in range(0, pos, block):
        stop = min(start + block, pos)
        sc = (K[:, start:stop] * q[:, None, :]).sum(-1) * scale  # [nh, n]
        m_new = torch.maximum(m, sc.max(-1).values)
        alpha = torch.exp(m - m_new)
        p = torch.exp(sc - m_new[:, None])
        acc = acc * alpha[:, None] + (p[:, :, None] * V[:, start:stop]).sum(1)
        l = l * alpha + p.sum(-1)
        m = m_new
    return (acc / l[:, None]).reshape(-1).to(BF16)


def silu_mul(gu, inter):
    """fast_talker.py:215-222: g, u = gu[..., :I], gu[..., I:2I]; out = bf16(bf16(g / (1 + exp(-g))) * u)."""
    g = gu[..., :inter].float()
    u = gu[..., inter:2 * inter].float()
    g = _bf(g / (1.0 + torch.exp(-g)))
    return (g * u).to(BF16)


def fast_qwen2_step(x, layers, k_cache, v_cache, pos, inv_freq, nh, nkv, hd, final_norm):
    """fast_talker.py:247-262, one token through the Talker LLM: per layer
    qkv = small_linear(x, wqkv, bqkv, norm=n1); a = decode attention (:255-256); h = small_linear(a, wo) + h;
    gu = small_linear(h, wgu, norm=n2); h = small_linear(silu_mul(gu), wd) + h; then torch's rms_norm.
    layers: dicts of CPU tensors wqkv, bqkv, wo, wgu, wd, n1 = (w, eps), n2; k_cache, v_cache
    [layers, nkv, max_len, hd] are written at row pos. Returns [1, 1, H] bf16."""
    from oracle.moe_oracle import small_linear
    H = x.shape[-1]
    h = x.reshape(1, H)
    scale = 1.0 / math.sqrt(hd)
    for i, L in enumerate(layers):
        qkv = small_linear(h, L["wqkv"], L["bqkv"], norm=L["n1"])
        a = qwen_decode_attn(qkv.reshape(-1), k_cache[i], v_cache[i], pos, inv_freq, scale, nh, nkv, hd)
        h = small_linear(a.reshape(1, -1), L["wo"], residual=h)
        gu = small_linear(h, L["wgu"], norm=L["n2"])
        h = small_linear(silu_mul(gu, L["wgu"].shape[0] // 2), L["wd"], residual=h)
    w, eps = final_norm
    return F.rms_norm(h.float(), (H,), w.float(), eps).to(BF16).reshape(1, 1, H)


def static_qwen2_step_fp32(x, layers, k_cache, v_cache, pos, inv_freq, nh, nkv, hd, final_norm):
    """engine.py:1268-1293 (StaticQwen2.forward) for one token in fp32, with HF Qwen2 modules' math:
    RMSNorm x * rsqrt(mean(x^2) + eps) * w; q/k/v = Linear (+ bias); rotate-half rotary with emb = [f, f];
    cache write at pos; SDPA over the GQA-expanded cache with mask ar <= pos; o_proj + residual;
    down(silu(gate(x)) * up(x)) + residual; final RMSNorm. layers: dicts as for fast_qwen2_step (the fused
    q|k|v and gate|up weights are split back by rows). k_cache, v_cache fp32 [layers, nkv, max_len, hd]."""
    H = x.shape[-1]
    h = x.float().reshape(1, H)

    def rms(t, n):
        w, eps = n
        return t * torch.rsqrt((t * t).mean(-1, keepdim=True) + eps) * w.float()

    def rotate_half(t):
        t1, t2 = t.chunk(2, dim=-1)
        return torch.cat((-t2, t1), dim=-1)

    f = float(pos) * inv_freq.float()
    emb = torch.cat([f, f])
    cos, sin = emb.cos(), emb.sin()
    rep = nh // nkv
    max_len = k_cache.shape[2]
    mask = (torch.arange(max_len) <= pos)[None, None]
    for i, L in enumerate(layers):
        xn = rms(h, L["n1"])
        qkv = xn @ L["wqkv"].float().t() + L["bqkv"].float()
        q = qkv[0, : nh * hd].reshape(nh, hd)
        k = qkv[0, nh * hd:(nh + nkv) * hd].reshape(nkv, hd)
        v = qkv[0, (nh + nkv) * hd:].reshape(nkv, hd)
        q = q * cos + rotate_half(q) * sin
        k = k * cos + rotate_half(k) * sin
        k_cache[i, :, pos] = k
        v_cache[i, :, pos] = v
        kk = k_cache[i][:, None].expand(nkv, rep, max_len, hd).reshape(nh, max_len, hd)
        vv = v_cache[i][:, None].expand(nkv, rep, max_len, hd).reshape(nh, max_len, hd)
        o = F.scaled_dot_product_attention(q[:, None], kk, vv, attn_mask=mask)
        h = h + o.reshape(1, -1) @ L["wo"].float().t()
        xn = rms(h, L["n2"])
        inter = L["wgu"].shape[0] // 2
        gu = xn @ L["wgu"].float().t()
        h = h + (F.silu(gu[:, :inter]) * gu[:, inter:]) @ L["wd"].float().t()
    return rms(h, final_norm).reshape(1, 1, H)


def _dit_block(b, h, cos, sin):
    """fast_talker.py:97-102 on the oracle's small_linear and rope_attn."""
    from oracle.moe_oracle import small_linear
    att = rope_attn(small_linear(h, b["wqkv"], b["bqkv"], norm=b["n1"]), cos, sin, b["heads"])
    h = small_linear(att, b["wo"], b["bo"], residual=h)
    f = small_linear(h, b["w1"], b["b1"], act=1, norm=b["n2"])
    return small_linear(f, b["w2"], b["b2"], residual=h)


def fast_tail(P, hidden, hist, noise):
    """fast_talker.py:139-160 (FastTail.__call__) on the CPU: P holds FastTail's hoisted constants as CPU
    tensors (c_w, c_b, x_w, x_b, t_emb list, dts list, cfg, blocks / a_blocks as dicts, cos3 / sin3,
    cos2 / sin2, f_norm, f_w, f_b, cls, a_x_w, a_x_b, a_norm, a_w, a_b, s_w, s_b). The latent update
    y + (pred + (pred - null) * cfg) * dt runs in bf16 torch ops in the same order as the reference.
    Returns (latent [1, 1, L], next input [1, 1, H], stop probability)."""
    from oracle.moe_oracle import small_linear
    D = P["x_w"].shape[0]
    c = small_linear(hidden.reshape(1, -1), P["c_w"], P["c_b"])
    c2 = torch.cat([c, P["c_b"].reshape(1, -1)], 0)
    he = small_linear(hist.reshape(1, -1), P["x_w"], P["x_b"])
    y = noise.reshape(1, -1)
    for s, dt in enumerate(P["dts"]):
        ye = small_linear(y, P["x_w"], P["x_b"])
        h = torch.stack([c2 + P["t_emb"][s], he.expand(2, D), ye.expand(2, D)], 1)
        for b in P["blocks"]:
            h = _dit_block(b, h, P["cos3"], P["sin3"])
        out = small_linear(h[:, -1], P["f_w"], P["f_b"], norm=P["f_norm"])
        pred, null = out[0:1], out[1:2]
        y = y + (pred + (pred - null) * P["cfg"]) * dt
    Da = P["a_x_w"].shape[0]
    a = torch.stack([P["cls"].reshape(1, Da), small_linear(y, P["a_x_w"], P["a_x_b"])], 1)
    for b in P["a_blocks"]:
        a = _dit_block(b, a, P["cos2"], P["sin2"])
    x_next = small_linear(a[:, 0], P["a_w"], P["a_b"], norm=P["a_norm"]).reshape(1, 1, -1)
    stop = small_linear(hidden.reshape(1, -1), P["s_w"], P["s_b"]).float().softmax(-1)[0, 1]
    return y.reshape(1, 1, -1), x_next, stop


def _cpu(v):
    if torch.is_tensor(v):
        return v.detach().cpu()
    if isinstance(v, (tuple, list)):
        return type(v)(_cpu(x) for x in v)
    return v


def tail_constants(ft):
    """FastTail's hoisted constants (attributes of a fast_talker.FastTail) as CPU tensors: fast_tail's P."""
    keys = ("c_w", "c_b", "x_w", "x_b", "t_emb", "dts", "cfg", "cos3", "sin3", "cos2", "sin2", "f_norm", "f_w", "f_b",
            "cls", "a_x_w", "a_x_b", "a_norm", "a_w", "a_b", "s_w", "s_b")
    P = {k: _cpu(getattr(ft, k)) for k in keys}
    bk = ("heads", "wqkv", "bqkv", "wo", "bo", "n1", "n2", "w1", "b1", "w2", "b2")
    P["blocks"] = [{k: _cpu(getattr(b, k)) for k in bk} for b in ft.blocks]
    P["a_blocks"] = [{k: _cpu(getattr(b, k)) for k in bk} for b in ft.a_blocks]
    return P
