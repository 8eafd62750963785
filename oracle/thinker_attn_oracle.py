"""CPU oracle of the thinker's attention mixers (KDA and MLA layers) — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only to check
results against; the product path (ming-voice_amd/) never calls it.

The KDA functions restate the published algorithm of fla-core 0.5.2 (requirements.txt:11), which the reference calls
(engine.py:242-262) and which is not in the reference tree: the recurrent form of Kimi delta attention
(fused_recurrent_kda with its in-kernel l2 norm and gate), fla's ShortConvolution step and FusedRMSNormGated.
Every function computes in float64. Their equivalence to fla's own kernels is PARITY UNPINNED: fla is absent, and
the reference holds no vectors for it. What pins the restatement (tests/test_thinker_attn_oracle.py): closed forms
(one step from a zero state, a zero write strength with unit decay, the softplus gate's sigmoid form), the
Householder matrix form of the same recurrence, T steps against T single steps, torch library routines (conv1d,
rms_norm, scaled_dot_product_attention) and planted mistakes.

The MLA function restates the static-cache update (engine.py:537-548: index_copy_ of the new k, v rows at the
position) and the masked softmax attention over positions 0..pos that the model runs on it (the mask of
engine.py:679-682).
"""
import torch

F64 = torch.float64


def l2norm(x, eps=1e-6):
    """fla's l2norm: x / sqrt(sum(x^2) + eps) over the last dim."""
    return x / torch.sqrt((x * x).sum(-1, keepdim=True) + eps)


def softplus(x, threshold=20.0):
    """log(1 + exp(x)), with x itself above the threshold (torch's softplus default)."""
    return torch.where(x > threshold, x, torch.log1p(torch.exp(torch.clamp(x, max=threshold))))


def kda_gate(g, A_log, dt_bias, lower_bound=None):
    """The in-kernel gate of fused_recurrent_kda: g [T, H, K] -> log decay. x = g + dt_bias[h];
    -exp(A_log[h]) * softplus(x), or lower_bound * sigmoid(exp(A_log[h]) * x) with a lower bound."""
    H, K = g.shape[-2:]
    x = g.to(F64) + dt_bias.to(F64).reshape(H, K)
    a = torch.exp(A_log.to(F64)).reshape(H, 1)
    if lower_bound is None:
        return -a * softplus(x)
    return lower_bound * torch.sigmoid(a * x)


def kda_recurrent(q, k, v, g, beta, state=None, *, scale=None, A_log=None, dt_bias=None, use_qk_l2norm=True,
                  use_gate=True, lower_bound=None):
    """Recurrent Kimi delta attention for one sequence. q, k, g [T, H, K]; v [T, H, V]; beta [T, H]; state [H, K, V]
    (zeros when None). For each token and head: q, k l2-normalised (optional), q *= scale (K ** -0.5 default);
    decay = exp(gate(g)) per key channel; S = decay[:, None] * S; u = beta * (v - S^T k); S = S + k u^T; o = S^T q.
    Returns (o [T, H, V], state [H, K, V]), float64."""
    T, H, K = q.shape
    V = v.shape[-1]
    S = torch.zeros(H, K, V, dtype=F64) if state is None else state.to(F64).clone()
    q, k, v, beta = q.to(F64), k.to(F64), v.to(F64), beta.to(F64)
    if use_qk_l2norm:
        q, k = l2norm(q), l2norm(k)
    q = q * (K ** -0.5 if scale is None else scale)
    lg = kda_gate(g, A_log, dt_bias, lower_bound) if use_gate else g.to(F64)
    o = torch.empty(T, H, V, dtype=F64)
    for t in range(T):
        S = S * torch.exp(lg[t])[:, :, None]
        u = beta[t][:, None] * (v[t] - torch.einsum("hk,hkv->hv", k[t], S))
        S = S + k[t][:, :, None] * u[:, None, :]
        o[t] = torch.einsum("hk,hkv->hv", q[t], S)
    return o, S


def short_conv(x, cache, w, b=None, act=True):
    """ShortConvolution's step form over T tokens: x [T, C]; cache [C, W] (last W inputs, oldest first); w [C, W].
    Each token shifts into the window; y[t] = silu(sum_j w[:, j] * window[:, j] + b). Returns (y, cache)."""
    win = cache.to(F64).clone()
    wf = w.to(F64).reshape(win.shape)
    y = torch.empty(x.shape, dtype=F64)
    for t in range(x.shape[0]):
        win = torch.cat([win[:, 1:], x[t].to(F64)[:, None]], 1)
        acc = (win * wf).sum(1)
        if b is not None:
            acc = acc + b.to(F64)
        y[t] = acc * torch.sigmoid(acc) if act else acc
    return y, win


def rms_norm_gated(x, g, w, eps):
    """FusedRMSNormGated (sigmoid): x * rsqrt(mean(x^2) + eps) * w * sigmoid(g), over the last dim."""
    xf = x.to(F64)
    return xf * torch.rsqrt((xf * xf).mean(-1, keepdim=True) + eps) * w.to(F64) * torch.sigmoid(g.to(F64))


def mla_decode_attn(q, k_new, v_new, k_cache, v_cache, pos, scale=None):
    """One token of an MLA layer: the caches [nh, L, d] take k_new / v_new at row pos; out[h] = softmax(scale *
    q[h] . K[h, :pos+1]^T) . V[h, :pos+1]. Returns (out [nh, dv], k_cache, v_cache), float64 (caches in their dtype)."""
    kc, vc = k_cache.clone(), v_cache.clone()
    kc[:, pos] = k_new.to(kc.dtype)
    vc[:, pos] = v_new.to(vc.dtype)
    d = q.shape[-1]
    s = (q.to(F64)[:, None, :] * kc[:, : pos + 1].to(F64)).sum(-1) * (d ** -0.5 if scale is None else scale)
    p = torch.softmax(s, -1)
    out = (p[:, :, None] * vc[:, : pos + 1].to(F64)).sum(1)
    return out, kc, vc


def mla_prefill_attn(q, k_new, v_new, k_cache, v_cache, pos, scale=None):
    """The T tokens of a prompt through an MLA layer (engine.py:938-972 over the static cache): the caches [nh, L, d]
    take k_new[t] / v_new[t] ([T, nh, d]) at rows pos + t (engine.py:537-541), then token t attends to rows
    0 .. pos + t (the causal mask of engine.py:679-682): out[t, h] = softmax(scale * q[t, h] . K[h, :pos+t+1]^T) .
    V[h, :pos+t+1]. Returns (out [T, nh, dv], k_cache, v_cache), float64 (caches in their dtype)."""
    T = q.shape[0]
    kc, vc = k_cache.clone(), v_cache.clone()
    kc[:, pos:pos + T] = k_new.transpose(0, 1).to(kc.dtype)
    vc[:, pos:pos + T] = v_new.transpose(0, 1).to(vc.dtype)
    d = q.shape[-1]
    n = pos + T
    s = torch.einsum("thd,hjd->htj", q.to(F64), kc[:, :n].to(F64)) * (d ** -0.5 if scale is None else scale)
    keys = torch.arange(n)
    mask = keys[None, :] <= (pos + torch.arange(T))[:, None]  # [T, n]
    s = s.masked_fill(~mask[None], float("-inf"))
    p = torch.softmax(s, -1)
    out = torch.einsum("htj,hjd->thd", p, vc[:, :n].to(F64))
    return out, kc, vc
