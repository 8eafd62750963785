"""CPU oracle of the Ming thinker MoE block — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only to
check results against (or as the timed CPU baseline); the product path (ming-voice_amd/) never calls it.

It restates, in plain torch (fp32 math on the CPU) and numpy (integer work), the algorithm of the reference
kernels and torch paths, with the same rounding points. Each function cites the reference file:line it
follows (paths relative to the Ming Voice sources). How each function is pinned (closed forms, invariants,
brute force, library routines) is in tests/test_oracle.py; none is "parity unpinned" except the sigmoid
group router's equivalence to the remote HF group_limited_topk, which no file in the reference holds.

Rounding points (fused_moe.py:34-38, 60-61, 118-121, 147-148, 196):
  g = bf16(x . Wg^T [* s_g]); u = bf16(x . Wu^T [* s_u]); a = bf16(bf16(silu(g)) * u)
  part = bf16(a . Wd^T [* s_d]); y = bf16(sum_k w_k * part_k)   (fp32 sum over slots in order)
"""
import numpy as np
import torch

BF16 = torch.bfloat16


def _bf(t):
    """Round an fp32 tensor through bf16 (round to nearest even) and back to fp32."""
    return t.to(BF16).float()


# ---------------------------------------------------------------------------------------------- RMSNorm

def rms_norm(x, w, eps):
    """fused_ops.py:16-25: var = mean(x^2) (fp32); y = bf16(x * rsqrt(var + eps)); out = (w * y) in
    promote(w.dtype, x.dtype)."""
    xf = x.float()
    var = (xf * xf).mean(-1, keepdim=True)
    y = _bf(xf * torch.rsqrt(var + eps))
    return (w.float() * y).to(torch.promote_types(w.dtype, x.dtype))


# ----------------------------------------------------------------------------------------------- router

def router_logits(x, w32):
    """fused_ops.py:40-50 / engine.py:328: logits = x_f32 . w32^T (fp32)."""
    return x.float() @ w32.float().t()


def _stable_desc(v):
    """Indices sorting v descending; equal values keep ascending index order (lowest index first)."""
    return torch.sort(v, dim=-1, descending=True, stable=True).indices


def router_select(logits, bias=None, *, scoring="sigmoid", n_group=1, topk_group=1, top_k=6, scale=1.0,
                  append_shared=True):
    """Selection and weights for logits [N, E] -> (ids [N, top_k(+1)] int64, wts [N, top_k(+1)] fp32).

    sigmoid (fused_ops.py:53-93, engine.py:326-333): s = sigmoid(l); r = s + bias; group score = sum of
      the two largest r of each group of E/n_group; keep the topk_group best groups (ties: lowest group);
      top_k of r among kept (ties: lowest expert); w = s / (sum s + 1e-20) * scale.
    softmax (the configs' router): z = l + bias; top_k of z (ties: lowest expert); p = softmax(z);
      w = p / (sum p_selected + 1e-20) * scale.
    The shared expert (id E, weight 1) follows when append_shared.
    """
    logits = logits.float()
    N, E = logits.shape
    b = bias.float() if bias is not None else torch.zeros(E)
    if scoring == "sigmoid":
        score = 1.0 / (1.0 + torch.exp(-logits))
        key = score + b
        if n_group > 1:
            GS = E // n_group
            kg = key.view(N, n_group, GS)
            srt = torch.sort(kg, dim=-1, descending=True, stable=True).values
            second = srt[..., 1] if GS > 1 else torch.full((N, n_group), float("-inf"))
            gscore = srt[..., 0] + second
            keep_g = _stable_desc(gscore)[:, :topk_group]
            gmask = torch.zeros(N, n_group, dtype=torch.bool)
            gmask.scatter_(1, keep_g, True)
            key = torch.where(gmask.repeat_interleave(GS, dim=1), key, torch.full_like(key, float("-inf")))
    elif scoring == "softmax":
        if n_group != 1:
            raise ValueError("softmax scoring takes n_group=1")
        key = logits + b
        score = torch.softmax(key, dim=-1)
    else:
        raise ValueError(scoring)
    idx = _stable_desc(key)[:, :top_k]
    sel = torch.gather(score, 1, idx)
    w = sel / (sel.sum(-1, keepdim=True) + 1e-20) * scale
    if append_shared:
        idx = torch.cat([idx, torch.full((N, 1), E, dtype=idx.dtype)], 1)
        w = torch.cat([w, torch.ones(N, 1)], 1)
    return idx.to(torch.int64), w.float()


# ------------------------------------------------------------------------------------------------ align

def align_blocks(flat, E1, BM):
    """fused_moe.py:154-173 in numpy: stable counting sort of pair indices by expert, each expert's run
    padded to a multiple of BM. Returns (sorted_ids int32 [nb*BM] with pad value P, bexp int32 [nb] with
    -1 past the last used block, nb, expert_offsets int32 [E1+1]). Ids outside [0, E1) are dropped."""
    flat = np.asarray(flat, dtype=np.int64).reshape(-1)
    P = flat.size
    valid = (flat >= 0) & (flat < E1)
    counts = np.bincount(flat[valid], minlength=E1).astype(np.int64)
    padded = (counts + BM - 1) // BM * BM
    pend = np.cumsum(padded)
    pstart = pend - padded
    order = np.argsort(np.where(valid, flat, E1), kind="stable")[: int(valid.sum())]
    se = flat[order]
    cstart = np.cumsum(counts) - counts
    dest = pstart[se] + np.arange(order.size) - cstart[se]
    nb = (P + E1 * (BM - 1) + BM - 1) // BM
    sorted_ids = np.full(nb * BM, P, dtype=np.int32)
    sorted_ids[dest] = order.astype(np.int32)
    bexp = np.searchsorted(pend, np.arange(nb) * BM, side="right")
    bexp = np.where(bexp < E1, bexp, -1).astype(np.int32)
    offsets = np.concatenate([pstart, pend[-1:]]).astype(np.int32)
    return sorted_ids, bexp, nb, offsets


# --------------------------------------------------------------------------------------------- quantise

def quantize_rows_int8(w, scale_dtype=torch.float32):
    """fused_moe.py:199-204: amax = max(max|w|, 1e-8) (fp32); scale = amax / 127;
    q = clamp(round_half_even(w / scale), -127, 127). With bf16 scales, q divides by the rounded scale."""
    amax = w.abs().amax(dim=-1).float().clamp_min(1e-8)
    scale = amax / 127.0
    if scale_dtype == torch.bfloat16:
        scale = _bf(scale)
    q = torch.round(w.float() / scale[..., None]).clamp_(-127, 127).to(torch.int8)
    return q, scale.to(scale_dtype)


# ------------------------------------------------------------------------------------------------ MoE

def _expert_rows(w, e, s, row_lo, row_hi):
    """fp32 weight rows [row_lo, row_hi) of expert e and their row scales (1 for bf16)."""
    wr = w[e, row_lo:row_hi].float()
    sc = s[e, row_lo:row_hi].float() if s is not None else None
    return wr, sc


def moe_pairs(x, w_gu, w_d, ids, s_gu=None, s_d=None):
    """Per-pair expert outputs for x [N, H] and ids [N, NK]:
    returns (a [N*NK, I] bf16, part [N*NK, H] fp32 holding bf16 values), pairs p = t*NK + k.
    Follows fused_moe.py:13-61 (decode) and :92-148 (prefill), grouped per expert like
    dev/test_moe_prefill.py:24-38; ids outside [0, E1) leave zero rows."""
    N, H = x.shape
    NK = ids.shape[1]
    E1, I = w_d.shape[0], w_d.shape[-1]
    flat = ids.reshape(-1).long()
    P = flat.numel()
    a = torch.zeros(P, I, dtype=BF16)
    part = torch.zeros(P, H, dtype=torch.float32)
    xf = x.float()
    for e in torch.unique(flat).tolist():
        if e < 0 or e >= E1:
            continue
        pairs = (flat == e).nonzero().view(-1)
        xe = xf[pairs // NK]
        wg, sg = _expert_rows(w_gu, e, s_gu, 0, I)
        wu, su = _expert_rows(w_gu, e, s_gu, I, 2 * I)
        g = xe @ wg.t()
        u = xe @ wu.t()
        if sg is not None:
            g = g * sg
            u = u * su
        g, u = _bf(g), _bf(u)
        act = _bf(g / (1.0 + torch.exp(-g)))
        ae = (act * u).to(BF16)
        a[pairs] = ae
        wd, sd = _expert_rows(w_d, e, s_d, 0, H)
        pe = ae.float() @ wd.t()
        if sd is not None:
            pe = pe * sd
        part[pairs] = _bf(pe)
    return a, part


def moe(x, w_gu, w_d, ids, weights, s_gu=None, s_d=None, residual=None, return_a=False):
    """MoE block output y [N, H] bf16 = bf16(sum_k weights[:, k] * part_k) (+ residual, rounded again).
    fused_moe.py:60-61 / :147-148 + :196; the residual add is the decoder layer's bf16 add."""
    N, H = x.shape
    NK = ids.shape[1]
    a, part = moe_pairs(x, w_gu, w_d, ids, s_gu, s_d)
    w = weights.float().reshape(N, NK)
    y = torch.zeros(N, H, dtype=torch.float32)
    for k in range(NK):
        y = y + w[:, k : k + 1] * part.view(N, NK, H)[:, k]
    y = _bf(y)
    if residual is not None:
        y = y + residual.float()
    y = y.to(BF16)
    return (y, a) if return_a else y


def moe_int8_fallback(x, q_gu, q_d, s_gu, s_d, ids, weights):
    """engine.py:455-486: the reference's unfused int8 prefill: dequantise with fp16 rounding
    (q.half() * s.half()).to(bf16), then the bf16 per-expert loop; fp32 index_add over slots."""
    d_gu = (q_gu.half() * s_gu[:, :, None].half()).to(BF16)
    d_d = (q_d.half() * s_d[:, :, None].half()).to(BF16)
    return moe(x, d_gu, d_d, ids, weights)


# -------------------------------------------------------------------------------------------- small linear

def small_linear(x, w, b=None, act=0, residual=None, norm=None):
    """fastlinear.py:123-165 for M <= 16 rows: optional RMSNorm prologue (rstd = 1/sqrt(ss/K + eps);
    x -> bf16(bf16(x * rstd) * g)), acc = x . W^T (fp32), + b, act with a bf16 rounding first
    (1 = GELU tanh, 2 = SiLU), residual after a bf16 rounding, cast to x.dtype.
    More than 16 rows take the reference's torch path instead (small_linear_torch)."""
    K = x.shape[-1]
    if x.reshape(-1, K).shape[0] > 16:
        return small_linear_torch(x, w, b, act, residual, norm)
    xf = x.float().reshape(-1, K)
    if norm is not None:
        g, eps = norm
        rstd = 1.0 / torch.sqrt((xf * xf).sum(-1, keepdim=True) / K + eps)
        xf = _bf(_bf(xf * rstd) * g.float())
    acc = xf @ w.float().t()
    if b is not None:
        acc = acc + b.float()
    if act == 1:
        acc = _bf(acc)
        c = 0.7978845608028654 * (acc + 0.044715 * acc * acc * acc)
        t = 2.0 / (1.0 + torch.exp(-2.0 * c)) - 1.0
        acc = 0.5 * acc * (1.0 + t)
    elif act == 2:
        acc = _bf(acc)
        acc = acc / (1.0 + torch.exp(-acc))
    if residual is not None:
        acc = _bf(acc) + residual.float().reshape(acc.shape)
    return acc.to(x.dtype).reshape(*x.shape[:-1], w.shape[0])


def small_linear_torch(x, w, b=None, act=0, residual=None, norm=None):
    """fastlinear.py:151-160, the reference's path for M > 16 rows, as torch computes it on x.dtype tensors:
    F.rms_norm (x * rsqrt(mean(x^2) + eps) * w in fp32, rounded once), F.linear (fp32 accumulation, + b, one
    rounding), F.gelu(approximate="tanh") / F.silu on the rounded output (fp32 inside, rounded), then
    + residual (rounded). Each rounding is to x.dtype. Only the norm differs from the M <= 16 formula, which
    rounds x * rstd before the weight."""
    F = torch.nn.functional
    dt = x.dtype
    K = x.shape[-1]
    xf = x.float().reshape(-1, K)
    if norm is not None:
        g, eps = norm
        xf = (xf * torch.rsqrt((xf * xf).mean(-1, keepdim=True) + eps) * g.float()).to(dt).float()
    acc = xf @ w.float().t()
    if b is not None:
        acc = acc + b.float()
    y = acc.to(dt).float()
    if act == 1:
        y = F.gelu(y, approximate="tanh").to(dt).float()
    elif act == 2:
        y = F.silu(y).to(dt).float()
    y = y.reshape(*x.shape[:-1], w.shape[0])
    if residual is not None:
        y = y + residual.float()
    return y.to(dt)


# ------------------------------------------------------------------------------- reference torch loop

def moe_reference_loop(x, w_gu, w_d, ids, weights):
    """dev/test_moe_prefill.py:24-38, the reference's per-expert torch loop ("what the HF path does: one small
    GEMM pair per active expert"), on x.dtype tensors: pairs sorted by expert (argsort of the flat ids), then
    for each expert with pairs: gu = x[tok] @ W_gu[e]^T, a = silu(gu[:, :I]) * gu[:, I:], and
    index_add of (a @ W_d[e]^T).float() * w into an fp32 [N, H] sum. Returns the fp32 sum. The CPU baseline
    times this loop; torch's own bf16 ops round where the reference's do on the GPU."""
    F = torch.nn.functional
    N, H = x.shape
    NK = ids.shape[1]
    E1, I = w_d.shape[0], w_d.shape[-1]
    y = torch.zeros(N, H, dtype=torch.float32)
    flat = ids.reshape(-1)
    order = flat.argsort()
    counts = torch.bincount(flat, minlength=E1).tolist()
    tok = order // NK
    wf = weights.reshape(-1).float()
    s = 0
    for e, c in enumerate(counts):
        if c:
            t = tok[s:s + c]
            gu = x[t] @ w_gu[e].T
            a = F.silu(gu[:, :I]) * gu[:, I:]
            y.index_add_(0, t, (a @ w_d[e].T).float() * wf[order[s:s + c]][:, None])
        s += c
    return y
