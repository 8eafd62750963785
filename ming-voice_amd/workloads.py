"""Seeded synthetic inputs of the thinker MoE block and the composed block forward.

Shapes of the benchmarked block (a Ling-lite-like thinker): hidden 2048, 64 routed experts of
intermediate 1408 plus one always-on shared expert (slot 64), softmax top-6 router. Weights ~ N(0, 0.02)
in bf16 (the router kept in fp32 like the thinker's `w32`, engine.py:324), the RMSNorm weight ~ 1 + N(0, 0.02).
Every tensor comes from its own seeded torch generator on the device it is drawn on (CPU and GPU
generators give different values for one seed), so a run that compares against the CPU oracle draws on
one device and copies.

  block(...)            one MoE block's weights (optionally int8 experts with bf16 row scales)
  tokens(n, ...)        x ~ N(0, 1) bf16 [n, hidden]
  ragged_bias(...)      router bias ~ N(0, 0.5): ragged per-expert token counts (512-token prefill)
  zipf_bias(...)        router bias log p_e, p_e ~ rank^-1.2 under a fixed permutation (2048-token prefill)
  moe_block_forward     RMSNorm -> router -> MoE (+ residual) through the HIP kernels
"""
import math

import torch

HIDDEN, INTER, EXPERTS, TOP_K = 2048, 1408, 64, 6
EPS = 1e-6
VOCAB = 126464


def _gen(seed, device):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def normal(shape, std, seed, device="cpu", dtype=torch.bfloat16, mean=0.0):
    """N(mean, std^2) drawn in fp32 from a generator seeded with `seed`, then cast."""
    t = torch.randn(shape, generator=_gen(seed, device), device=device, dtype=torch.float32)
    if std != 1.0:
        t.mul_(std)
    if mean != 0.0:
        t.add_(mean)
    return t.to(dtype)


def tokens(n, seed=1, device="cpu", hidden=HIDDEN):
    return normal((n, hidden), 1.0, seed, device)


def block(seed=0, device="cpu", hidden=HIDDEN, inter=INTER, experts=EXPERTS, int8=False):
    """Weights of one MoE block. Seeds: seed+0 norm, +1 router, +2 gate/up, +3 down."""
    b = {
        "norm_w": normal((hidden,), 0.02, seed, device, mean=1.0),
        "w32": normal((experts, hidden), 0.02, seed + 1, device, dtype=torch.float32),
        "w_gu": normal((experts + 1, 2 * inter, hidden), 0.02, seed + 2, device),
        "w_d": normal((experts + 1, hidden, inter), 0.02, seed + 3, device),
    }
    if int8:
        quantize_block(b)
    return b


def quantize_block(b, scale_dtype=torch.bfloat16):
    """Replaces the bf16 experts by int8 + row scales (absmax / 127, bf16 by default) from the same masters."""
    from fused_moe import quantize_rows_int8
    b["q_gu"], b["s_gu"] = quantize_rows_int8(b["w_gu"], scale_dtype=scale_dtype)
    b["q_d"], b["s_d"] = quantize_rows_int8(b["w_d"], scale_dtype=scale_dtype)
    return b


def ragged_bias(seed=7, device="cpu", experts=EXPERTS):
    return normal((experts,), 0.5, seed, device, dtype=torch.float32)


def zipf_bias(seed=11, device="cpu", experts=EXPERTS, s=1.2):
    """bias_e = log p_e with p_e proportional to rank^-s, ranks assigned by a seeded permutation."""
    perm = torch.randperm(experts, generator=_gen(seed, "cpu"))
    ranks = torch.empty(experts, dtype=torch.float32)
    ranks[perm] = torch.arange(1, experts + 1, dtype=torch.float32)
    p = ranks.pow(-s)
    p = p / p.sum()
    return p.log().to(device)


def moe_block_forward(x, b, bias=None, *, int8=False, top_k=TOP_K):
    """One MoE block: xn = RMSNorm(x); softmax top-k router (+ shared expert); y = MoE(xn) + x."""
    from fused_moe import fused_moe_prefill
    from fused_ops import rms_norm, route
    xn = rms_norm(x, b["norm_w"], EPS)
    ids, wts, _ = route(xn, b["w32"], bias, top_k=top_k, scoring="softmax")
    if int8:
        return fused_moe_prefill(xn, b["q_gu"], b["q_d"], ids, wts, s_gu=b["s_gu"], s_d=b["s_d"], residual=x)
    return fused_moe_prefill(xn, b["w_gu"], b["w_d"], ids, wts, residual=x)


def expert_bytes(hidden=HIDDEN, inter=INTER, int8=False, scale_bytes=2):
    """HBM bytes of one expert's weights (+ int8 row scales)."""
    if int8:
        return 3 * hidden * inter + (2 * inter + hidden) * scale_bytes
    return 3 * hidden * inter * 2


def flops_per_pair(hidden=HIDDEN, inter=INTER):
    return 2 * 3 * hidden * inter


def nb_blocks(P, E1, BM=64):
    return math.ceil((P + E1 * (BM - 1)) / BM)
