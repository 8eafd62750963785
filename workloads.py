"""Seeded synthetic inputs of the thinker MoE block and the composed block forward: the harness of bench.py, the GPU
tests and the smoke run, outside the product package (ming-voice_amd/ never imports it).

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
  expert_tensors, write_checkpoint   a layer's experts in the checkpoint key layout, as safetensors shards
  thinker_layer(...)    one synthetic thinker layer (q|k|v and o projections + MoE block)
  ThinkerDecodeStep     the synthetic 28-layer thinker decode step + LM head (one token)
  HybridThinkerStep     the same with the thinker's KDA / MLA attention mixers between the projections
  TalkerLLM(...)        a synthetic Qwen2 Talker LLM with StaticQwen2's attributes and KV cache layout
  TalkerTail(...)       a synthetic Talker (DiT + aggregator + stop head) with the attributes FastTail reads
"""
import math
from types import SimpleNamespace

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


# ------------------------------------------------------------------------------ synthetic checkpoints

def expert_tensors(prefix, n_experts, hidden, inter, seed, dtype=torch.bfloat16):
    """One MoE layer's experts in the thinker's checkpoint key layout: `{prefix}.experts.{e}.{gate,up,down}_proj
    .weight` for e < n_experts and `{prefix}.shared_experts.*`, ~ N(0, 0.05^2), drawn on the CPU from `seed`."""
    g = torch.Generator().manual_seed(seed)
    out = {}
    for e in list(range(n_experts)) + ["shared"]:
        p = f"{prefix}.shared_experts." if e == "shared" else f"{prefix}.experts.{e}."
        out[p + "gate_proj.weight"] = (torch.randn(inter, hidden, generator=g) * 0.05).to(dtype)
        out[p + "up_proj.weight"] = (torch.randn(inter, hidden, generator=g) * 0.05).to(dtype)
        out[p + "down_proj.weight"] = (torch.randn(hidden, inter, generator=g) * 0.05).to(dtype)
    return out


def write_checkpoint(root, tensors, shards=2, extra=True):
    """Writes `tensors` as a sharded safetensors checkpoint under `root` (round robin over `shards` files, with
    two unrelated tensors per shard when `extra`) and its model.safetensors.index.json. Returns `root`."""
    import json
    import os

    from safetensors.torch import save_file
    os.makedirs(root, exist_ok=True)
    keys = sorted(tensors)
    files = [{} for _ in range(shards)]
    for i, k in enumerate(keys):
        files[i % shards][k] = tensors[k].contiguous()
    if extra:
        for s in range(shards):
            files[s][f"model.layers.{s}.input_layernorm.weight"] = torch.ones(64, dtype=torch.bfloat16)
            files[s][f"model.layers.{s}.self_attn.q_proj.weight"] = torch.zeros(8, 64, dtype=torch.float32)
    weight_map = {}
    for s, f in enumerate(files):
        name = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        save_file(f, os.path.join(root, name), metadata={"format": "pt"})
        weight_map.update({k: name for k in f})
    with open(os.path.join(root, "model.safetensors.index.json"), "w") as fh:
        json.dump({"metadata": {}, "weight_map": weight_map}, fh)
    return root


# ------------------------------------------------------------------------------ thinker decode step

ATTN_Q, ATTN_KV = 2048, 256  # q and o are 2048 x 2048; k and v 256 x 2048


def thinker_layer(li, device="cpu", seed=1000, proj=True, int8=False, scale_dtype=torch.bfloat16):
    """Weights of thinker layer li: RMSNorm ln1 (seed s = seed + 16 li), the q | k | v rows stacked into one
    [2048 + 256 + 256, 2048] matrix (seeds s+1..s+3, one GEMV), o (s+4) and one MoE block (seeds s+5..s+8).
    proj False leaves the projections out; int8 replaces the block's experts by int8 + row scales."""
    s = seed + 16 * li
    p = {"blk": block(seed=s + 5, device=device)}
    if int8:
        quantize_block(p["blk"], scale_dtype)
        del p["blk"]["w_gu"], p["blk"]["w_d"]
    if proj:
        q = normal((ATTN_Q, HIDDEN), 0.02, s + 1, device)
        k = normal((ATTN_KV, HIDDEN), 0.02, s + 2, device)
        v = normal((ATTN_KV, HIDDEN), 0.02, s + 3, device)
        p["ln1"] = normal((HIDDEN,), 0.02, s, device, mean=1.0)
        p["qkv"] = torch.cat([q, k, v])
        p["o"] = normal((HIDDEN, ATTN_Q), 0.02, s + 4, device)
    return p


class ThinkerDecodeStep:
    """The synthetic thinker decode step of one token on the HIP kernels:
    `layers` x (RMSNorm fused into the q | k | v GEMV -> o projection + residual -> MoE block with its RMSNorm,
    softmax top-6 + shared expert, + residual) -> final RMSNorm fused into the LM head [vocab, 2048].
    The attention itself (the KDA / MLA mixers of the real thinker) is not part of this step: the o projection
    reads the q rows of the projection output. Weights ~ N(0, 0.02) bf16 (norm weights 1 + N(0, 0.02)), seeds
    as thinker_layer; final norm seed 999, head 998, input token x0 ~ N(0, 1) seed 997. The router outputs
    and the gated activations share one set of buffers across layers. Calling the object runs the step and
    returns the logits [1, vocab]; x0 may be overwritten in place between calls (a captured graph reads it)."""

    def __init__(self, layers=28, device="cuda", vocab=VOCAB, seed=1000):
        self.L = [thinker_layer(li, device, seed) for li in range(layers)]
        self.final_norm = normal((HIDDEN,), 0.02, 999, device, mean=1.0)
        self.head = normal((vocab, HIDDEN), 0.02, 998, device)
        self.x0 = tokens(1, seed=997, device=device)
        self.logits = torch.empty(1, EXPERTS, device=device)
        self.ids = torch.empty(1, TOP_K + 1, device=device, dtype=torch.long)
        self.wts = torch.empty(1, TOP_K + 1, device=device)
        self.a_buf = torch.empty(TOP_K + 1, INTER, device=device, dtype=torch.bfloat16)

    def layer_moe(self, b, h):
        """The MoE block of a layer on h (its norm, router, experts and the residual add), router buffers shared."""
        from fused_moe import moe_block_decode
        return moe_block_decode(h, b["norm_w"], EPS, b["w32"], b["w_gu"], b["w_d"], top_k=TOP_K, logits=self.logits,
                                ids=self.ids, wts=self.wts, a_buf=self.a_buf)[0]

    def layer(self, p, h):
        from fastlinear import small_linear
        qkv = small_linear(h, p["qkv"], norm=(p["ln1"], EPS))
        h = small_linear(qkv[:, :HIDDEN], p["o"], residual=h)
        return self.layer_moe(p["blk"], h)

    def __call__(self):
        from fastlinear import small_linear
        h = self.x0
        for p in self.L:
            h = self.layer(p, h)
        return small_linear(h, self.head, norm=(self.final_norm, EPS))

    def trace(self):
        """The same step run eagerly, keeping each layer's input and router picks:
        ([(h_in, ids, wts)] per layer, the last layer's output, logits)."""
        from fastlinear import small_linear
        h, out = self.x0, []
        for p in self.L:
            h_in = h.clone()
            h = self.layer(p, h)
            out.append((h_in, self.ids.clone(), self.wts.clone()))
        return out, h, small_linear(h, self.head, norm=(self.final_norm, EPS))

    def moe_only(self):
        """The MoE blocks alone, chained, every layer's experts distinct memory."""
        from fused_moe import moe_block_decode
        h = self.x0
        for p in self.L:
            b = p["blk"]
            h = moe_block_decode(h, b["norm_w"], EPS, b["w32"], b["w_gu"], b["w_d"], top_k=TOP_K, logits=self.logits,
                                 ids=self.ids, wts=self.wts, a_buf=self.a_buf)[0]
        return h

    def bytes_per_step(self):
        """HBM bytes one step must read: projections, 7 experts and the router of every layer, the LM head."""
        n = len(self.L)
        proj = n * ((ATTN_Q + 2 * ATTN_KV) * HIDDEN + HIDDEN * ATTN_Q) * 2
        moe = n * (TOP_K + 1) * expert_bytes()
        router = n * EXPERTS * HIDDEN * 4
        return proj + moe + router + self.head.numel() * 2


# ----------------------------------------------------------------------- hybrid thinker decode step

KDA_HEADS, KDA_DIM, KDA_CONV, KDA_LORA = 16, 128, 4, 128
MLA_HEADS, MLA_QK, MLA_V = 16, 192, 128


def _ns(**kw):
    from types import SimpleNamespace
    return SimpleNamespace(**kw)


def _linear_ns(w):
    return _ns(weight=w, bias=None)


class HybridThinkerStep:
    """One decode token of a synthetic hybrid thinker (the layer kinds engine.py:636-648 caches): `layers` layers,
    every `mla_every`-th an MLA layer and the others KDA layers, each followed by the MoE block of ThinkerDecodeStep
    (softmax top-6 + shared expert); final RMSNorm and LM head; greedy: the word embedding [vocab, 2048] (~ N(0, 1))
    of the token in `tok` is the input row and the argmax of the logits is written back there, the position advances
    on the device (engine.py:685-689).
    The weights and caches are held as engine.Thinker holds them (model.model.word_embeddings, .layers[i] with
    .attention / .attention_layer_type / .input_layernorm / .post_attention_layernorm / .mlp, .norm, model.lm_head,
    _KDAState- and _MLAState-like cache layers, tok_buf, pos_buf), and the step is the product's
    thinker_step.FastThinkerStep built from them.
      KDA layer: q | k | v (16 x 128 each), f_a | g_a (rank 128), b (16) projections, the q / k / v short convolutions
        (window 4, caches [1, 2048, 4] each), fused_recurrent_kda's state [1, 16, 128, 128] fp32, o_norm, o_proj.
      MLA layer: q | k (16 x 192), v (16 x 128) projections, no rotary or latent compression (the remote model code
        that holds them is not in the reference tree), caches k [1, 16, max_len, 192], v [1, 16, max_len, 128].
    Shapes beyond the configs' hidden 2048 (head counts, dims, the 3:1 mix) are an assumption. Weights ~ N(0, 0.02)
    (norm weights 1 + N(0, 0.02), A_log, dt_bias ~ N(0, 0.5), conv ~ N(0, 0.5)); the caches hold a context of `pos`
    tokens (random rows, states ~ N(0, 0.1)). self.L keeps each layer's tensors by name (views of the same memory)
    for the checks. Calling the object runs one step and returns the logits [1, vocab]."""

    def __init__(self, layers=28, device="cuda", vocab=VOCAB, max_len=1024, pos=512, mla_every=4, seed=5000,
                 fused_kda=True):
        import thinker_step
        H, dev = HIDDEN, device
        kd = KDA_HEADS * KDA_DIM
        self.max_len = max_len
        self.L, mods, caches = [], [], []
        for li in range(layers):
            s = seed + 64 * li
            w = lambda shape, j, std=0.02, **kw: normal(shape, std, s + j, dev, **kw)  # noqa: E731
            p = {"blk": block(seed=s + 1, device=dev), "ln1": w((H,), 6, mean=1.0)}
            if (li + 1) % mla_every == 0:
                p["kind"] = "mla"
                p["qkv"] = torch.cat([w((MLA_HEADS * MLA_QK, H), 10), w((MLA_HEADS * MLA_QK, H), 11),
                                      w((MLA_HEADS * MLA_V, H), 12)])
                p["o"] = w((H, MLA_HEADS * MLA_V), 13)
                p["kc"] = normal((1, MLA_HEADS, max_len, MLA_QK), 1.0, s + 14, dev)
                p["vc"] = normal((1, MLA_HEADS, max_len, MLA_V), 1.0, s + 15, dev)
                nq = MLA_HEADS * MLA_QK
                q, k, v = p["qkv"][:nq], p["qkv"][nq:2 * nq], p["qkv"][2 * nq:]
                attn = _ns(q_proj=_linear_ns(q), k_proj=_linear_ns(k), v_proj=_linear_ns(v),
                           o_proj=_linear_ns(p["o"]), num_heads=MLA_HEADS, qk_head_dim=MLA_QK, v_head_dim=MLA_V)
                caches.append(_ns(k=p["kc"], v=p["vc"]))
            else:
                p["kind"] = "kda"
                p["proj"] = torch.cat([w((3 * kd, H), 20), w((KDA_LORA, H), 21), w((KDA_LORA, H), 22),
                                       w((KDA_HEADS, H), 23)])
                p["f_b"] = w((kd, KDA_LORA), 24)
                p["g_b"] = w((kd, KDA_LORA), 25)
                p["conv_w"] = w((3 * kd, 1, KDA_CONV), 26, std=0.5)
                p["conv"] = tuple(c.clone() for c in w((1, 3 * kd, KDA_CONV), 27, std=1.0).split(kd, dim=1))
                p["A_log"] = w((KDA_HEADS,), 28, std=0.5, dtype=torch.float32)
                p["dt_bias"] = w((kd,), 29, std=0.5, dtype=torch.float32)
                p["o_norm"] = w((KDA_DIM,), 30, mean=1.0)
                p["o"] = w((H, kd), 31)
                p["state"] = w((1, KDA_HEADS, KDA_DIM, KDA_DIM), 32, std=0.1, dtype=torch.float32)
                pr = p["proj"].split([kd, kd, kd, KDA_LORA, KDA_LORA, KDA_HEADS])
                cw = p["conv_w"].split(kd)
                conv = lambda wt: _ns(weight=wt, bias=None, hidden_size=kd, kernel_size=(KDA_CONV,))  # noqa: E731
                attn = _ns(mode="fused_recurrent", q_proj=_linear_ns(pr[0]), k_proj=_linear_ns(pr[1]),
                           v_proj=_linear_ns(pr[2]), f_a_proj=_linear_ns(pr[3]), g_a_proj=_linear_ns(pr[4]),
                           b_proj=_linear_ns(pr[5]), f_b_proj=_linear_ns(p["f_b"]), g_b_proj=_linear_ns(p["g_b"]),
                           q_conv1d=conv(cw[0]), k_conv1d=conv(cw[1]), v_conv1d=conv(cw[2]),
                           o_norm=_ns(weight=p["o_norm"], eps=1e-5), o_proj=_linear_ns(p["o"]), A_log=p["A_log"],
                           dt_bias=p["dt_bias"], lower_bound=None, num_heads=KDA_HEADS, head_k_dim=KDA_DIM,
                           head_dim=KDA_DIM, no_kda_lora=False)
                caches.append(_ns(keys=p["state"], values=p["conv"]))
            b = p["blk"]
            gate = _ns(weight=None, w32=b["w32"], expert_bias=None, top_k=TOP_K, n_group=1, topk_group=1,
                       routed_scaling_factor=1.0)
            mods.append(_ns(attention=attn, attention_layer_type="attention" if p["kind"] == "mla" else "kda",
                            input_layernorm=_ns(weight=p["ln1"], variance_epsilon=EPS),
                            post_attention_layernorm=_ns(weight=b["norm_w"], variance_epsilon=EPS),
                            mlp=_ns(gate=gate, w_gu=b["w_gu"], w_d=b["w_d"])))
            self.L.append(p)
        self.embed = normal((vocab, H), 1.0, seed + 1, dev)
        self.final_norm = normal((HIDDEN,), 0.02, 999, device, mean=1.0)
        self.head = normal((vocab, HIDDEN), 0.02, 998, device)
        self.model = _ns(model=_ns(word_embeddings=_ns(weight=self.embed), layers=mods,
                                   norm=_ns(weight=self.final_norm, variance_epsilon=EPS)),
                         lm_head=_linear_ns(self.head))
        self.cache_layers = caches
        self.tok = torch.tensor([[(seed * 7919) % vocab]], device=dev, dtype=torch.long)
        self.pos = torch.tensor([pos], device=dev, dtype=torch.long)
        self.fast = thinker_step.FastThinkerStep(self.model, caches, self.tok, self.pos, scoring="softmax",
                                                 fused_kda=fused_kda)

    def use_int8_experts(self, scale_dtype=torch.float32):
        """Every layer's experts as int8 + row scales from the same bf16 masters, the way engine._quantize_moe_int8
        leaves a block (mlp.q_gu / q_d / s_gu / s_d, no bf16 stacks); the step is rebuilt on them."""
        import thinker_step
        for p, layer in zip(self.L, self.model.model.layers):
            b = quantize_block(p["blk"], scale_dtype)
            b.pop("w_gu"), b.pop("w_d")
            mlp = layer.mlp
            mlp.w_gu = mlp.w_d = None
            mlp.q_gu, mlp.q_d, mlp.s_gu, mlp.s_d = b["q_gu"], b["q_d"], b["s_gu"], b["s_d"]
        self.int8_scale_bytes = torch.finfo(scale_dtype).bits // 8
        self.fast = thinker_step.FastThinkerStep(self.model, self.cache_layers, self.tok, self.pos, scoring="softmax",
                                                 fused_kda=self.fast.fused_kda)

    @property
    def fused_kda(self):
        """The KDA cores as kda_decode_step's one kernel (True) or the chain of calls it replaces."""
        return self.fast.fused_kda

    @fused_kda.setter
    def fused_kda(self, v):
        self.fast.fused_kda = v

    def __call__(self):
        return self.fast()

    def trace(self):
        """thinker_step.FastThinkerStep.trace: per layer (input, mixer output, router ids, weights), the last
        output, the logits."""
        return self.fast.trace()

    def bytes_per_step(self, pos=None):
        """HBM bytes one step must read or write at position pos (default: the current one): every weight of the
        mixers, the KDA states (read + written) and conv caches, the MLA cache rows 0..pos, the 7 experts and
        router of every MoE block, the embedding row, the LM head and its logits (written, then read by the
        argmax)."""
        pos = int(self.pos) if pos is None else pos
        H, total = HIDDEN, 0
        for p in self.L:
            if p["kind"] == "mla":
                total += (p["qkv"].numel() + p["o"].numel()) * 2
                total += (pos + 1) * MLA_HEADS * (MLA_QK + MLA_V) * 2
            else:
                total += (p["proj"].numel() + p["f_b"].numel() + p["g_b"].numel() + p["o"].numel()) * 2
                total += p["conv_w"].numel() * 2 + 2 * sum(c.numel() for c in p["conv"]) * 2 + 2 * p["state"].numel() * 4
            sb = getattr(self, "int8_scale_bytes", None)
            total += H * 2 + (TOP_K + 1) * expert_bytes(int8=sb is not None, scale_bytes=sb or 2) + EXPERTS * H * 4
        vocab = self.head.shape[0]
        return total + H * 2 + self.head.numel() * 2 + 2 * vocab * 2

    def state_copy(self):
        """A copy of the step's mutable state: KDA states and conv caches, MLA caches, the position, the token."""
        keys = ("state", "conv", "kc", "vc")
        clone = lambda t: tuple(c.clone() for c in t) if isinstance(t, tuple) else t.clone()  # noqa: E731
        return {"pos": self.pos.clone(), "tok": self.tok.clone(),
                "L": [{k: clone(p[k]) for k in keys if k in p} for p in self.L]}


# ------------------------------------------------------------------------------------------- Talker LLM

TALKER_HIDDEN, TALKER_HEADS, TALKER_KV_HEADS, TALKER_INTER, TALKER_LAYERS = 896, 14, 2, 4864, 24


class _RMSNorm(torch.nn.Module):
    """Holds what FastQwen2Step reads of a Qwen2RMSNorm: `weight` and `variance_epsilon`."""

    def __init__(self, w, eps):
        super().__init__()
        self.weight = torch.nn.Parameter(w, requires_grad=False)
        self.variance_epsilon = eps


def _linear(w, b=None):
    lin = torch.nn.Linear(w.shape[1], w.shape[0], bias=b is not None, device=w.device, dtype=w.dtype)
    lin.requires_grad_(False)
    lin.weight.copy_(w)
    if b is not None:
        lin.bias.copy_(b)
    return lin


class TalkerLLM:
    """A Qwen2 decoder with random weights, exposing the attributes of engine.py's StaticQwen2
    (engine.py:1250-1266): `m.layers[i].{self_attn.{q,k,v,o}_proj, mlp.{gate,up,down}_proj,
    input_layernorm, post_attention_layernorm}`, `m.norm`, nh / nkv / hd, the static KV cache
    k, v [layers, 1, nkv, max_len, hd] (bf16, zeros) and inv_freq [hd/2] fp32 (rope theta 1e6).
    Defaults are Qwen2-0.5B-shaped (hidden 896, 14 query / 2 KV heads of 64, intermediate 4864, 24 layers).
    Weights ~ N(0, 0.02) bf16 (q/k/v biases too), norm weights ~ 1 + N(0, 0.02); seeds seed + 16 i + j."""

    def __init__(self, layers=TALKER_LAYERS, max_len=1024, seed=0, device="cpu", hidden=TALKER_HIDDEN,
                 heads=TALKER_HEADS, kv_heads=TALKER_KV_HEADS, inter=TALKER_INTER, theta=1e6, eps=1e-6):
        hd = hidden // heads
        self.nh, self.nkv, self.hd, self.max_len = heads, kv_heads, hd, max_len
        L = []
        for i in range(layers):
            s = seed + 16 * i
            w = lambda shape, j, **kw: normal(shape, 0.02, s + j, device, **kw)  # noqa: E731
            attn = SimpleNamespace(q_proj=_linear(w((heads * hd, hidden), 0), w((heads * hd,), 1)),
                                   k_proj=_linear(w((kv_heads * hd, hidden), 2), w((kv_heads * hd,), 3)),
                                   v_proj=_linear(w((kv_heads * hd, hidden), 4), w((kv_heads * hd,), 5)),
                                   o_proj=_linear(w((hidden, heads * hd), 6)))
            mlp = SimpleNamespace(gate_proj=_linear(w((inter, hidden), 7)), up_proj=_linear(w((inter, hidden), 8)),
                                  down_proj=_linear(w((hidden, inter), 9)))
            L.append(SimpleNamespace(self_attn=attn, mlp=mlp,
                                     input_layernorm=_RMSNorm(w((hidden,), 10, mean=1.0), eps),
                                     post_attention_layernorm=_RMSNorm(w((hidden,), 11, mean=1.0), eps)))
        self.m = SimpleNamespace(layers=L, norm=_RMSNorm(normal((hidden,), 0.02, seed + 16 * layers, device,
                                                                mean=1.0), eps))
        self.k = torch.zeros(layers, 1, kv_heads, max_len, hd, dtype=torch.bfloat16, device=device)
        self.v = torch.zeros_like(self.k)
        self.inv_freq = 1.0 / (theta ** (torch.arange(0, hd, 2, device=device, dtype=torch.float32) / hd))

    def fill_cache(self, n, seed=1):
        """Rows [0, n) of every layer's cache ~ N(0, 1): a stand-in for an already-prefilled context."""
        self.k[:, :, :, :n] = normal(self.k[:, :, :, :n].shape, 1.0, seed, self.k.device)
        self.v[:, :, :, :n] = normal(self.v[:, :, :, :n].shape, 1.0, seed + 1, self.v.device)


class _Rotary:
    """forward_from_seq_len(n) -> (freqs [1, n, hd], 1.0) with each pair's angle t * inv_freq[p] twice,
    interleaved, as x_transformers' RotaryEmbedding returns them."""

    def __init__(self, hd, device, theta=10000.0):
        self.inv_freq = 1.0 / (theta ** (torch.arange(0, hd, 2, device=device, dtype=torch.float32) / hd))

    def forward_from_seq_len(self, n):
        f = torch.arange(n, device=self.inv_freq.device, dtype=torch.float32)[:, None] * self.inv_freq[None]
        return torch.stack([f, f], -1).reshape(1, n, -1), 1.0


class _TimestepEmbedder:
    """t [1] -> [1, D] bf16: sinusoidal features of t through a fixed random linear map."""

    def __init__(self, D, seed, device, nf=32):
        self.freqs = torch.exp(-math.log(1000.0) * torch.arange(nf // 2, device=device, dtype=torch.float32) / (nf // 2))
        self.proj = normal((nf, D), 0.5, seed, device, dtype=torch.float32)

    def __call__(self, t):
        a = t.float().reshape(-1, 1) * 1000.0 * self.freqs[None]
        return (torch.cat([a.sin(), a.cos()], -1) @ self.proj).to(torch.bfloat16)


def _dit_block(D, heads, F, seed, device):
    w = lambda shape, j, **kw: normal(shape, 0.02, seed + j, device, **kw)  # noqa: E731
    attn = SimpleNamespace(heads=heads, to_q=_linear(w((D, D), 0), w((D,), 1)), to_k=_linear(w((D, D), 2), w((D,), 3)),
                           to_v=_linear(w((D, D), 4), w((D,), 5)), to_out=[_linear(w((D, D), 6), w((D,), 7))],
                           q_norm=None, pe_attn_head=None)
    ff = [[_linear(w((F, D), 8), w((F,), 9)), SimpleNamespace(approximate="tanh")], None,
          _linear(w((D, F), 10), w((D,), 11))]
    return SimpleNamespace(attn=attn, mlp=SimpleNamespace(ff=ff),
                           norm1=SimpleNamespace(weight=w((D,), 12, mean=1.0), eps=1e-6),
                           norm2=SimpleNamespace(weight=w((D,), 13, mean=1.0), eps=1e-6))


class TalkerTail:
    """A Talker with random weights exposing what FastTail reads (fast_talker.py:114-137): t.cfm.model (the
    DiT: t_embedder, c_embedder.cond_embedder, x_embedder, blocks, rotary_embed, final_layer), t.aggregator
    (word_embedder, x_embedder, blocks, rotary_embed, final_layer) and t.stop_head; ts (steps + 1 bf16
    timesteps in [0, 1]), dts and cfg_strength 2.0. Default shapes (an assumption: the reference loads its
    Talker config from the model directory): DiT hidden 1024, 16 heads, MLP 4096, 4 blocks; aggregator 2
    blocks; latent 64; LLM hidden 896; 10 steps."""

    def __init__(self, seed=0, device="cpu", llm_hidden=TALKER_HIDDEN, dim=1024, heads=16, mlp=4096, depth=4,
                 agg_depth=2, latent=64, steps=10):
        w = lambda shape, j, **kw: normal(shape, 0.02, seed + j, device, **kw)  # noqa: E731
        hd = dim // heads
        final = lambda j, out: SimpleNamespace(norm_final=SimpleNamespace(weight=w((dim,), j, mean=1.0), eps=1e-6),  # noqa: E731
                                               linear=_linear(w((out, dim), j + 1), w((out,), j + 2)))
        dit = SimpleNamespace(
            spk_embedder=None, t_embedder=_TimestepEmbedder(dim, seed + 1, device),
            c_embedder=SimpleNamespace(cond_embedder=_linear(w((dim, llm_hidden), 2), w((dim,), 3))),
            x_embedder=_linear(w((dim, latent), 4), w((dim,), 5)),
            blocks=[_dit_block(dim, heads, mlp, seed + 100 + 20 * i, device) for i in range(depth)],
            rotary_embed=_Rotary(hd, device), final_layer=final(10, latent))
        emb = torch.nn.Embedding(1, dim, device=device, dtype=torch.bfloat16)
        emb.requires_grad_(False)
        emb.weight.copy_(normal((1, dim), 1.0, seed + 20, device))
        agg = SimpleNamespace(
            word_embedder=emb, x_embedder=_linear(w((dim, latent), 21), w((dim,), 22)),
            blocks=[_dit_block(dim, heads, mlp, seed + 500 + 20 * i, device) for i in range(agg_depth)],
            rotary_embed=_Rotary(hd, device), final_layer=final(30, llm_hidden))
        self.t = SimpleNamespace(cfm=SimpleNamespace(model=dit), aggregator=agg,
                                 stop_head=_linear(normal((2, llm_hidden), 0.05, seed + 40, device), w((2,), 41)))
        self.ts = torch.linspace(0, 1, steps + 1, device=device).to(torch.bfloat16)
        self.dts = [self.ts[s + 1] - self.ts[s] for s in range(steps)]
        self.cfg_strength = 2.0
