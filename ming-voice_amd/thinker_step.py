"""The hybrid thinker's greedy decode step (engine.py:665-689) and its prefill (engine.py:938-972, with the padded
prefill graphs of engine.py:716-757) on this build's kernels, built from the engine's objects.

FastThinkerStep(model, cache_layers, tok_buf, pos_buf) takes what engine.Thinker holds once it is loaded and patched
(engine.py:570-660): `model` is Thinker.model, `cache_layers` Thinker._layers, `tok_buf` / `pos_buf` its [1, 1] token
and [1] position buffers. It reads, by the attribute paths the engine and its dev scripts use:

  model.model.word_embeddings.weight     the input row of a step (engine.py:686)
  model.model.layers[i]                  .attention, .attention_layer_type ("attention" = an MLA layer,
                                         engine.py:640), .input_layernorm, .post_attention_layernorm, .mlp
                                         (engine.py:1277, 1291; dev/profile_decode_layers.py:12-13)
  model.model.norm, model.lm_head        the final norm and the head (engine.py:678-679)
  RMSNorm modules                        .weight, .variance_epsilon (engine.py:229)
  KDA attention (engine.py:234-267)      q_proj, k_proj, v_proj, f_a_proj, g_a_proj, b_proj (fused here into one GEMV
                                         with the input norm), q_conv1d / k_conv1d / v_conv1d, f_b_proj, g_b_proj,
                                         A_log, dt_bias, lower_bound, o_norm (.weight, .eps), o_proj, num_heads,
                                         head_k_dim, head_dim; the LoRA gate form (no_kda_lora false)
  MoE block, as _patch_moe leaves it     w_gu / w_d (or q_gu, q_d, s_gu, s_d for int8 experts) with the shared expert
  (engine.py:313-391)                    in the last slot; gate.w32, gate.expert_bias, gate.top_k, gate.n_group,
                                         gate.topk_group, gate.routed_scaling_factor (engine.py:284-297, 326-333)
  cache_layers[i]                        engine._KDAState (.keys: the fp32 state [1, H, K, V]; .values: the q, k, v
                                         conv caches [1, C, W]) or engine._MLAState (.k [1, nh, max_ctx, dqk],
                                         .v [1, nh, max_ctx, dv]) (engine.py:495-526, 636-648)

A step: h = word_embeddings(tok_buf); per layer h += mixer(input_layernorm(h)), then the MoE block with
post_attention_layernorm and the residual (moe_block_decode: router, experts, combine); logits = lm_head(norm(h));
tok_buf = argmax(logits); pos_buf += 1. KDA layers run the norm-fused projection GEMV, kda_decode_step (convolutions,
gate LoRA up-projections, recurrence, gated norm) and the o projection with the residual: 3 launches. MLA layers run
mla_qkv, mla_decode_attn (cache rows written at pos, attention over 0..pos) and the o projection.

The MLA layers' projections are the model's remote code, which is not in the reference tree: pass
mla_qkv(li, attention, h) -> (q [nh, dqk], k [nh, dqk], v [nh, dv]) computing a layer's new query, key and value rows
from its input row h [1, H] (norm included). Without it, a layer whose attention has q_proj, k_proj and v_proj runs
them fused with the input norm, with no rotary part (the synthetic thinker of this build's benchmark).

Every call enqueues on torch's current stream and can be captured in one hipGraph (engine.py:694-713); the state
lives in the engine's own buffers, so replays advance it as the engine's decode graphs do.

A prefill (FastThinkerStep.prefill) runs the same layers over a prompt's T rows: the projections as GEMMs, the KDA
recurrence over the T tokens from the layer's state, the MLA layers' causal attention over the cache (rows stored at
pos .. pos + T - 1), the prefill MoE block, then the head on the last real row; with n_valid on the device, one
capture per bucket length serves shorter prompts padded to it.
"""
import torch
import torch.nn.functional as F

import fastlinear
import fused_moe
import fused_ops
import thinker_attn as TA

__all__ = ["FastThinkerStep"]

_SCORING = ("sigmoid", "softmax")
# Prompts longer than this take the KDA recurrence in chunked form (chunk_kda), as the engine switches its KDA layers'
# mode (engine.py:946-949, 964-967). Measured per call over 16 heads of 128 x 128 (graph replays): 200 / 256 / 384 /
# 512 tokens 42.1 / 48.2 / 71.2 / 87.1 us chunked against 43.2 / 51.7 / 72.7 / 93.4 us recurrent.
KDA_CHUNK_ABOVE = 192


def _norm(mod, what):
    w = getattr(mod, "weight", None)
    eps = getattr(mod, "variance_epsilon", getattr(mod, "eps", None))
    if w is None or eps is None:
        raise ValueError(f"FastThinkerStep: {what} needs .weight and .variance_epsilon (or .eps)")
    return w, float(eps)


def _fuse(mods, what):
    """One GEMV matrix (and bias, or None) from linear modules applied to the same input, rows stacked in order."""
    ws = [m.weight for m in mods]
    bs = [getattr(m, "bias", None) for m in mods]
    if any(w.dim() != 2 or w.shape[1] != ws[0].shape[1] or w.dtype != torch.bfloat16 for w in ws):
        raise ValueError(f"FastThinkerStep: {what} projections must be bf16 [out, hidden] matrices")
    w = torch.cat(ws).contiguous()
    if all(b is None for b in bs):
        return w, None
    b = torch.cat([bb if bb is not None else torch.zeros(ww.shape[0], device=w.device, dtype=w.dtype)
                   for ww, bb in zip(ws, bs)]).to(torch.bfloat16).contiguous()
    return w, b


def _bias(mod):
    b = getattr(mod, "bias", None)
    return None if b is None else b.to(torch.bfloat16).contiguous()


class FastThinkerStep:
    """See the module docstring. scoring: the MoE router's form, "sigmoid" (the thinker's gate: sigmoid + expert
    bias, group-limited top-k, engine.py:326-333) or "softmax" (softmax top-k, renormalised). n_layers: the first
    n layers (Thinker.n_layers). fused_kda False runs each KDA core as its five calls (short_conv, the f and g
    projections, fused_recurrent_kda, rms_norm_gated) instead of kda_decode_step's one kernel. Calling the object
    runs one step and returns the logits [1, vocab]."""

    def __init__(self, model, cache_layers, tok_buf, pos_buf, *, n_layers=None, scoring="sigmoid", mla_qkv=None,
                 fused_kda=True):
        if scoring not in _SCORING:
            raise ValueError(f"FastThinkerStep: scoring must be one of {_SCORING}")
        m = model.model
        layers = list(m.layers)[: n_layers if n_layers is not None else len(m.layers)]
        if len(cache_layers) < len(layers):
            raise ValueError(f"FastThinkerStep: {len(layers)} layers but {len(cache_layers)} cache layers")
        if tok_buf.dtype != torch.int64 or tok_buf.numel() != 1 or pos_buf.dtype != torch.int64 or pos_buf.numel() != 1:
            raise ValueError("FastThinkerStep: tok_buf and pos_buf must be one-element int64 device tensors")
        self.embed = m.word_embeddings.weight
        self.final_norm = _norm(m.norm, "model.model.norm")
        self.head = model.lm_head.weight
        self.tok, self.pos = tok_buf, pos_buf
        self.scoring, self.mla_qkv, self.fused_kda = scoring, mla_qkv, fused_kda
        dev = self.embed.device
        self.H = self.embed.shape[1]
        self.h_in = torch.empty(1, 1, self.H, device=dev, dtype=self.embed.dtype)
        # the argmax of the logits split over many workgroups (sized for fp32 logits, which need the most)
        self.amx_ws = TA.argmax_workspace(1, self.head.shape[0], torch.float32, dev)
        self.L = [self._layer(li, layer, cache_layers[li]) for li, layer in enumerate(layers)]
        # router outputs and gated activations, shared by the layers (a layer reads them before the next writes)
        nk = max(p["blk"]["top_k"] for p in self.L) + 1 if self.L else 1
        ne = max(p["blk"]["w32"].shape[0] for p in self.L) if self.L else 1
        inter = max(p["blk"]["inter"] for p in self.L) if self.L else 1
        self.logits = torch.empty(1, ne, device=dev)
        self.ids = torch.empty(1, nk, device=dev, dtype=torch.int64)
        self.wts = torch.empty(1, nk, device=dev)
        self.a_buf = torch.empty(nk, inter, device=dev, dtype=torch.bfloat16)
        mla = [p for p in self.L if p["kind"] == "mla"]
        self.ws = None
        if mla:
            nh = max(p["kc"].shape[1] for p in mla)
            dv = max(p["vc"].shape[-1] for p in mla)
            max_len = max(p["kc"].shape[2] for p in mla)
            self.ws = TA.mla_attn_workspace(nh, dv, max_len, dev)

    # ------------------------------------------------------------------------------------------- set-up

    def _layer(self, li, layer, cache):
        a = layer.attention
        p = {"ln1": _norm(layer.input_layernorm, f"layer {li} input_layernorm"), "blk": self._moe(li, layer)}
        if getattr(layer, "attention_layer_type", None) == "attention":  # engine.py:640
            p["kind"] = "mla"
            p["kc"], p["vc"] = cache.k, cache.v
            p["nh"], p["dqk"], p["dv"] = int(a.num_heads), int(a.qk_head_dim), int(a.v_head_dim)
            if tuple(cache.k.shape[1:2]) != (p["nh"],) or cache.k.shape[-1] != p["dqk"] or cache.v.shape[-1] != p["dv"]:
                raise ValueError(f"FastThinkerStep: layer {li}: the MLA cache does not match num_heads / head dims")
            if self.mla_qkv is None:
                if not all(hasattr(a, n) for n in ("q_proj", "k_proj", "v_proj")):
                    raise ValueError(f"FastThinkerStep: layer {li} is an MLA layer without q_proj / k_proj / v_proj: "
                                     "pass mla_qkv(li, attention, h) -> (q, k, v) for the model's projections")
                p["qkv"], p["qkv_b"] = _fuse([a.q_proj, a.k_proj, a.v_proj], f"layer {li} MLA q | k | v")
            p["o"], p["o_b"] = a.o_proj.weight, _bias(a.o_proj)
            return p
        p["kind"] = "kda"
        if getattr(a, "no_kda_lora", False):
            raise ValueError(f"FastThinkerStep: layer {li}: KDA without the gate LoRA (no_kda_lora) is not supported")
        H, K, V = int(a.num_heads), int(a.head_k_dim), int(a.head_dim)
        p["heads"], p["K"], p["V"] = H, K, V
        p["proj"], p["proj_b"] = _fuse([a.q_proj, a.k_proj, a.v_proj, a.f_a_proj, a.g_a_proj, a.b_proj],
                                       f"layer {li} KDA q | k | v | f_a | g_a | b")
        p["rank"] = a.f_a_proj.weight.shape[0]
        if a.g_a_proj.weight.shape[0] != p["rank"] or a.b_proj.weight.shape[0] != H:
            raise ValueError(f"FastThinkerStep: layer {li}: f_a / g_a ranks differ or b_proj is not [heads, hidden]")
        convs = (a.q_conv1d, a.k_conv1d, a.v_conv1d)
        if any(getattr(c, "bias", None) is not None for c in convs):
            raise ValueError(f"FastThinkerStep: layer {li}: short convolutions with a bias are not supported")
        p["conv_w"] = tuple(c.weight for c in convs)
        p["conv"] = tuple(cache.values)
        p["state"] = cache.keys
        p["f_b"], p["g_b"] = a.f_b_proj.weight, a.g_b_proj.weight
        if _bias(a.f_b_proj) is not None or _bias(a.g_b_proj) is not None:
            raise ValueError(f"FastThinkerStep: layer {li}: f_b_proj / g_b_proj with a bias are not supported")
        p["A_log"], p["dt_bias"] = a.A_log, a.dt_bias
        lb = getattr(a, "lower_bound", None)
        p["lower_bound"] = None if lb is None else float(lb)
        p["o_norm"] = _norm(a.o_norm, f"layer {li} o_norm")
        p["o"], p["o_b"] = a.o_proj.weight, _bias(a.o_proj)
        return p

    def _moe(self, li, layer):
        mlp, g = layer.mlp, layer.mlp.gate
        norm_w, eps = _norm(layer.post_attention_layernorm, f"layer {li} post_attention_layernorm")
        if getattr(mlp, "w_gu", None) is not None:
            exp = {"w_gu": mlp.w_gu, "w_d": mlp.w_d, "s_gu": None, "s_d": None}
        elif getattr(mlp, "q_gu", None) is not None:
            exp = {"w_gu": mlp.q_gu, "w_d": mlp.q_d, "s_gu": mlp.s_gu, "s_d": mlp.s_d}
        else:
            raise ValueError(f"FastThinkerStep: layer {li}: the MoE block has no stacked experts (engine._patch_moe)")
        bias = getattr(g, "expert_bias", None)
        return dict(exp, norm_w=norm_w, eps=eps, w32=g.w32, bias=None if bias is None else bias.float().contiguous(),
                    top_k=int(g.top_k), n_group=int(getattr(g, "n_group", 1) or 1),
                    topk_group=int(getattr(g, "topk_group", 1) or 1),
                    scale=float(getattr(g, "routed_scaling_factor", 1.0) or 1.0), inter=exp["w_d"].shape[-1])

    # ----------------------------------------------------------------------------------------- decode step

    def embed_token(self):
        """word_embeddings(tok_buf) -> the step's input row [1, H] (a view of a buffer the step owns)."""
        return TA.embed_rows(self.embed, self.tok, out=self.h_in)[0]

    def mixer(self, li, h):
        """The attention half of layer li: h -> h + o(mixer(input_layernorm(h)))."""
        p = self.L[li]
        sl = fastlinear.small_linear
        if p["kind"] == "mla":
            if self.mla_qkv is not None:
                q, k, v = self.mla_qkv(li, p, h)
            else:
                qkv = sl(h, p["qkv"], b=p["qkv_b"], norm=p["ln1"])
                nq = p["nh"] * p["dqk"]
                q, k, v = qkv[:, :nq], qkv[:, nq:2 * nq], qkv[:, 2 * nq:]
            o = TA.mla_decode_attn(q, k, v, p["kc"], p["vc"], self.pos, workspace=self.ws)
            return sl(o.reshape(1, -1), p["o"], b=p["o_b"], residual=h)
        H, K, V, R = p["heads"], p["K"], p["V"], p["rank"]
        pr = sl(h, p["proj"], b=p["proj_b"], norm=p["ln1"])
        ow, oe = p["o_norm"]
        if self.fused_kda:
            on = TA.kda_decode_step(pr, p["conv_w"], p["conv"], p["f_b"], p["g_b"], p["A_log"], p["dt_bias"], p["state"],
                                    ow, heads=H, eps=oe, lower_bound=p["lower_bound"])
            return sl(on.reshape(1, H * V), p["o"], b=p["o_b"], residual=h)
        nqk, nv = H * K, H * V
        qkv = [TA.short_conv(pr[:, a:b], c, w) for (a, b), c, w in
               zip(((0, nqk), (nqk, 2 * nqk), (2 * nqk, 2 * nqk + nv)), p["conv"], p["conv_w"])]
        base = 2 * nqk + nv
        f = sl(pr[:, base:base + R], p["f_b"])
        gg = sl(pr[:, base + R:base + 2 * R], p["g_b"])
        beta = pr[:, base + 2 * R:]  # the beta projection: the kernel applies its sigmoid
        o, _ = TA.fused_recurrent_kda(qkv[0].reshape(1, 1, H, K), qkv[1].reshape(1, 1, H, K), qkv[2].reshape(1, 1, H, V),
                                      f.reshape(1, 1, H, K), beta.reshape(1, 1, H), A_log=p["A_log"],
                                      dt_bias=p["dt_bias"], initial_state=p["state"], inplace=True,
                                      use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True, beta_is_logits=True,
                                      lower_bound=p["lower_bound"])
        on = TA.rms_norm_gated(o.reshape(H, V), gg.reshape(H, V), ow, oe)
        return sl(on.reshape(1, H * V), p["o"], b=p["o_b"], residual=h)

    def moe(self, li, h):
        """The MoE half of layer li with its residual (router outputs in the step's shared buffers)."""
        b = self.L[li]["blk"]
        return fused_moe.moe_block_decode(h, b["norm_w"], b["eps"], b["w32"], b["w_gu"], b["w_d"], top_k=b["top_k"],
                                          bias=b["bias"], scoring=self.scoring, n_group=b["n_group"],
                                          topk_group=b["topk_group"], scale=b["scale"], s_gu=b["s_gu"], s_d=b["s_d"],
                                          logits=self.logits[:, :b["w32"].shape[0]], ids=self.ids[:, :b["top_k"] + 1],
                                          wts=self.wts[:, :b["top_k"] + 1], a_buf=self.a_buf)[0]

    def head_logits(self, h):
        return fastlinear.small_linear(h, self.head, norm=self.final_norm)

    # -------------------------------------------------------------------------------------------- prefill

    @staticmethod
    def _rows(x, w, b=None, residual=None, norm=None, in_place=False):
        """A projection of T rows: up to fastlinear.MAX_M rows on the small_linear GEMV (norm and residual fused),
        more as rms_norm (HIP) -> the library GEMM (hipBLASLt through torch; the residual, without a bias, as its C
        operand), the form of the reference's own prefill (nn.Linear after the patched norm, engine.py:220-228).
        in_place: the residual is a buffer nobody reads afterwards, so the GEMM accumulates into it (beta = 1 on C = D,
        the same single rounding) instead of first copying it into a new output."""
        if x.shape[0] <= fastlinear.MAX_M:
            return fastlinear.small_linear(x, w, b=b, residual=residual, norm=norm)
        if norm is not None:
            x = fused_ops.rms_norm(x, norm[0], norm[1])
        if residual is not None and b is None:
            return residual.addmm_(x, w.t()) if in_place else torch.addmm(residual, x, w.t())
        y = F.linear(x, w, b)
        return y if residual is None else y.add_(residual)

    def prompt_mixer(self, li, h, n_valid=None, own=False):
        """The attention half of layer li over a prompt's T rows h [T, H] at positions pos_buf .. pos_buf + T - 1:
        h + o(mixer(input_layernorm(h))). KDA: the projection, the q / k / v short convolutions (their caches end
        on the prompt's last real inputs), the f / g LoRA up-projections, the recurrence from the layer's state
        (fused_recurrent_kda up to KDA_CHUNK_ABOVE rows, chunk_kda beyond: the engine's mode switch,
        engine.py:946-949; padding rows past n_valid leave the state unchanged), rms_norm_gated; MLA: the
        q | k | v projection and mla_prefill_attn (padding rows are stored past the real ones, where the next
        decode steps overwrite them before any query reads them). own: h is the step's and dead after this call, so
        the o projection past fastlinear.MAX_M rows adds into it in place."""
        p = self.L[li]
        T = h.shape[0]
        if p["kind"] == "mla":
            if self.mla_qkv is not None:
                q, k, v = self.mla_qkv(li, p, h)
            else:
                qkv = self._rows(h, p["qkv"], p["qkv_b"], norm=p["ln1"])
                nq = p["nh"] * p["dqk"]
                q, k, v = qkv[:, :nq], qkv[:, nq:2 * nq], qkv[:, 2 * nq:]
            o = TA.mla_prefill_attn(q, k, v, p["kc"], p["vc"], self.pos)
            return self._rows(o, p["o"], p["o_b"], residual=h, in_place=own)
        H, K, V, R = p["heads"], p["K"], p["V"], p["rank"]
        pr = self._rows(h, p["proj"], p["proj_b"], norm=p["ln1"])
        nqk, nv = H * K, H * V
        q, k, v = TA.short_conv_many([pr[:, a:b] for a, b in ((0, nqk), (nqk, 2 * nqk), (2 * nqk, 2 * nqk + nv))],
                                     p["conv"], p["conv_w"], n_valid=n_valid)
        base = 2 * nqk + nv
        f = self._rows(pr[:, base:base + R], p["f_b"])
        gg = self._rows(pr[:, base + R:base + 2 * R], p["g_b"])
        kda = TA.chunk_kda if T > KDA_CHUNK_ABOVE else TA.fused_recurrent_kda
        o, _ = kda(q.view(1, T, H, K), k.view(1, T, H, K), v.view(1, T, H, V), f.view(1, T, H, K), pr[:, base + 2 * R:],
                   A_log=p["A_log"], dt_bias=p["dt_bias"], initial_state=p["state"], inplace=True,
                   use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True, beta_is_logits=True,
                   lower_bound=p["lower_bound"], n_valid=n_valid)
        ow, oe = p["o_norm"]
        on = TA.rms_norm_gated(o.reshape(T * H, V), gg.reshape(T * H, V), ow, oe)
        return self._rows(on.reshape(T, H * V), p["o"], p["o_b"], residual=h, in_place=own)

    def prompt_moe(self, li, h):
        """The MoE half of layer li over T rows: moe_block_decode up to fused_moe.MAX_DECODE_TOKENS rows (the
        reference's own split, engine.py:300-310 -> fused_moe.py:13-61), moe_block_prefill beyond.
        Returns (y, ids, wts)."""
        b = self.L[li]["blk"]
        kw = dict(top_k=b["top_k"], bias=b["bias"], scoring=self.scoring, n_group=b["n_group"],
                  topk_group=b["topk_group"], scale=b["scale"], s_gu=b["s_gu"], s_d=b["s_d"])
        if h.shape[0] <= fused_moe.MAX_DECODE_TOKENS:
            y, ids, wts, _ = fused_moe.moe_block_decode(h, b["norm_w"], b["eps"], b["w32"], b["w_gu"], b["w_d"], **kw)
        else:
            y, ids, wts, _ = fused_moe.moe_block_prefill(h, b["norm_w"], b["eps"], b["w32"], b["w_gu"], b["w_d"], **kw)
        return y, ids, wts

    def _prompt_rows(self, ids, h):
        if (ids is None) == (h is None):
            raise ValueError("FastThinkerStep.prefill: pass the prompt's token ids or its input rows h")
        if h is not None:
            h = h.reshape(-1, self.H)
            if h.dtype != self.embed.dtype:
                raise ValueError(f"FastThinkerStep.prefill: h must be {self.embed.dtype} rows of {self.H}")
            return h.contiguous()
        ids = ids.reshape(-1)
        if ids.dtype not in (torch.int64, torch.int32):
            raise ValueError("FastThinkerStep.prefill: ids must be int64 / int32 device tokens")
        return TA.embed_rows(self.embed, ids)

    def prefill(self, ids=None, h=None, *, n_valid=None, trace=False):
        """The engine's _prefill (engine.py:938-972) of one prompt at positions pos_buf .. pos_buf + T - 1: ids
        [1, T] / [T] device token ids (word_embeddings, engine.py:940), or h [1, T, H] / [T, H] input rows (the
        embeddings with audio features merged in, engine.py:941-944). Per layer h = prompt_moe(prompt_mixer(h)),
        then logits = lm_head(norm(h[T - 1])), tok_buf = argmax(logits), pos_buf += T: the state (KDA states and
        conv caches, MLA cache rows) advances as T decode steps would advance it. Returns the last token's logits
        [1, vocab]; with trace=True also the per-layer (input, mixer output, router ids, weights) list.
        n_valid: a one-element int64 device tensor n (the engine's prefill graphs, engine.py:716-757, 950-961: a
        prompt padded to a bucket length T, p_valid / p_conv_idx / p_last): the first n rows are the prompt, the rest
        padding that leaves the KDA states and conv caches as the n real tokens leave them; the logits are row
        n - 1's and pos_buf advances by n. Eager calls, or one capture per (padded) length: the position and n stay
        on the device, so a graph captured for T serves every prompt of up to T tokens (pos_buf + T <= max_len)."""
        h = self._prompt_rows(ids, h)
        T = h.shape[0]
        if T == 0:
            raise ValueError("FastThinkerStep.prefill: an empty prompt")
        if n_valid is not None and (n_valid.dtype != torch.int64 or n_valid.numel() != 1 or
                                    n_valid.device != h.device):
            raise ValueError("FastThinkerStep.prefill: n_valid must be a one-element int64 tensor on the device")
        nv = None if n_valid is None else n_valid.reshape(1).clamp(0, T)
        out = []
        owned = ids is not None  # the embedding rows are the step's own; rows handed in are the caller's
        for li in range(len(self.L)):
            h_in = h.clone() if trace else None
            # a layer's input is dead after its mixer unless it is the caller's: the o projection then adds into it
            hm = self.prompt_mixer(li, h, nv, own=owned or li > 0)
            h, rid, rw = self.prompt_moe(li, hm)
            if trace:
                out.append((h_in, hm.clone(), rid.clone(), rw.clone()))
        last = h[-1:] if nv is None else TA.embed_rows(h, (nv - 1).clamp_(min=0))
        logits = self.head_logits(last)
        TA.argmax_rows(logits, out=self.tok, workspace=self.amx_ws)
        self.pos.add_(T if nv is None else nv)
        return (logits, out) if trace else logits

    # ----------------------------------------------------------------------------------------------- step

    def __call__(self):
        h = self.embed_token()
        for li in range(len(self.L)):
            h = self.moe(li, self.mixer(li, h))
        logits = self.head_logits(h)
        TA.argmax_rows(logits, out=self.tok, workspace=self.amx_ws)
        self.pos.add_(1)
        return logits

    def trace(self):
        """The step run eagerly, keeping per layer (input, mixer output, router ids, weights): returns that list, the
        last layer's output and the logits. The state advances as in a call."""
        h, out = self.embed_token(), []
        for li in range(len(self.L)):
            h_in = h.clone()
            hm = self.mixer(li, h)
            h = self.moe(li, hm)
            nk = self.L[li]["blk"]["top_k"] + 1
            out.append((h_in, hm.clone(), self.ids[:, :nk].clone(), self.wts[:, :nk].clone()))
        logits = self.head_logits(h)
        TA.argmax_rows(logits, out=self.tok, workspace=self.amx_ws)
        self.pos.add_(1)
        return out, h, logits
