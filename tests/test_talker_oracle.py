"""Pins the CPU oracle of the Talker kernels (oracle/talker_oracle.py) without the reference code:
closed forms, an independent complex-number statement of the interleaved rotary, engine.py's unfused
StaticQwen2 attention (rotate_half + masked scaled_dot_product_attention over the GQA-expanded cache,
engine.py:1268-1291) in float64, torch's silu, and invariances of the online softmax. Each check is chosen
so that a plausible mistake (a flipped sign, the wrong pair partner, a transposed operand, the wrong KV
head of a query head) fails; the planted-mistake tests below show two such failures."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import talker_oracle as T

BF = torch.bfloat16


def _qkv(B, S, D, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(B, S, 3 * D, generator=g).to(BF)


def _angles(S, P, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.rand(S, P, generator=g) * 2 * math.pi


def _rope_attn_independent(qkv, ang, heads):
    """Interleaved pairs as complex numbers times e^{i angle}, rounded to bf16, then float64 SDPA."""
    B, S, D3 = qkv.shape
    D = D3 // 3
    HD = D // heads
    x = qkv.double().reshape(B, S, 3, heads, HD // 2, 2)
    rot = torch.polar(torch.ones_like(ang, dtype=torch.float64), ang.double())[None, :, None, :]

    def turn(t):
        z = torch.view_as_complex(t.contiguous()) * rot
        return torch.view_as_real(z).float().to(BF).double().reshape(B, S, heads, HD)

    q, k = turn(x[:, :, 0]), turn(x[:, :, 1])
    v = x[:, :, 2].reshape(B, S, heads, HD)
    o = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2))
    return o.transpose(1, 2).reshape(B, S, D)


@pytest.mark.parametrize("B,S,D,heads", [(2, 3, 256, 4), (1, 2, 128, 2), (3, 5, 384, 3)])
def test_rope_attn_matches_complex_rotation_and_sdpa(B, S, D, heads):
    qkv = _qkv(B, S, D, 1)
    ang = _angles(S, D // heads // 2, 2)
    got = T.rope_attn(qkv, ang.cos(), ang.sin(), heads)
    want = _rope_attn_independent(qkv, ang, heads)
    # p is rounded to bf16 before p . v (fast_talker.py:64), so the outputs differ by ~2^-9 relative
    torch.testing.assert_close(got.double(), want, rtol=2e-2, atol=2e-2)


def test_rope_attn_one_token_returns_v():
    qkv = _qkv(2, 1, 128, 3)
    ang = _angles(1, 16, 4)
    got = T.rope_attn(qkv, ang.cos(), ang.sin(), 4)
    assert torch.equal(got, qkv[:, :, 256:])


def test_rope_attn_rejects_a_flipped_rotation():
    qkv = _qkv(2, 3, 256, 5)
    ang = _angles(3, 32, 6)
    want = _rope_attn_independent(qkv, ang, 4)
    wrong = T.rope_attn(qkv, ang.cos(), -ang.sin(), 4)  # the same as e c + o s, o c - e s
    assert (wrong.double() - want).abs().max() > 0.1


def _static_qwen2_attention(qkv, k_cache, v_cache, pos, inv_freq, nh, nkv, hd):
    """engine.py:1268-1291 for one token in float64: emb = [f, f]; cos / sin rounded to bf16 (DTYPE);
    q*cos + rotate_half(q)*sin; index_copy into the cache; SDPA over the expanded cache with mask ar <= pos."""
    f = torch.tensor(float(pos), dtype=torch.float32) * inv_freq.float()
    emb = torch.cat([f, f])
    cos, sin = emb.cos().to(BF).double(), emb.sin().to(BF).double()

    def rotate_half(x):
        x1, x2 = x.chunk(2, dim=-1)
        return torch.cat((-x2, x1), dim=-1)

    x = qkv.double()
    q = x[: nh * hd].reshape(nh, hd)
    k = x[nh * hd:(nh + nkv) * hd].reshape(nkv, hd)
    v = x[(nh + nkv) * hd:].reshape(nkv, hd)
    q = (q * cos + rotate_half(q) * sin).float().to(BF).double()
    k = (k * cos + rotate_half(k) * sin).float().to(BF)
    kc, vc = k_cache.clone(), v_cache.clone()
    kc[:, pos] = k
    vc[:, pos] = v.to(BF)
    rep = nh // nkv
    max_len = kc.shape[1]
    kk = kc.double()[:, None].expand(nkv, rep, max_len, hd).reshape(nh, max_len, hd)
    vv = vc.double()[:, None].expand(nkv, rep, max_len, hd).reshape(nh, max_len, hd)
    mask = (torch.arange(max_len) <= pos)[None, None]
    o = F.scaled_dot_product_attention(q[:, None], kk, vv, attn_mask=mask)
    return o.reshape(-1), kc, vc


def _decode_case(nh, nkv, hd, max_len, pos, seed):
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn((nh + 2 * nkv) * hd, generator=g).to(BF)
    kc = torch.randn(nkv, max_len, hd, generator=g).to(BF)
    vc = torch.randn(nkv, max_len, hd, generator=g).to(BF)
    inv_freq = 1.0 / (10000.0 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))
    return qkv, kc, vc, inv_freq


@pytest.mark.parametrize("nh,nkv,hd,max_len,pos", [(14, 2, 64, 300, 0), (14, 2, 64, 300, 1), (14, 2, 64, 300, 129),
                                                   (14, 2, 64, 300, 299), (8, 8, 128, 80, 50), (16, 1, 32, 70, 64)])
def test_qwen_decode_matches_static_qwen2_path(nh, nkv, hd, max_len, pos):
    qkv, kc, vc, inv_freq = _decode_case(nh, nkv, hd, max_len, pos, 7)
    want, kw, vw = _static_qwen2_attention(qkv, kc, vc, pos, inv_freq, nh, nkv, hd)
    got = T.qwen_decode_attn(qkv, kc, vc, pos, inv_freq, 1.0 / math.sqrt(hd), nh, nkv, hd)
    torch.testing.assert_close(got.double(), want, rtol=2e-2, atol=1e-2)
    assert torch.equal(vc, vw)
    # the fused form rounds once, the unfused one too here; a 1-ulp tie may still differ
    torch.testing.assert_close(kc.float(), kw.float(), rtol=2 ** -7, atol=0)


def test_qwen_decode_position_zero_returns_v_and_keeps_k():
    nh, nkv, hd = 14, 2, 64
    qkv, kc, vc, inv_freq = _decode_case(nh, nkv, hd, 16, 0, 8)
    got = T.qwen_decode_attn(qkv, kc, vc, 0, inv_freq, 0.125, nh, nkv, hd)
    v = qkv[(nh + nkv) * hd:].reshape(nkv, hd)
    assert torch.equal(got.reshape(nh, hd), v[torch.arange(nh) // (nh // nkv)])
    assert torch.equal(kc[:, 0], qkv[nh * hd:(nh + nkv) * hd].reshape(nkv, hd))  # cos 0 = 1, sin 0 = 0


def test_qwen_decode_zero_query_averages_values():
    nh, nkv, hd, pos = 4, 2, 64, 77
    qkv, kc, vc, inv_freq = _decode_case(nh, nkv, hd, 100, pos, 9)
    qkv[: nh * hd] = 0
    got = T.qwen_decode_attn(qkv, kc, vc, pos, inv_freq, 0.125, nh, nkv, hd)
    mean = vc.double()[:, : pos + 1].mean(1)  # row pos now holds the current v
    want = mean[torch.arange(nh) // 2].reshape(-1)
    torch.testing.assert_close(got.double(), want, rtol=2 ** -8, atol=1e-6)


def test_qwen_decode_online_softmax_is_blocking_invariant():
    nh, nkv, hd, pos = 14, 2, 64, 200
    qkv, kc, vc, inv_freq = _decode_case(nh, nkv, hd, 256, pos, 10)
    outs = [T.qwen_decode_attn(qkv, kc.clone(), vc.clone(), pos, inv_freq, 0.125, nh, nkv, hd, block=b)
            for b in (1, 7, 64, 1 << 20)]
    for o in outs[1:]:
        torch.testing.assert_close(o.float(), outs[0].float(), rtol=2 ** -7, atol=1e-3)


def test_qwen_decode_rejects_the_wrong_kv_head():
    nh, nkv, hd, pos = 8, 2, 64, 40
    qkv, kc, vc, inv_freq = _decode_case(nh, nkv, hd, 64, pos, 11)
    want, _, _ = _static_qwen2_attention(qkv, kc, vc, pos, inv_freq, nh, nkv, hd)
    # planted mistake: heads assigned to KV heads round-robin (h % nkv) instead of in groups (h // G)
    perm = torch.arange(nh).reshape(nkv, nh // nkv).t().reshape(-1)
    q = qkv[: nh * hd].reshape(nh, hd)[perm].reshape(-1)
    wrong = T.qwen_decode_attn(torch.cat([q, qkv[nh * hd:]]), kc.clone(), vc.clone(), pos, inv_freq,
                               0.125, nh, nkv, hd)
    assert (wrong.reshape(nh, hd)[perm.argsort()].double() - want.reshape(nh, hd)).abs().max() > 0.1


def test_silu_mul_matches_torch_silu_and_closed_forms():
    g = torch.Generator().manual_seed(12)
    I = 1000
    gu = (torch.randn(3, 2 * I, generator=g) * 4).to(BF)
    got = T.silu_mul(gu, I)
    want = (F.silu(gu[:, :I].double()).float().to(BF).double() * gu[:, I:].double()).float().to(BF)
    torch.testing.assert_close(got.float(), want.float(), rtol=2 ** -7, atol=0)
    special = torch.tensor([[0.0, 30.0, -100.0, 1.5, 2.0, 3.0]]).to(BF)  # g | u
    out = T.silu_mul(special, 3).float()
    assert out[0, 0] == 0 and out[0, 1] == 60.0 and out[0, 2] == 0


def _layers_of(llm):
    """The fused per-layer weights FastQwen2Step builds (q|k|v and gate|up stacked by rows), on the CPU."""
    out = []
    for layer in llm.m.layers:
        a, mlp = layer.self_attn, layer.mlp
        out.append({"wqkv": torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight]),
                    "bqkv": torch.cat([a.q_proj.bias, a.k_proj.bias, a.v_proj.bias]),
                    "wo": a.o_proj.weight, "wgu": torch.cat([mlp.gate_proj.weight, mlp.up_proj.weight]),
                    "wd": mlp.down_proj.weight,
                    "n1": (layer.input_layernorm.weight.detach(), layer.input_layernorm.variance_epsilon),
                    "n2": (layer.post_attention_layernorm.weight.detach(),
                           layer.post_attention_layernorm.variance_epsilon)})
    return out


@pytest.mark.parametrize("pos", [0, 40])
def test_fast_step_oracle_matches_unfused_static_qwen2(pos):
    import workloads as W
    llm = W.TalkerLLM(layers=2, max_len=64, seed=30)
    llm.fill_cache(pos, seed=31)
    layers = _layers_of(llm)
    x = W.normal((1, 1, W.TALKER_HIDDEN), 0.1, 32)  # small like embeddings, so the layers dominate the output
    fn = (llm.m.norm.weight.detach(), llm.m.norm.variance_epsilon)
    kc, vc = llm.k[:, 0].clone(), llm.v[:, 0].clone()
    got = T.fast_qwen2_step(x, layers, kc, vc, pos, llm.inv_freq, 14, 2, 64, fn).float()
    k32, v32 = llm.k[:, 0].float(), llm.v[:, 0].float()
    ref = T.static_qwen2_step_fp32(x, layers, k32, v32, pos, llm.inv_freq, 14, 2, 64, fn)
    assert ((got - ref).norm() / ref.norm()).item() < 2e-2
    torch.testing.assert_close(kc.float(), k32, rtol=2e-2, atol=2e-2)
    # planted mistake: k and v swapped in the fused projection
    bad = [dict(L, wqkv=torch.cat([L["wqkv"][:896], L["wqkv"][1024:], L["wqkv"][896:1024]]),
                bqkv=torch.cat([L["bqkv"][:896], L["bqkv"][1024:], L["bqkv"][896:1024]])) for L in layers]
    wrong = T.fast_qwen2_step(x, bad, llm.k[:, 0].clone(), llm.v[:, 0].clone(), pos, llm.inv_freq, 14, 2, 64, fn)
    assert ((wrong.float() - ref).norm() / ref.norm()).item() > 0.2


def test_fast_tail_oracle_closed_forms():
    """Zero step sizes leave the latent at the noise exactly; the stop probability is the 2-way softmax of
    the stop head on the LLM hidden state (F.linear in float64); the aggregator output depends on the latent."""
    import warnings
    import fast_talker as FT
    import workloads as W
    tk = W.TalkerTail(seed=5, depth=1, agg_depth=1, steps=2, dim=128, heads=2, mlp=256, latent=16, llm_hidden=64)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")  # autocast("cuda") on a CPU-only torch only warns
        ft = FT.FastTail(tk, tk.ts, tk.dts, tk.cfg_strength)
    P = T.tail_constants(ft)
    hidden, hist, noise = (W.normal(s, 1.0, 60 + i) for i, s in enumerate(((1, 1, 64), (1, 1, 16), (1, 1, 16))))
    lat0, x0, stop = T.fast_tail(dict(P, dts=[torch.zeros(1, dtype=BF)] * 2), hidden, hist, noise)
    assert torch.equal(lat0, noise)
    want = F.softmax(F.linear(hidden.double().reshape(1, -1), P["s_w"].double(), P["s_b"].double()), -1)[0, 1]
    assert abs(stop.item() - want.item()) < 1e-2
    lat, x1, _ = T.fast_tail(P, hidden, hist, noise)
    assert not torch.equal(lat, noise) and not torch.equal(x1, x0)
