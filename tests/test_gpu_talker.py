"""GPU parity of the Talker kernels (rope_attn, qwen_decode_attn, silu_mul) against the CPU oracle.

bf16 outputs must match within rtol 2e-2 / atol 1e-2; cache rows written by the decode attention within
one bf16 ulp (k: fp32 rotation rounded once on both sides) or bit-exact (v is copied); cache rows other
than pos must be untouched. The Talker LLM shape is Qwen2-0.5B-like (14 query heads, 2 KV heads,
head dim 64, a 1024-position cache); the DiT / aggregator attention is 16 heads of 64 over 3 / 2 tokens."""
import math

import pytest
import torch

import fast_talker as FT
import workloads as W
from oracle import talker_oracle as T

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16
RTOL, ATOL = 2e-2, 1e-2


def close(got, want, rtol=RTOL, atol=ATOL):
    torch.testing.assert_close(got.float().cpu(), want.float().cpu(), rtol=rtol, atol=atol)


# -------------------------------------------------------------------------------------------- rope_attn

@pytest.mark.parametrize("B,S,D,heads", [(2, 3, 1024, 16), (1, 2, 1024, 16), (2, 1, 256, 4), (3, 5, 384, 3),
                                         (2, 8, 512, 8), (1, 4, 1536, 6), (2, 3, 96, 3), (4, 6, 160, 2)])
def test_rope_attn(B, S, D, heads):
    print(f"rope_attn B={B} S={S} D={D} heads={heads}", flush=True)
    g = torch.Generator().manual_seed(B * 100 + S)
    qkv = torch.randn(B, S, 3 * D, generator=g).to(BF)
    ang = torch.rand(S, D // heads // 2, generator=g) * 2 * math.pi
    cos, sin = ang.cos(), ang.sin()
    got = FT.rope_attn(qkv.to(DEV), cos.to(DEV), sin.to(DEV), heads)
    torch.cuda.synchronize()
    want = T.rope_attn(qkv, cos, sin, heads)
    close(got, want)
    if S == 1:
        assert torch.equal(got.cpu(), qkv[:, :, 2 * D:])


def test_rope_attn_rejects_long_sequences():
    qkv = torch.zeros(1, 9, 3 * 64, device=DEV, dtype=BF)
    cs = torch.zeros(9, 16, device=DEV)
    with pytest.raises(ValueError, match="seq"):
        FT.rope_attn(qkv, cs, cs, 2)


# ------------------------------------------------------------------------------------- decode attention

def _decode_inputs(nh, nkv, hd, max_len, seed, theta=1e6):
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn((nh + 2 * nkv) * hd, generator=g).to(BF)
    kc = torch.randn(1, nkv, max_len, hd, generator=g).to(BF)
    vc = torch.randn(1, nkv, max_len, hd, generator=g).to(BF)
    inv_freq = 1.0 / (theta ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))
    return qkv, kc, vc, inv_freq


def _run_decode(qkv, kc, vc, pos, inv_freq, nh, nkv, hd, pos_dtype=torch.int64):
    max_len = kc.shape[2]
    kd, vd = kc.to(DEV), vc.to(DEV)
    out = FT.qwen_decode_attn(qkv.to(DEV)[None], kd, vd, torch.tensor([pos], device=DEV, dtype=pos_dtype),
                              inv_freq.to(DEV), None, max_len, 1.0 / math.sqrt(hd), nh, nkv, hd)
    torch.cuda.synchronize()
    return out.cpu().reshape(-1), kd.cpu(), vd.cpu()


def _check_decode(qkv, kc, vc, pos, inv_freq, nh, nkv, hd, got, kd, vd):
    kw, vw = kc[0].clone(), vc[0].clone()
    want = T.qwen_decode_attn(qkv, kw, vw, pos, inv_freq, 1.0 / math.sqrt(hd), nh, nkv, hd)
    close(got, want)
    torch.testing.assert_close(kd[0, :, pos].float(), kw[:, pos].float(), rtol=2 ** -7, atol=0)
    assert torch.equal(vd[0, :, pos], vw[:, pos])
    others = torch.ones(kc.shape[2], dtype=torch.bool)
    others[pos] = False
    assert torch.equal(kd[0][:, others], kc[0][:, others]) and torch.equal(vd[0][:, others], vc[0][:, others])


@pytest.mark.parametrize("pos", [0, 1, 15, 16, 63, 64, 65, 500, 1023])
def test_decode_attn_talker_shape(pos):
    nh, nkv, hd, max_len = 14, 2, 64, 1024
    print(f"decode_attn nh={nh} nkv={nkv} hd={hd} max_len={max_len} pos={pos}", flush=True)
    qkv, kc, vc, inv_freq = _decode_inputs(nh, nkv, hd, max_len, 20 + pos)
    got, kd, vd = _run_decode(qkv, kc, vc, pos, inv_freq, nh, nkv, hd)
    _check_decode(qkv, kc, vc, pos, inv_freq, nh, nkv, hd, got, kd, vd)


@pytest.mark.parametrize("nh,nkv,hd,max_len,pos", [(16, 16, 128, 200, 130), (16, 1, 32, 100, 99),
                                                   (12, 2, 128, 4096, 4000), (8, 4, 256, 300, 257),
                                                   (6, 2, 96, 129, 128), (7, 7, 64, 1, 0),
                                                   (14, 2, 64, 2048, 1500), (14, 2, 64, 1025, 1024),
                                                   (4, 2, 32, 1024, 1023)])
def test_decode_attn_shapes(nh, nkv, hd, max_len, pos):
    """Head dims 32-256, GQA groups 1-16, caches of 1 to 4096 positions (a partial last chunk, pos at a chunk
    edge and at the cache end)."""
    print(f"decode_attn nh={nh} nkv={nkv} hd={hd} max_len={max_len} pos={pos}", flush=True)
    qkv, kc, vc, inv_freq = _decode_inputs(nh, nkv, hd, max_len, 40 + hd)
    got, kd, vd = _run_decode(qkv, kc, vc, pos, inv_freq, nh, nkv, hd, pos_dtype=torch.int32)
    _check_decode(qkv, kc, vc, pos, inv_freq, nh, nkv, hd, got, kd, vd)


def test_decode_attn_consecutive_steps_fill_the_cache():
    """Four decode steps at positions T..T+3 on one cache (the pattern of the reference's
    dev/test_fast_llm.py): each step reads the rows the previous steps wrote."""
    nh, nkv, hd, max_len, T0 = 14, 2, 64, 256, 97
    _, kc, vc, inv_freq = _decode_inputs(nh, nkv, hd, max_len, 60)
    kw, vw = kc[0].clone(), vc[0].clone()
    kd, vd = kc.to(DEV), vc.to(DEV)
    inv_d = inv_freq.to(DEV)
    pos = torch.empty(1, device=DEV, dtype=torch.long)
    ws = FT.decode_attn_workspace(nh, hd, max_len, DEV)
    g = torch.Generator().manual_seed(61)
    for j in range(4):
        qkv = torch.randn((nh + 2 * nkv) * hd, generator=g).to(BF)
        pos.fill_(T0 + j)
        got = FT.qwen_decode_attn(qkv.to(DEV), kd, vd, pos, inv_d, None, max_len, 0.125, nh, nkv, hd, workspace=ws)
        want = T.qwen_decode_attn(qkv, kw, vw, T0 + j, inv_freq, 0.125, nh, nkv, hd)
        close(got.reshape(-1), want)
    torch.cuda.synchronize()
    torch.testing.assert_close(kd[0].float().cpu(), kw.float(), rtol=2 ** -7, atol=0)
    assert torch.equal(vd[0].cpu(), vw)


def test_decode_attn_position_out_of_range_gives_nan_and_leaves_cache():
    nh, nkv, hd, max_len = 14, 2, 64, 128
    qkv, kc, vc, inv_freq = _decode_inputs(nh, nkv, hd, max_len, 70)
    for bad in (max_len, -1):
        got, kd, vd = _run_decode(qkv, kc, vc, bad, inv_freq, nh, nkv, hd)
        assert torch.isnan(got.float()).all()
        assert torch.equal(kd, kc) and torch.equal(vd, vc)


def test_decode_attn_graph_replays_follow_position():
    """Captured once, replayed with a new pos and new qkv each time (the Talker replays its decode step in a
    graph): every replay matches the oracle on the cache state it sees."""
    nh, nkv, hd, max_len = 14, 2, 64, 512
    _, kc, vc, inv_freq = _decode_inputs(nh, nkv, hd, max_len, 80)
    kw, vw = kc[0].clone(), vc[0].clone()
    kd, vd = kc.to(DEV), vc.to(DEV)
    inv_d = inv_freq.to(DEV)
    qkv = torch.zeros((nh + 2 * nkv) * hd, device=DEV, dtype=BF)
    pos = torch.zeros(1, device=DEV, dtype=torch.long)
    out = torch.empty(1, nh * hd, device=DEV, dtype=BF)
    ws = FT.decode_attn_workspace(nh, hd, max_len, DEV)

    def step():
        FT.qwen_decode_attn(qkv, kd, vd, pos, inv_d, out, max_len, 0.125, nh, nkv, hd, workspace=ws)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()  # eager warm-up (writes row 0 of the cache; restored below)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        step()
    torch.cuda.synchronize()
    kd.copy_(kc)
    vd.copy_(vc)
    g = torch.Generator().manual_seed(81)
    for j, p in enumerate((5, 6, 64, 300, 301)):
        x = torch.randn((nh + 2 * nkv) * hd, generator=g).to(BF)
        qkv.copy_(x)
        pos.fill_(p)
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = T.qwen_decode_attn(x, kw, vw, p, inv_freq, 0.125, nh, nkv, hd)
        close(out.reshape(-1), want)
    torch.testing.assert_close(kd[0].float().cpu(), kw.float(), rtol=2 ** -7, atol=0)


def test_decode_attn_rejects_bad_shapes():
    z = torch.zeros(1024, device=DEV, dtype=BF)
    cache = torch.zeros(1, 2, 8, 48, device=DEV, dtype=BF)
    pos = torch.zeros(1, device=DEV, dtype=torch.long)
    with pytest.raises(ValueError, match="head dim"):
        FT.qwen_decode_attn(z[: (4 + 4) * 48], cache, cache, pos, torch.zeros(24, device=DEV), None, 8, 0.1, 4, 2, 48)
    cache32 = torch.zeros(1, 2, 8, 32, device=DEV, dtype=BF)
    with pytest.raises(ValueError, match="pos"):
        FT.qwen_decode_attn(z[:512], cache32, cache32, pos.float(), torch.zeros(16, device=DEV), None, 8, 0.1, 12, 2,
                            32)


# --------------------------------------------------------------------------------------------- silu_mul

@pytest.mark.parametrize("rows,I", [(1, 4864), (3, 4864), (1, 100), (2, 8), (1, 1), (4, 2816)])
def test_silu_mul(rows, I):
    g = torch.Generator().manual_seed(rows * 7 + I)
    gu = (torch.randn(rows, 2 * I, generator=g) * 3).to(BF)
    got = FT.silu_mul(gu.to(DEV)).cpu()
    want = T.silu_mul(gu, I)
    torch.testing.assert_close(got.float(), want.float(), rtol=2 ** -7, atol=0)
    assert (got == want).float().mean() > 0.99


@pytest.mark.parametrize("M,K,I,norm", [(1, 896, 4864, True), (2, 896, 4864, False), (1, 2048, 1408, True),
                                         (3, 64, 40, True), (1, 4864, 896, False), (16, 1024, 256, True)])
def test_gate_up_silu_equals_small_linear_then_silu_mul(M, K, I, norm):
    import fastlinear
    x = W.normal((M, K), 0.5, 600 + K, DEV)
    w = W.normal((2 * I, K), 0.05, 601, DEV)
    nm = (W.normal((K,), 0.02, 602, DEV, mean=1.0), 1e-6) if norm else None
    fused = FT.gate_up_silu(x, w, norm=nm)
    unfused = FT.silu_mul(fastlinear.small_linear(x, w, norm=nm))
    torch.cuda.synchronize()
    assert torch.equal(fused, unfused)
    gu_o = T.silu_mul(fastlinear.small_linear(x, w, norm=nm).cpu(), I)
    assert torch.equal(fused.cpu(), gu_o) or (fused.cpu().float() - gu_o.float()).abs().max() < 2e-2


def test_silu_mul_strided_rows_and_out():
    g = torch.Generator().manual_seed(5)
    big = (torch.randn(3, 2 * 4864 + 64, generator=g) * 3).to(BF).to(DEV)
    gu = big[:, : 2 * 4864]
    out = torch.empty(3, 4864 + 8, device=DEV, dtype=BF)
    res = FT.silu_mul(gu, out[:, :4864])
    torch.cuda.synchronize()
    torch.testing.assert_close(res.float().cpu(), T.silu_mul(gu.cpu(), 4864).float(), rtol=2 ** -7, atol=0)
    assert res.data_ptr() == out.data_ptr()


# ------------------------------------------------------------------------------------ Talker LLM step

def _cpu_layers(fs):
    """FastQwen2Step's fused per-layer weights as CPU tensors (the oracle's input)."""
    out = []
    for L in fs.layers:
        out.append({k: (v[0].cpu(), v[1]) if isinstance(v, tuple) else v.cpu() for k, v in L.items()})
    return out


def test_fast_qwen2_step_matches_oracle_and_unfused_path():
    """Three decode steps of a 4-layer Qwen2-0.5B-shaped Talker LLM after a 150-position context (the pattern
    of the reference's dev/test_fast_llm.py): each output matches the oracle's restatement of the fast step,
    and the unfused fp32 StaticQwen2 forward to bf16 accuracy; the caches match the oracle's."""
    nh, nkv, hd, T0 = 14, 2, 64, 150
    llm = W.TalkerLLM(layers=4, max_len=256, seed=200, device=DEV)
    llm.fill_cache(T0, seed=300)
    fs = FT.FastQwen2Step(llm)
    layers = _cpu_layers(fs)
    kc, vc = llm.k[:, 0].cpu(), llm.v[:, 0].cpu()
    k32, v32 = kc.float(), vc.float()
    inv = llm.inv_freq.cpu()
    fn = (llm.m.norm.weight.detach().cpu(), llm.m.norm.variance_epsilon)
    for j in range(3):
        x = W.normal((1, 1, W.TALKER_HIDDEN), 0.1, 400 + j)
        pos = T0 + j
        print(f"talker step pos={pos}", flush=True)
        out = fs(x.to(DEV), torch.tensor([pos], device=DEV)).float().cpu()
        want = T.fast_qwen2_step(x, layers, kc, vc, pos, inv, nh, nkv, hd, fn)
        ref = T.static_qwen2_step_fp32(x, layers, k32, v32, pos, inv, nh, nkv, hd, fn)
        close(out, want, atol=2e-2)
        rel = ((out - ref.float()).norm() / ref.float().norm()).item()
        assert rel < 3e-2, rel
    torch.cuda.synchronize()
    close(llm.k[:, 0], kc)
    close(llm.v[:, 0], vc)


def test_fast_qwen2_step_graph_replays_match_eager():
    """The step captured once and replayed with new inputs and positions equals eager calls bit for bit,
    cache writes included."""
    H, T0 = W.TALKER_HIDDEN, 60
    llm = W.TalkerLLM(layers=3, max_len=128, seed=210, device=DEV)
    llm.fill_cache(T0, seed=310)
    fs = FT.FastQwen2Step(llm)
    k0, v0 = llm.k.clone(), llm.v.clone()
    xs = [W.normal((1, 1, H), 0.1, 500 + j, DEV) for j in range(3)]
    eager = [fs(xs[j], torch.tensor([T0 + j], device=DEV)).clone() for j in range(3)]
    k_e, v_e = llm.k.clone(), llm.v.clone()
    x_s = xs[0].clone()
    pos_s = torch.full((1,), T0, device=DEV, dtype=torch.long)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fs(x_s, pos_s)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out_s = fs(x_s, pos_s)
    torch.cuda.synchronize()
    llm.k.copy_(k0)
    llm.v.copy_(v0)
    for j in range(3):
        x_s.copy_(xs[j])
        pos_s.fill_(T0 + j)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_s, eager[j]), f"replay {j}"
    assert torch.equal(llm.k, k_e) and torch.equal(llm.v, v_e)


# ------------------------------------------------------------------------------------------ Talker tail

def test_fast_tail_matches_oracle():
    """Three flow-matching steps of a 2-block DiT (hidden 1024, 16 heads) and a 1-block aggregator: latent,
    next LLM input and stop probability against the oracle's restatement of FastTail on the same constants."""
    tk = W.TalkerTail(seed=700, device=DEV, depth=2, agg_depth=1, steps=3)
    ft = FT.FastTail(tk, tk.ts, tk.dts, tk.cfg_strength)
    P = T.tail_constants(ft)
    for trial in range(2):
        hidden = W.normal((1, 1, W.TALKER_HIDDEN), 1.0, 710 + trial)
        hist = W.normal((1, 1, 64), 1.0, 720 + trial)
        noise = W.normal((1, 1, 64), 1.0, 730 + trial)
        print(f"fast_tail trial {trial}", flush=True)
        lat, x_next, stop = ft(hidden.to(DEV), hist.to(DEV), noise.to(DEV))
        w_lat, w_x, w_stop = T.fast_tail(P, hidden, hist, noise)
        # the CFG update y += (3 pred - 2 null) dt amplifies one-ulp bf16 differences from step to step, so
        # the composed tail is held to a norm-relative bar (as the reference's dev/test_fast_tail.py reports
        # it); every kernel inside is held to the elementwise bar in its own tests
        for got, want in ((lat, w_lat), (x_next, w_x)):
            d = got.float().cpu() - want.float()
            assert (d.norm() / want.float().norm()).item() < 2e-2 and d.abs().max().item() < 0.1
        assert abs(stop.item() - w_stop.item()) < 1e-2


@pytest.mark.parametrize("L,dt_dtype", [(64, torch.bfloat16), (1000, torch.float32), (1, torch.bfloat16)])
def test_cfg_update_equals_the_torch_expression(L, dt_dtype):
    g = torch.Generator().manual_seed(L)
    y = torch.randn(1, L, generator=g).to(BF).to(DEV)
    out = torch.randn(2, L, generator=g).to(BF).to(DEV)
    dt = torch.tensor([0.1015625] if dt_dtype == BF else 0.1015625, dtype=dt_dtype, device=DEV)
    got = FT.cfg_update(y, out, 2.0, dt)
    pred, null = out[0:1], out[1:2]
    want = y + (pred + (pred - null) * 2.0) * dt
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_fast_tail_graph_replays_match_eager():
    """The tail captured once and replayed on new inputs equals eager calls bit for bit (the engine replays
    it from a graph, engine.py:1412-1414)."""
    tk = W.TalkerTail(seed=740, device=DEV, depth=1, agg_depth=1, steps=2)
    ft = FT.FastTail(tk, tk.ts, tk.dts, tk.cfg_strength)
    ins = [[W.normal(shape, 1.0, 750 + 3 * j + k, DEV) for k, shape in enumerate(((1, 1, W.TALKER_HIDDEN),
                                                                                     (1, 1, 64), (1, 1, 64)))]
           for j in range(3)]
    eager = [tuple(t.clone() for t in ft(*x)) for x in ins]
    bufs = [t.clone() for t in ins[0]]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ft(*bufs)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        outs = ft(*bufs)
    for j in range(3):
        for b, x in zip(bufs, ins[j]):
            b.copy_(x)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager[j]):
            assert torch.equal(o, e), f"replay {j}"
