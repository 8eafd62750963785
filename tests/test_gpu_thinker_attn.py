"""GPU parity of the thinker's attention mixers (KDA recurrent core, short convolution, gated norm, MLA decode and
prompt attention, the hybrid step's decode and prefill) against oracle/thinker_attn_oracle.py on seeded inputs. bf16 outputs within rtol 2e-2 / atol 1e-2; the fp32
KDA state within rtol 1e-3 / atol 1e-4 of the float64 oracle; cache rows bit-exact."""
import pytest
import torch
import torch.nn.functional as F

import thinker_attn as TA
import workloads as W
from oracle import thinker_attn_oracle as A

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def close(got, want, rtol=2e-2, atol=1e-2):
    torch.testing.assert_close(got.float().cpu(), want.float().cpu(), rtol=rtol, atol=atol)


def _kda_inputs(T, H, K, V, seed, gdt=torch.float32):
    q = W.normal((1, T, H, K), 1.0, seed, DEV)
    k = W.normal((1, T, H, K), 1.0, seed + 1, DEV)
    v = W.normal((1, T, H, V), 1.0, seed + 2, DEV)
    g = W.normal((1, T, H, K), 1.0, seed + 3, DEV, dtype=gdt)
    beta = torch.sigmoid(W.normal((1, T, H), 1.0, seed + 4, DEV, dtype=torch.float32))
    A_log = W.normal((H,), 0.5, seed + 5, DEV, dtype=torch.float32)
    dt = W.normal((H * K,), 0.5, seed + 6, DEV, dtype=torch.float32)
    S0 = W.normal((1, H, K, V), 0.3, seed + 7, DEV, dtype=torch.float32)
    return q, k, v, g, beta, A_log, dt, S0


@pytest.mark.parametrize("T,H,K,V", [(1, 16, 128, 128), (7, 4, 128, 128), (64, 2, 128, 128), (3, 5, 64, 64),
                                     (9, 3, 128, 64), (4, 2, 64, 128), (3, 2, 64, 48), (2, 3, 128, 32),
                                     (37, 2, 128, 40), (130, 3, 128, 128), (33, 2, 64, 56), (16, 1, 128, 8)])
@pytest.mark.parametrize("gate", ["softplus", "lower_bound", "none"])
def test_kda_recurrent_matches_oracle(T, H, K, V, gate):
    print(f"[kda] T={T} H={H} K={K} V={V} gate={gate}", flush=True)
    q, k, v, g, beta, A_log, dt, S0 = _kda_inputs(T, H, K, V, 200 + T + K, torch.bfloat16 if gate == "none" else torch.float32)
    if gate == "none":  # g is already a log decay: keep it small and negative
        g = (-0.1 * g.float().abs()).to(BF)
    lb = -5.0 if gate == "lower_bound" else None
    state = S0.clone()
    o, fin = TA.fused_recurrent_kda(q, k, v, g, beta, A_log=A_log, dt_bias=dt, initial_state=state,
                                    output_final_state=True, use_qk_l2norm_in_kernel=True,
                                    use_gate_in_kernel=gate != "none", lower_bound=lb)
    assert torch.equal(state, S0)  # not in place by default
    ro, rS = A.kda_recurrent(q[0].cpu(), k[0].cpu(), v[0].cpu(), g[0].cpu(), beta[0].cpu(), S0[0].cpu(),
                             A_log=A_log.cpu(), dt_bias=dt.cpu(), use_gate=gate != "none", lower_bound=lb)
    close(o[0], ro)
    torch.testing.assert_close(fin[0].cpu().double(), rS, rtol=1e-3, atol=1e-4)


@pytest.mark.parametrize("T,H,K,V", [(2, 3, 128, 32), (3, 5, 64, 64), (9, 3, 128, 64), (16, 1, 128, 8), (17, 2, 128, 128),
                                     (33, 2, 64, 56), (37, 2, 128, 40), (130, 3, 128, 128), (200, 2, 128, 128)])
@pytest.mark.parametrize("gate", ["softplus", "lower_bound", "none"])
def test_kda_chunk_matches_oracle(T, H, K, V, gate):
    """chunk_kda (16-token chunks in closed form) against the float64 recurrence, chunk boundaries and partial last
    chunks included; T <= 2 takes the one-launch decode kernel."""
    print(f"[kda chunk] T={T} H={H} K={K} V={V} gate={gate}", flush=True)
    q, k, v, g, beta, A_log, dt, S0 = _kda_inputs(T, H, K, V, 700 + T + K, torch.bfloat16 if gate == "none" else torch.float32)
    if gate == "none":
        g = (-0.1 * g.float().abs()).to(BF)
    lb = -5.0 if gate == "lower_bound" else None
    o, fin = TA.chunk_kda(q, k, v, g, beta, A_log=A_log, dt_bias=dt, initial_state=S0, output_final_state=True,
                          use_qk_l2norm_in_kernel=True, use_gate_in_kernel=gate != "none", lower_bound=lb)
    ro, rS = A.kda_recurrent(q[0].cpu(), k[0].cpu(), v[0].cpu(), g[0].cpu(), beta[0].cpu(), S0[0].cpu(),
                             A_log=A_log.cpu(), dt_bias=dt.cpu(), use_gate=gate != "none", lower_bound=lb)
    close(o[0], ro)
    torch.testing.assert_close(fin[0].cpu().double(), rS, rtol=1e-3, atol=1e-4)


def test_kda_chunk_full_prompt_and_strong_decay():
    """The hybrid thinker's shape, 512 tokens over 16 heads of 128 x 128, against the float64 recurrence; then decays
    of e^-30 .. e^-80 per token, whose products over a chunk underflow: the chunk form takes them as products, never
    as ratios, so the outputs stay finite and match."""
    H, K, V, T = 16, 128, 128, 512
    q, k, v, g, beta, A_log, dt, S0 = _kda_inputs(T, H, K, V, 720)
    beta = W.normal((1, T, H), 1.0, 721, DEV)
    kw = dict(A_log=A_log, dt_bias=dt, output_final_state=True, use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
              beta_is_logits=True)
    print("[kda chunk] 512 tokens x 16 heads", flush=True)
    o, fin = TA.chunk_kda(q, k, v, g, beta, initial_state=S0, **kw)
    ro, rS = A.kda_recurrent(q[0].cpu(), k[0].cpu(), v[0].cpu(), g[0].cpu(), torch.sigmoid(beta[0].float()).cpu(),
                             S0[0].cpu(), A_log=A_log.cpu(), dt_bias=dt.cpu())
    close(o[0], ro)
    torch.testing.assert_close(fin[0].cpu().double(), rS, rtol=1e-3, atol=1e-4)
    T = 48
    q, k, v, g, beta, A_log, dt, S0 = _kda_inputs(T, 2, K, V, 730, torch.bfloat16)
    g = (-30.0 - 50.0 * torch.rand(g.shape, generator=torch.Generator().manual_seed(731))).to(DEV, BF)  # log decays
    print("[kda chunk] strong decay", flush=True)
    o, fin = TA.chunk_kda(q, k, v, g, beta, initial_state=S0, output_final_state=True, use_qk_l2norm_in_kernel=True)
    assert torch.isfinite(o).all() and torch.isfinite(fin).all()
    ro, rS = A.kda_recurrent(q[0].cpu(), k[0].cpu(), v[0].cpu(), g[0].cpu(), beta[0].cpu(), S0[0].cpu(), use_gate=False)
    close(o[0], ro)
    torch.testing.assert_close(fin[0].cpu().double(), rS, rtol=1e-3, atol=1e-4)


def test_kda_inplace_decode_steps_and_graph_replays():
    """A decode step (T = 1) updates the state in place; a captured step replayed with new tokens advances it
    exactly as eager steps do."""
    H, K, V = 8, 128, 128
    q, k, v, g, beta, A_log, dt, S0 = _kda_inputs(1, H, K, V, 300)
    st_e, st_g = S0.clone(), S0.clone()
    out_g = torch.empty(1, 1, H, V, device=DEV, dtype=BF)

    def step(state, out=None):
        return TA.fused_recurrent_kda(q, k, v, g, beta, A_log=A_log, dt_bias=dt, initial_state=state, inplace=True,
                                      use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True, out=out)[0]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=s):
        step(st_g, out_g)
    torch.cuda.synchronize()
    assert torch.equal(st_g, S0)  # capture does not run the kernel
    for i in range(3):
        for t, seed in ((q, 310), (k, 311), (v, 312)):
            t.copy_(W.normal(t.shape, 1.0, seed + 10 * i, DEV))
        want = step(st_e).clone()
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, want) and torch.equal(st_g, st_e), i
    assert not torch.equal(st_e, S0)


def test_kda_zero_write_strength_keeps_the_state():
    """beta = 0 with gate inputs of -1e30 (the padded-prompt trick, engine.py:252-253): the state is unchanged."""
    H, K, V = 4, 128, 128
    q, k, v, g, beta, A_log, dt, S0 = _kda_inputs(3, H, K, V, 320)
    g = torch.full_like(g, -1e30)
    _, fin = TA.fused_recurrent_kda(q, k, v, g, torch.zeros_like(beta), A_log=A_log, dt_bias=dt, initial_state=S0,
                                    output_final_state=True, use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True)
    assert torch.equal(fin, S0)


@pytest.mark.parametrize("chunked", [False, True])
def test_kda_prompt_recurrence_is_deterministic(chunked):
    """The prompt forms' waves share each staged chunk (and its v values) through LDS; a wave running ahead into the
    next chunk must not overwrite what the others still read. Five runs of a 300-token prompt (19 chunks) over 16
    heads from one state, eagerly and from a graph, give the same outputs and states bit for bit (fused_recurrent_kda
    and chunk_kda)."""
    H, K, V, T = 16, 128, 128, 300
    fn = TA.chunk_kda if chunked else TA.fused_recurrent_kda
    q, k, v, g, beta, A_log, dt, S0 = _kda_inputs(T, H, K, V, 640)
    beta = W.normal((1, T, H), 1.0, 641, DEV)
    kw = dict(A_log=A_log, dt_bias=dt, inplace=True, use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
              beta_is_logits=True)
    st = S0.clone()
    o_ref, _ = fn(q, k, v, g, beta, initial_state=st, **kw)
    s_ref = st.clone()
    ws = (TA.kda_chunk_workspace if chunked else TA.kda_workspace)(T, H, K, DEV)
    out = torch.empty_like(o_ref)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=s):
        fn(q, k, v, g, beta, initial_state=st, out=out, workspace=ws, **kw)
    for i in range(5):
        st.copy_(S0)
        o, _ = fn(q, k, v, g, beta, initial_state=st, **kw)
        torch.cuda.synchronize()
        assert torch.equal(o, o_ref) and torch.equal(st, s_ref), ("eager", i)
        st.copy_(S0)
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, o_ref) and torch.equal(st, s_ref), ("graph", i)


@pytest.mark.parametrize("T,n,H,V", [(32, 20, 3, 128), (40, 33, 2, 64), (2, 1, 4, 128), (17, 0, 2, 128), (16, 16, 1, 32),
                                     (64, 23, 2, 128)])
@pytest.mark.parametrize("chunked", [False, True])
def test_kda_padding_tokens_leave_the_state_unchanged(T, n, H, V, chunked):
    """A prompt padded from n to T tokens with n_valid = n (the engine's prefill graphs): the state after it and the
    first n outputs equal those of the n-token prompt bit for bit, whatever the padding rows hold (both forms: in the
    chunk form a padding token's u is 0 and its decay 1, so it adds exact zeros and multiplies by exact ones)."""
    K = 128
    fn = TA.chunk_kda if chunked else TA.fused_recurrent_kda
    print(f"[kda pad] T={T} n={n} H={H} V={V} chunked={chunked}", flush=True)
    q, k, v, g, beta, A_log, dt, S0 = _kda_inputs(T, H, K, V, 600 + T)
    beta = W.normal((1, T, H), 1.0, 610, DEV)  # logits
    kw = dict(A_log=A_log, dt_bias=dt, inplace=True, use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
              beta_is_logits=True)
    s_pad, s_ref = S0.clone(), S0.clone()
    o_pad, _ = fn(q, k, v, g, beta, initial_state=s_pad, n_valid=torch.tensor([n], device=DEV), **kw)
    if n:
        o_ref, _ = fn(q[:, :n], k[:, :n], v[:, :n], g[:, :n], beta[:, :n], initial_state=s_ref, **kw)
        assert torch.equal(o_pad[:, :n], o_ref)
    assert torch.equal(s_pad, s_ref)


@pytest.mark.parametrize("T,n,C,Wd", [(40, 23, 2048, 4), (32, 2, 77, 4), (16, 0, 130, 3), (5, 5, 64, 8)])
def test_short_conv_cache_ends_on_the_real_tokens(T, n, C, Wd):
    x = W.normal((T, C), 1.0, 620 + T, DEV)
    cache = W.normal((1, C, Wd), 1.0, 621, DEV)
    w = W.normal((C, 1, Wd), 0.5, 622, DEV)
    c_pad, c_ref = cache.clone(), cache.clone()
    y_pad = TA.short_conv(x, c_pad, w, n_valid=torch.tensor([n], device=DEV))
    if n:
        y_ref = TA.short_conv(x[:n], c_ref, w)
        assert torch.equal(y_pad[:n], y_ref)
    assert torch.equal(c_pad, c_ref)


@pytest.mark.parametrize("T,C,Wd", [(1, 6144, 4), (5, 6144, 4), (3, 1000, 2), (2, 77, 8), (40, 2048, 4), (17, 77, 8),
                                    (100, 130, 3), (16, 64, 4)])
def test_short_conv_matches_oracle(T, C, Wd):
    x = W.normal((1, T, C), 1.0, 400 + T, DEV)
    cache = W.normal((1, C, Wd), 1.0, 401, DEV)
    w = W.normal((C, 1, Wd), 0.5, 402, DEV)
    b = W.normal((C,), 0.5, 403, DEV)
    c0 = cache.clone()
    y = TA.short_conv(x, cache, w, b)
    ry, rc = A.short_conv(x[0].cpu(), c0[0].cpu(), w[:, 0].cpu(), b.cpu())
    close(y[0], ry)
    assert torch.equal(cache[0].cpu(), rc.to(BF))  # the window holds bf16 inputs exactly


@pytest.mark.parametrize("T,Cs,Wd,n", [(1, (2048, 2048, 2048), 4, None), (40, (2048, 2048, 2048), 4, None),
                                       (17, (77, 300, 64), 3, None), (100, (130, 2048), 8, None), (33, (96,), 2, None),
                                       (24, (2048, 2048, 2048), 4, 19), (24, (150, 64, 77, 20), 4, 0)])
def test_short_conv_many_equals_separate_calls(T, Cs, Wd, n):
    """One launch over several convolutions (the q, k, v of a KDA prompt, and other channel counts, with and without
    n_valid): every output and every updated cache equals its own short_conv call bit for bit, read through strided
    column slices of one projection row as the prefill passes them."""
    pr = W.normal((T, sum(Cs) + 5), 1.0, 630 + T, DEV)
    xs, o = [], 0
    for C in Cs:
        xs.append(pr[:, o:o + C])
        o += C
    caches = [W.normal((1, C, Wd), 1.0, 631 + i, DEV) for i, C in enumerate(Cs)]
    ws = [W.normal((C, 1, Wd), 0.5, 641 + i, DEV) for i, C in enumerate(Cs)]
    nv = None if n is None else torch.tensor([n], device=DEV)
    c_one = [c.clone() for c in caches]
    ys = TA.short_conv_many(xs, caches, ws, n_valid=nv)
    for x, c, w, y in zip(xs, c_one, ws, ys):
        assert torch.equal(y, TA.short_conv(x, c, w, n_valid=nv))
    for c, c1 in zip(caches, c_one):
        assert torch.equal(c, c1)


def test_rms_norm_gated_matches_oracle():
    x = W.normal((7, 16, 128), 2.0, 410, DEV)
    g = W.normal((7, 16, 128), 1.0, 411, DEV)
    w = W.normal((128,), 0.1, 412, DEV, mean=1.0)
    close(TA.rms_norm_gated(x, g, w, 1e-5), A.rms_norm_gated(x.cpu(), g.cpu(), w.cpu(), 1e-5))


@pytest.mark.parametrize("nh,dq,dv,L", [(16, 192, 128, 1024), (4, 64, 64, 300), (2, 96, 32, 70), (3, 72, 40, 100),
                                        (2, 512, 256, 90), (1, 8, 8, 33), (2, 64, 64, 2048), (1, 32, 32, 9000)])
def test_mla_decode_attn_matches_oracle(nh, dq, dv, L):
    """Positions at chunk edges and the cache end; caches past 1024 positions take the merge's chunks beyond its
    loaded-ahead batch, past 8192 its maxima beyond the first 256 chunks."""
    kc = W.normal((1, nh, L, dq), 1.0, 420, DEV)
    vc = W.normal((1, nh, L, dv), 1.0, 421, DEV)
    for pos in sorted({p for p in (0, 1, 31, 32, 33, 63, 64, 65, L // 2, L - 1) if p < L}):
        print(f"[mla] nh={nh} dq={dq} dv={dv} L={L} pos={pos}", flush=True)
        q = W.normal((nh, dq), 1.0, 430 + pos, DEV)
        kn = W.normal((nh, dq), 1.0, 431 + pos, DEV)
        vn = W.normal((nh, dv), 1.0, 432 + pos, DEV)
        k0, v0 = kc.clone(), vc.clone()
        out = TA.mla_decode_attn(q, kn, vn, kc, vc, torch.tensor([pos], device=DEV))
        ro, rk, rv = A.mla_decode_attn(q.cpu(), kn.cpu(), vn.cpu(), k0[0].cpu(), v0[0].cpu(), pos)
        close(out, ro)
        assert torch.equal(kc[0].cpu(), rk) and torch.equal(vc[0].cpu(), rv)


def test_mla_rows_past_the_position_are_never_read():
    """Cache rows past pos filled with NaN (an uninitialised cache) leave the output finite and equal to the
    oracle's; the last position of a partial chunk and of the cache included."""
    nh, dq, dv, L = 4, 192, 128, 100
    for pos in (0, 31, 37, 99):
        kc = W.normal((1, nh, L, dq), 1.0, 470, DEV)
        vc = W.normal((1, nh, L, dv), 1.0, 471, DEV)
        kc[:, :, pos + 1:] = float("nan")
        vc[:, :, pos + 1:] = float("nan")
        k0, v0 = kc.clone(), vc.clone()
        q, kn, vn = W.normal((nh, dq), 1.0, 472, DEV), W.normal((nh, dq), 1.0, 473, DEV), W.normal((nh, dv), 1.0, 474, DEV)
        out = TA.mla_decode_attn(q, kn, vn, kc, vc, torch.tensor([pos], device=DEV, dtype=torch.int32))
        ro, _, _ = A.mla_decode_attn(q.cpu(), kn.cpu(), vn.cpu(), k0[0].cpu(), v0[0].cpu(), pos)
        assert torch.isfinite(out.float()).all(), pos
        close(out, ro)


def test_mla_out_of_range_position_writes_nothing():
    nh, dq, dv, L = 4, 64, 64, 128
    kc = W.normal((1, nh, L, dq), 1.0, 440, DEV)
    vc = W.normal((1, nh, L, dv), 1.0, 441, DEV)
    k0, v0 = kc.clone(), vc.clone()
    q = W.normal((nh, dq), 1.0, 442, DEV)
    out = TA.mla_decode_attn(q, q, q, kc, vc, torch.tensor([L], device=DEV))
    assert torch.isnan(out.float()).all() and torch.equal(kc, k0) and torch.equal(vc, v0)


def test_mla_graph_replays_follow_the_position():
    """The attention captured once and replayed at positions 5, 6, 7 equals eager calls on a copy of the cache."""
    nh, dq, dv, L = 16, 192, 128, 256
    kc = W.normal((1, nh, L, dq), 1.0, 450, DEV)
    vc = W.normal((1, nh, L, dv), 1.0, 451, DEV)
    ke, ve = kc.clone(), vc.clone()
    q = W.normal((nh, dq), 1.0, 452, DEV)
    kn, vn = W.normal((nh, dq), 1.0, 453, DEV), W.normal((nh, dv), 1.0, 454, DEV)
    pos = torch.tensor([5], device=DEV)
    out = torch.empty(nh, dv, device=DEV, dtype=BF)
    ws = TA.mla_attn_workspace(nh, dv, L, DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        TA.mla_decode_attn(q, kn, vn, kc, vc, pos, out=out, workspace=ws)
    for p in (5, 6, 7):
        pos.fill_(p)
        q.copy_(W.normal((nh, dq), 1.0, 460 + p, DEV))
        want = TA.mla_decode_attn(q, kn, vn, ke, ve, torch.tensor([p], device=DEV)).clone()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want) and torch.equal(kc, ke) and torch.equal(vc, ve), p


def _prompt(nh, dq, dv, T, seed, packed=False):
    """q, k, v of T tokens; packed: column slices of one [T, nh (2 dq + dv)] projection output (the product's form)."""
    if packed:
        qkv = W.normal((T, nh * (2 * dq + dv)), 1.0, seed, DEV)
        nq = nh * dq
        return qkv[:, :nq], qkv[:, nq:2 * nq], qkv[:, 2 * nq:]
    return (W.normal((T, nh, dq), 1.0, seed, DEV), W.normal((T, nh, dq), 1.0, seed + 1, DEV),
            W.normal((T, nh, dv), 1.0, seed + 2, DEV))


@pytest.mark.parametrize("nh,dq,dv,L,T,pos,packed", [
    (16, 192, 128, 1024, 128, 512, True), (16, 192, 128, 1024, 17, 0, False), (4, 64, 64, 300, 33, 31, False),
    (2, 96, 32, 70, 70, 0, True), (3, 72, 40, 100, 5, 95, False), (1, 8, 8, 40, 1, 7, False),
    (2, 256, 128, 600, 300, 200, True), (2, 200, 48, 64, 16, 16, False), (1, 32, 16, 2100, 64, 2000, False),
    (16, 192, 128, 1100, 520, 300, False), (16, 64, 64, 700, 530, 100, True)])
def test_mla_prefill_attn_matches_oracle(nh, dq, dv, L, T, pos, packed):
    """Prompts at the cache start and end, lengths off the 16-query and 32-key tiles, head dims off the 32-wide
    MFMA step, and q / k / v as column slices of a projection output; grids of 512 workgroups and more (the last
    two) take 4 waves per workgroup, smaller ones 8."""
    print(f"[mla prefill] nh={nh} dq={dq} dv={dv} L={L} T={T} pos={pos} packed={packed}", flush=True)
    kc = W.normal((1, nh, L, dq), 1.0, 500, DEV)
    vc = W.normal((1, nh, L, dv), 1.0, 501, DEV)
    k0, v0 = kc.clone(), vc.clone()
    q, kn, vn = _prompt(nh, dq, dv, T, 502, packed)
    out = TA.mla_prefill_attn(q, kn, vn, kc, vc, torch.tensor([pos], device=DEV))
    ro, rk, rv = A.mla_prefill_attn(q.reshape(T, nh, dq).cpu(), kn.reshape(T, nh, dq).cpu(),
                                    vn.reshape(T, nh, dv).cpu(), k0[0].cpu(), v0[0].cpu(), pos)
    assert out.shape == (T, nh * dv)
    close(out.reshape(T, nh, dv), ro)
    assert torch.equal(kc[0].cpu(), rk) and torch.equal(vc[0].cpu(), rv)


def test_mla_prefill_rows_past_the_prompt_are_never_read_and_out_of_range_writes_nothing():
    nh, dq, dv, L = 4, 192, 128, 200
    for T, pos in ((1, 0), (20, 13), (45, 155)):
        print(f"[mla prefill nan] T={T} pos={pos}", flush=True)
        kc = W.normal((1, nh, L, dq), 1.0, 510, DEV)
        vc = W.normal((1, nh, L, dv), 1.0, 511, DEV)
        kc[:, :, pos + T:] = float("nan")
        vc[:, :, pos + T:] = float("nan")
        k0, v0 = kc.clone(), vc.clone()
        q, kn, vn = _prompt(nh, dq, dv, T, 512)
        out = TA.mla_prefill_attn(q, kn, vn, kc, vc, torch.tensor([pos], device=DEV, dtype=torch.int32))
        ro, _, _ = A.mla_prefill_attn(q.cpu(), kn.cpu(), vn.cpu(), k0[0].cpu(), v0[0].cpu(), pos)
        assert torch.isfinite(out.float()).all()
        close(out.reshape(T, nh, dv), ro)
    kc = W.normal((1, nh, L, dq), 1.0, 513, DEV)
    vc = W.normal((1, nh, L, dv), 1.0, 514, DEV)
    k0, v0 = kc.clone(), vc.clone()
    q, kn, vn = _prompt(nh, dq, dv, 8, 515)
    for pos in (L - 7, -1):  # one row past the end; a negative position
        print(f"[mla prefill out of range] pos={pos}", flush=True)
        out = TA.mla_prefill_attn(q, kn, vn, kc, vc, torch.tensor([pos], device=DEV))
        assert torch.isnan(out.float()).all() and torch.equal(kc, k0) and torch.equal(vc, v0)


def test_mla_prefill_one_token_equals_decode_and_graph_replays_follow_the_position():
    nh, dq, dv, L = 16, 192, 128, 512
    kc = W.normal((1, nh, L, dq), 1.0, 520, DEV)
    vc = W.normal((1, nh, L, dv), 1.0, 521, DEV)
    kd, vd = kc.clone(), vc.clone()
    q, kn, vn = _prompt(nh, dq, dv, 1, 522)
    pos = torch.tensor([77], device=DEV)
    a = TA.mla_prefill_attn(q, kn, vn, kc, vc, pos)
    b = TA.mla_decode_attn(q, kn, vn, kd, vd, pos)
    close(a.reshape(nh, dv), b, rtol=1e-2, atol=1e-2)
    assert torch.equal(kc, kd) and torch.equal(vc, vd)
    # a 40-token prompt captured once, replayed at positions 10, 50, 90 on the graph's cache, against eager calls
    T = 40
    q, kn, vn = _prompt(nh, dq, dv, T, 523, packed=True)
    ke, ve = kc.clone(), vc.clone()
    pos = torch.tensor([10], device=DEV)
    out = torch.empty(T, nh * dv, device=DEV, dtype=BF)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        TA.mla_prefill_attn(q, kn, vn, kc, vc, pos, out=out)
    for p in (10, 50, 90):
        print(f"[mla prefill graph] pos={p}", flush=True)
        pos.fill_(p)
        g.replay()
        torch.cuda.synchronize()
        want = TA.mla_prefill_attn(q, kn, vn, ke, ve, torch.tensor([p], device=DEV))
        torch.cuda.synchronize()
        assert torch.equal(out, want) and torch.equal(kc, ke) and torch.equal(vc, ve)


def test_kda_beta_logits_apply_the_sigmoid():
    """beta_is_logits=True (the kernel applies the sigmoid of the beta projection) against the oracle given the
    sigmoid's values."""
    T, H, K, V = 2, 4, 128, 128
    q, k, v, g, _, A_log, dt, S0 = _kda_inputs(T, H, K, V, 330)
    b = W.normal((1, T, H), 2.0, 335, DEV)
    o, fin = TA.fused_recurrent_kda(q, k, v, g, b, A_log=A_log, dt_bias=dt, initial_state=S0, output_final_state=True,
                                    use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True, beta_is_logits=True)
    ro, rS = A.kda_recurrent(q[0].cpu(), k[0].cpu(), v[0].cpu(), g[0].cpu(), torch.sigmoid(b[0].cpu().double()),
                             S0[0].cpu(), A_log=A_log.cpu(), dt_bias=dt.cpu())
    close(o[0], ro)
    torch.testing.assert_close(fin[0].cpu().double(), rS, rtol=1e-3, atol=1e-4)


# ------------------------------------------------------------------------------ the hybrid decode step

def test_hybrid_step_graph_replays_equal_eager_steps():
    """The hybrid thinker decode step (KDA and MLA layers + MoE blocks + LM head, the position advancing on the
    device) captured once: three replays equal three eager steps of an identical copy, logits, every KDA state
    and conv cache, the MLA caches and the position bit for bit."""
    print("[hybrid] graph vs eager, 8 layers", flush=True)
    eager = W.HybridThinkerStep(8, DEV, pos=100, seed=7000)
    graphed = W.HybridThinkerStep(8, DEV, pos=100, seed=7000)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = graphed()
    torch.cuda.synchronize()
    for i in range(3):
        want = eager().clone()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), i
        a, b = eager.state_copy(), graphed.state_copy()
        assert torch.equal(a["pos"], b["pos"]) and int(b["pos"]) == 101 + i
        assert torch.equal(a["tok"], b["tok"]) and int(b["tok"]) == int(out.float().cpu().argmax()), i
        for la, lb in zip(a["L"], b["L"]):
            for key in la:
                xa, xb = la[key], lb[key]
                for ta, tb in zip(xa if isinstance(xa, tuple) else (xa,), xb if isinstance(xb, tuple) else (xb,)):
                    assert torch.equal(ta, tb), (i, key)
    del eager, graphed, g, out
    torch.cuda.empty_cache()


def _oracle_mixer(p, st, h, pos):
    """One hybrid layer's mixer on the oracle (state st: the layer's KDA state / conv cache or MLA caches before)."""
    from oracle import moe_oracle as O
    H = W.HIDDEN
    kd = W.KDA_HEADS * W.KDA_DIM
    if p["kind"] == "mla":
        qkv = O.small_linear(h, p["qkv"].cpu(), norm=(p["ln1"].cpu(), W.EPS))
        nq = W.MLA_HEADS * W.MLA_QK
        o, _, _ = A.mla_decode_attn(qkv[0, :nq].reshape(W.MLA_HEADS, -1), qkv[0, nq:2 * nq].reshape(W.MLA_HEADS, -1),
                                    qkv[0, 2 * nq:].reshape(W.MLA_HEADS, -1), st["kc"][0].cpu(), st["vc"][0].cpu(),
                                    pos)
        return O.small_linear(o.reshape(1, -1).to(BF), p["o"].cpu(), residual=h)
    pr = O.small_linear(h, p["proj"].cpu(), norm=(p["ln1"].cpu(), W.EPS))
    f = O.small_linear(pr[:, 3 * kd:3 * kd + W.KDA_LORA], p["f_b"].cpu())
    gg = O.small_linear(pr[:, 3 * kd + W.KDA_LORA:3 * kd + 2 * W.KDA_LORA], p["g_b"].cpu())
    conv = torch.cat([c[0] for c in st["conv"]]).cpu()  # the q, k and v caches of the layer, [3 kd, 4]
    qkv, _ = A.short_conv(pr[:, :3 * kd], conv, p["conv_w"][:, 0].cpu())
    qkv = qkv.to(BF)
    beta = torch.sigmoid(pr[:, 3 * kd + 2 * W.KDA_LORA:].double())
    shp = (1, W.KDA_HEADS, W.KDA_DIM)
    o, _ = A.kda_recurrent(qkv[:, :kd].reshape(shp), qkv[:, kd:2 * kd].reshape(shp), qkv[:, 2 * kd:].reshape(shp),
                           f.reshape(shp), beta.reshape(1, -1), st["state"][0].cpu(), A_log=p["A_log"].cpu(),
                           dt_bias=p["dt_bias"].cpu())
    on = A.rms_norm_gated(o[0].to(BF), gg.reshape(W.KDA_HEADS, W.KDA_DIM), p["o_norm"].cpu(), 1e-5)
    return O.small_linear(on.reshape(1, kd).to(BF), p["o"].cpu(), residual=h)


def test_hybrid_step_layers_match_the_oracle():
    """4 layers (3 KDA, 1 MLA) at full width, each half checked on the GPU's own input: the mixer (projections,
    convolutions, KDA recurrence or MLA attention, output norm / projection) and the MoE block, within the bf16
    tolerance on at least 99.5 % of elements (an element can be the small difference of two large bf16 values)."""
    from oracle import moe_oracle as O
    print("[hybrid] 4 layers vs oracle", flush=True)
    step = W.HybridThinkerStep(4, DEV, pos=200, seed=7100)
    before = step.state_copy()
    trace, _, logits = step.trace()
    # the step's two ends: its input is the embedding row of the token, the argmax of its logits the next token
    assert torch.equal(trace[0][0].cpu(), step.embed[int(before["tok"])].cpu()[None])
    assert int(step.tok) == int(logits.float().cpu().argmax())
    for li, (p, st, (h_in, hm, ids, wts)) in enumerate(zip(step.L, before["L"], trace)):
        want = _oracle_mixer(p, st, h_in.cpu(), 200)
        d = (hm.float().cpu() - want.float()).abs()
        ok = float((d <= 1e-2 + 2e-2 * want.float().abs()).float().mean())
        print(f"[hybrid] layer {li} ({p['kind']}) mixer: max |d| {float(d.max()):.4f} within-tol {ok:.4f}", flush=True)
        assert ok >= 0.995, (li, p["kind"], ok)
        assert float((hm.float() - h_in.float()).abs().mean()) > 0.05 * float(h_in.float().abs().mean())  # it mixes
        b = {k: v.cpu() for k, v in p["blk"].items()}
        xn = O.rms_norm(hm.cpu(), b["norm_w"], W.EPS)
        moe = O.moe(xn, b["w_gu"], b["w_d"], ids.cpu(), wts.cpu(), residual=hm.cpu())
        nxt = trace[li + 1][0] if li + 1 < len(trace) else None
        if nxt is not None:
            d = (nxt.float().cpu() - moe.float()).abs()
            assert float((d <= 1e-2 + 2e-2 * moe.float().abs()).float().mean()) >= 0.995, li


def _oracle_prompt_mixer(p, st, h, pos):
    """One hybrid layer's mixer over a prompt's T rows h [T, H] on the oracle (state st: the layer's state before).
    Returns (out [T, H], the state after: KDA state and the conv windows, or the MLA caches)."""
    from oracle import moe_oracle as O
    T = h.shape[0]
    kd = W.KDA_HEADS * W.KDA_DIM
    if p["kind"] == "mla":
        qkv = O.small_linear(h, p["qkv"].cpu(), norm=(p["ln1"].cpu(), W.EPS))
        nq = W.MLA_HEADS * W.MLA_QK
        o, kc, vc = A.mla_prefill_attn(qkv[:, :nq].reshape(T, W.MLA_HEADS, -1),
                                       qkv[:, nq:2 * nq].reshape(T, W.MLA_HEADS, -1),
                                       qkv[:, 2 * nq:].reshape(T, W.MLA_HEADS, -1), st["kc"][0].cpu(),
                                       st["vc"][0].cpu(), pos)
        return O.small_linear(o.reshape(T, -1).to(BF), p["o"].cpu(), residual=h), {"kc": kc, "vc": vc}
    pr = O.small_linear(h, p["proj"].cpu(), norm=(p["ln1"].cpu(), W.EPS))
    f = O.small_linear(pr[:, 3 * kd:3 * kd + W.KDA_LORA], p["f_b"].cpu())
    gg = O.small_linear(pr[:, 3 * kd + W.KDA_LORA:3 * kd + 2 * W.KDA_LORA], p["g_b"].cpu())
    conv = torch.cat([c[0] for c in st["conv"]]).cpu()
    qkv, win = A.short_conv(pr[:, :3 * kd], conv, p["conv_w"][:, 0].cpu())
    qkv = qkv.to(BF)
    beta = torch.sigmoid(pr[:, 3 * kd + 2 * W.KDA_LORA:].double())
    shp = (T, W.KDA_HEADS, W.KDA_DIM)
    o, S = A.kda_recurrent(qkv[:, :kd].reshape(shp), qkv[:, kd:2 * kd].reshape(shp), qkv[:, 2 * kd:].reshape(shp),
                           f.reshape(shp), beta, st["state"][0].cpu(), A_log=p["A_log"].cpu(),
                           dt_bias=p["dt_bias"].cpu())
    on = A.rms_norm_gated(o.to(BF), gg.reshape(shp), p["o_norm"].cpu(), 1e-5)
    return O.small_linear(on.reshape(T, kd).to(BF), p["o"].cpu(), residual=h), {"state": S, "conv": win}


def _within(got, want, atol=1e-2, rtol=2e-2):
    d = (got.float().cpu() - want.float()).abs()
    return float((d <= atol + rtol * want.float().abs()).float().mean()), float(d.max())


@pytest.mark.parametrize("T", [40, 5])
def test_fast_thinker_prefill_layers_match_the_oracle(T):
    """A T-token prompt through 4 layers (3 KDA, 1 MLA) at full width, each half checked on the GPU's own input: the
    mixer (projections, convolutions, the KDA recurrence over T tokens or the causal MLA attention) and the MoE
    block; the layers' states after the prompt (KDA state, conv windows, MLA cache rows); the head on the last
    token. T = 40 takes the library GEMMs and the prefill MoE block, T = 5 the GEMVs and the decode MoE block."""
    from oracle import moe_oracle as O
    pos = 200
    print(f"[hybrid prefill] T={T} 4 layers vs oracle", flush=True)
    step = W.HybridThinkerStep(4, DEV, pos=pos, seed=7200)
    before = step.state_copy()
    ids = torch.randint(0, step.embed.shape[0], (T,), generator=torch.Generator().manual_seed(T)).to(DEV)
    logits, trace = step.fast.prefill(ids, trace=True)
    assert int(step.pos) == pos + T and int(step.tok) == int(logits.float().cpu().argmax())
    assert torch.equal(trace[0][0].cpu(), step.embed[ids].cpu())
    after = step.state_copy()
    for li, (p, st, (h_in, hm, rid, rw)) in enumerate(zip(step.L, before["L"], trace)):
        want, st_want = _oracle_prompt_mixer(p, st, h_in.cpu(), pos)
        ok, dmax = _within(hm, want)
        print(f"[hybrid prefill] T={T} layer {li} ({p['kind']}) mixer: max |d| {dmax:.4f} within-tol {ok:.4f}",
              flush=True)
        assert ok >= 0.995, (li, p["kind"], ok)
        if p["kind"] == "mla":
            for key in ("kc", "vc"):
                got = after["L"][li][key][0]
                assert torch.equal(got[:, :pos].cpu(), st[key][0][:, :pos].cpu())
                assert torch.equal(got[:, pos + T:].cpu(), st[key][0][:, pos + T:].cpu())
                ok, _ = _within(got[:, pos:pos + T], st_want[key][:, pos:pos + T])
                assert ok >= 0.995, (li, key, ok)
        else:
            ok, _ = _within(after["L"][li]["state"][0], st_want["state"], atol=2e-3)
            assert ok >= 0.995, (li, "state", ok)
            win = torch.cat([c[0] for c in after["L"][li]["conv"]])
            ok, _ = _within(win, st_want["conv"])
            assert ok >= 0.995, (li, "conv", ok)
        b = {k: v.cpu() for k, v in p["blk"].items()}
        xn = O.rms_norm(hm.cpu(), b["norm_w"], W.EPS)
        moe = O.moe(xn, b["w_gu"], b["w_d"], rid.cpu(), rw.cpu(), residual=hm.cpu())
        if li + 1 < len(trace):
            ok, _ = _within(trace[li + 1][0], moe)
            assert ok >= 0.995, (li, "moe", ok)
    del step
    torch.cuda.empty_cache()


def test_fast_thinker_prefill_then_decode_follows_token_by_token_decode():
    """A 24-token prompt in one prefill, and the same 24 tokens fed one decode step at a time to an identical
    model: the same position, the layer states and the last logits agree to the bf16 level, and the next decode
    step from either state picks the same token; a prefill captured in a graph replays bit for bit."""
    T, pos = 24, 100
    a = W.HybridThinkerStep(4, DEV, pos=pos, seed=7300)
    b = W.HybridThinkerStep(4, DEV, pos=pos, seed=7300)
    ids = torch.randint(0, a.embed.shape[0], (T,), generator=torch.Generator().manual_seed(3)).to(DEV)
    print("[hybrid prefill] prefill vs 24 decode steps", flush=True)
    la = a.fast.prefill(ids)
    for t in range(T):
        b.tok.fill_(int(ids[t]))
        lb = b.fast()
    torch.cuda.synchronize()
    assert int(a.pos) == int(b.pos) == pos + T
    cos = F.cosine_similarity(la.float().reshape(-1), lb.float().reshape(-1), dim=0)
    assert float(cos) > 0.999, float(cos)
    sa, sb = a.state_copy(), b.state_copy()
    for li, (x, y) in enumerate(zip(sa["L"], sb["L"])):
        for key in x:
            for ta, tb in zip(x[key] if isinstance(x[key], tuple) else (x[key],),
                              y[key] if isinstance(y[key], tuple) else (y[key],)):
                c = F.cosine_similarity(ta.float().reshape(-1), tb.float().reshape(-1), dim=0)
                assert float(c) > 0.999, (li, key, float(c))
    b.tok.copy_(a.tok)
    na, nb = a.fast(), b.fast()
    assert int(a.tok) == int(b.tok) or float(F.cosine_similarity(na.float().reshape(-1), nb.float().reshape(-1),
                                                                 dim=0)) > 0.999
    # graph capture: the prompt captured once at the current position, replayed against eager prefills of a copy
    c = W.HybridThinkerStep(4, DEV, pos=pos, seed=7400)
    d = W.HybridThinkerStep(4, DEV, pos=pos, seed=7400)
    c.fast.prefill(ids)  # warm-up (library GEMM plans); both models stay in the same state
    d.fast.prefill(ids)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = c.fast.prefill(ids)
    torch.cuda.synchronize()
    for i in range(3):
        print(f"[hybrid prefill graph] replay {i}", flush=True)
        g.replay()
        torch.cuda.synchronize()
        want = d.fast.prefill(ids)
        torch.cuda.synchronize()
        assert torch.equal(out, want), i
        assert int(c.pos) == int(d.pos) and int(c.tok) == int(d.tok)
        for x, y in zip(c.state_copy()["L"], d.state_copy()["L"]):
            for key in x:
                for ta, tb in zip(x[key] if isinstance(x[key], tuple) else (x[key],),
                                  y[key] if isinstance(y[key], tuple) else (y[key],)):
                    assert torch.equal(ta, tb), (i, key)
    del a, b, c, d, g, out
    torch.cuda.empty_cache()


def _states_close(a, b, what, rows=None, exact=False, min_cos=0.999, keys=("state", "conv", "kc", "vc")):
    """KDA states and conv caches, and the MLA cache rows `rows` (a slice; all when None), of two state copies."""
    for li, (x, y) in enumerate(zip(a["L"], b["L"])):
        for key in (kk for kk in x if kk in keys):
            for ta, tb in zip(x[key] if isinstance(x[key], tuple) else (x[key],),
                              y[key] if isinstance(y[key], tuple) else (y[key],)):
                if key in ("kc", "vc") and rows is not None:
                    ta, tb = ta[:, :, rows], tb[:, :, rows]
                if exact:
                    assert torch.equal(ta, tb), (what, li, key)
                    continue
                c = float(F.cosine_similarity(ta.float().reshape(-1), tb.float().reshape(-1), dim=0))
                assert c > min_cos, (what, li, key, c)


def test_fast_thinker_long_prompt_takes_the_chunked_recurrence(monkeypatch):
    """Past KDA_CHUNK_ABOVE rows the prompt's KDA layers run chunk_kda (the engine's chunk mode, engine.py:946-949);
    the same 200-token prompt with the recurrent form in every layer gives the same logits and layer states to the
    fp32 level (the two forms differ only in the order of their fp32 sums)."""
    import thinker_step
    T, pos = 200, 300
    a = W.HybridThinkerStep(4, DEV, pos=pos, seed=7500)
    b = W.HybridThinkerStep(4, DEV, pos=pos, seed=7500)
    ids = torch.randint(0, a.embed.shape[0], (T,), generator=torch.Generator().manual_seed(7501)).to(DEV)
    calls, orig = [], TA.chunk_kda
    monkeypatch.setattr(TA, "chunk_kda", lambda *x, **kw: (calls.append(1), orig(*x, **kw))[1])
    print("[hybrid prefill] 200 tokens, chunked KDA", flush=True)
    la = a.fast.prefill(ids)
    assert len(calls) == 3  # the 3 KDA layers
    monkeypatch.setattr(thinker_step, "KDA_CHUNK_ABOVE", 1 << 30)
    print("[hybrid prefill] 200 tokens, recurrent KDA", flush=True)
    lb = b.fast.prefill(ids)
    torch.cuda.synchronize()
    assert len(calls) == 3 and int(a.pos) == int(b.pos) == pos + T
    assert float(F.cosine_similarity(la.float().reshape(-1), lb.float().reshape(-1), dim=0)) > 0.999
    _states_close(a.state_copy(), b.state_copy(), "chunked vs recurrent", rows=slice(0, pos + T))


def test_fast_thinker_prefill_graph_for_a_bucket_serves_shorter_prompts():
    """The engine's prefill graphs (engine.py:716-757, 950-961): one capture for a 32-token bucket, replayed for
    prompts of 20, 7 and 32 tokens padded with token 0 (n_valid on the device), against eager prefills of the
    unpadded prompts on an identical model: the same position and next token, the layer states and logits
    agree (bit for bit at the full length, to the bf16 level otherwise: the projection GEMMs see another row count)."""
    Tb, pos = 32, 300
    a = W.HybridThinkerStep(4, DEV, pos=pos, seed=7500)
    b = W.HybridThinkerStep(4, DEV, pos=pos, seed=7500)
    vocab = a.embed.shape[0]
    prompt = torch.randint(0, vocab, (Tb,), generator=torch.Generator().manual_seed(11)).to(DEV)
    ids = torch.zeros(Tb, device=DEV, dtype=torch.long)
    nv = torch.tensor([Tb], device=DEV)
    ids.copy_(prompt)
    a.fast.prefill(ids, n_valid=nv)  # warm-up on both models, which stay identical
    b.fast.prefill(prompt)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        logits = a.fast.prefill(ids, n_valid=nv)
    torch.cuda.synchronize()
    for n in (20, 7, 32):
        print(f"[hybrid prefill bucket] n={n} of {Tb}", flush=True)
        p = torch.randint(0, vocab, (n,), generator=torch.Generator().manual_seed(100 + n)).to(DEV)
        ids.zero_()
        ids[:n] = p
        nv.fill_(n)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = b.fast.prefill(p)
        torch.cuda.synchronize()
        sa, sb = a.state_copy(), b.state_copy()
        p0 = int(sa["pos"]) - n
        assert int(sa["pos"]) == int(sb["pos"])
        if n == Tb:
            assert torch.equal(logits, want) and int(a.tok) == int(b.tok)
            _states_close(sa, sb, n, exact=True)
        else:
            c = float(F.cosine_similarity(logits.float().reshape(-1), want.float().reshape(-1), dim=0))
            assert c > 0.999, (n, c)
            _states_close(sa, sb, n, rows=slice(0, p0 + n))  # rows past the prompt hold the padding in a
            _states_close(sa, sb, n, rows=slice(p0 + Tb, None), exact=True, keys=("kc", "vc"))
        # the next decode steps write over the padding rows of the MLA caches before any query reads them
        a.tok.copy_(b.tok)
        for key in ("kc", "vc"):
            for pa, pb in zip(a.L, b.L):
                if key in pa:
                    pa[key].copy_(pb[key])
        for pa, pb in zip(a.L, b.L):  # realign the two models for the next prompt
            for key in ("state", "conv"):
                if key in pa:
                    for ta, tb in zip(pa[key] if isinstance(pa[key], tuple) else (pa[key],),
                                      pb[key] if isinstance(pb[key], tuple) else (pb[key],)):
                        ta.copy_(tb)
    del a, b, g
    torch.cuda.empty_cache()


@pytest.mark.parametrize("H,V,R,lower_bound", [(16, 128, 128, None), (3, 64, 64, None), (5, 128, 32, -5.0),
                                                (2, 256, 128, None), (1, 512, 256, None), (4, 144, 160, None),
                                                (2, 16, 16, None), (1, 496, 32, -2.0)])
def test_kda_decode_step_equals_the_five_call_chain(H, V, R, lower_bound):
    """kda_decode_step (one kernel) against short_conv -> small_linear(f) -> fused_recurrent_kda ->
    small_linear(g) -> rms_norm_gated on identical copies of the layer state, three tokens in a row: the conv caches
    bit for bit, the KDA state and the normed output within tolerance (the f / g dots round in another order).
    V above 128 takes several passes of 128 value columns and 128 g rows (144: a partial second pass; 512: four;
    496: a partial last block), R above 128 a second LoRA piece (160: a partial one); V = 16 leaves most of a
    wave's columns past V, R = 16 one lane of each pair without a piece."""
    from fastlinear import small_linear
    K, Wd = 128, 4
    C = 2 * H * K + H * V
    s = 300 + H + R
    conv_w = W.normal((C, 1, Wd), 0.5, s, DEV)
    f_b = W.normal((H * K, R), 0.02 * 8, s + 1, DEV)
    g_b = W.normal((H * V, R), 0.02 * 8, s + 2, DEV)
    A_log = W.normal((H,), 0.5, s + 3, DEV, dtype=torch.float32)
    dt = W.normal((H * K,), 0.5, s + 4, DEV, dtype=torch.float32)
    o_norm = W.normal((V,), 0.02, s + 5, DEV, mean=1.0)
    st_a = W.normal((1, H, K, V), 0.1, s + 6, DEV, dtype=torch.float32)
    cache_a = W.normal((1, C, Wd), 1.0, s + 7, DEV)
    st_b, cache_b = st_a.clone(), cache_a.clone()
    for t in range(3):
        print(f"[kda_step] H={H} V={V} R={R} token {t}", flush=True)
        pr = W.normal((1, C + 2 * R + H), 1.0, s + 10 + t, DEV)
        got = TA.kda_decode_step(pr, conv_w, cache_a, f_b, g_b, A_log, dt, st_a, o_norm, heads=H,
                                 lower_bound=lower_bound)
        qkv = TA.short_conv(pr[:, :C], cache_b, conv_w)
        f = small_linear(pr[:, C:C + R], f_b)
        gg = small_linear(pr[:, C + R:C + 2 * R], g_b)
        b = pr[:, C + 2 * R:]
        o, _ = TA.fused_recurrent_kda(qkv[:, :H * K].reshape(1, 1, H, K), qkv[:, H * K:2 * H * K].reshape(1, 1, H, K),
                                      qkv[:, 2 * H * K:].reshape(1, 1, H, V), f.reshape(1, 1, H, K), b.reshape(1, 1, H),
                                      A_log=A_log, dt_bias=dt, initial_state=st_b, inplace=True,
                                      use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True, beta_is_logits=True,
                                      lower_bound=lower_bound)
        want = TA.rms_norm_gated(o.reshape(H, V), gg.reshape(H, V), o_norm, 1e-5)
        torch.cuda.synchronize()
        assert torch.equal(cache_a, cache_b), t
        close(got, want)
        torch.testing.assert_close(st_a.cpu(), st_b.cpu(), rtol=2e-2, atol=2e-3)


def test_kda_decode_step_rejects_bad_shapes():
    K = 128
    st = torch.zeros(1, 2, K, 64, device=DEV)
    C = 2 * 2 * K + 2 * 64
    pr = torch.zeros(1, C + 2 * 32 + 2, device=DEV, dtype=BF)
    conv_w = torch.zeros(C, 1, 4, device=DEV, dtype=BF)
    cache = torch.zeros(1, C, 4, device=DEV, dtype=BF)
    f_b = torch.zeros(2 * K, 32, device=DEV, dtype=BF)
    g_b = torch.zeros(2 * 64, 32, device=DEV, dtype=BF)
    a = torch.zeros(2, device=DEV)
    dt = torch.zeros(2 * K, device=DEV)
    on = torch.ones(64, device=DEV, dtype=BF)
    with pytest.raises((ValueError, RuntimeError)):
        TA.kda_decode_step(pr[:, :-1], conv_w, cache, f_b, g_b, a, dt, st, on, heads=2)  # row one element short
    with pytest.raises((ValueError, RuntimeError)):
        TA.kda_decode_step(pr, conv_w, cache, f_b, g_b, a, dt, torch.zeros(1, 2, 64, 64, device=DEV), on, heads=2)


def test_kda_decode_step_takes_the_three_caches_of_the_reference_layout():
    """The q, k and v conv weights and caches as three separate tensors (the model's conv1d modules and
    _KDAState's tuple, engine.py:645-647) give exactly what one combined tensor gives."""
    H, K, V, R = 4, 128, 128, 128
    C = 2 * H * K + H * V
    w_all = W.normal((C, 1, 4), 0.5, 410, DEV)
    c_all = W.normal((1, C, 4), 1.0, 411, DEV)
    f_b, g_b = W.normal((H * K, R), 0.1, 412, DEV), W.normal((H * V, R), 0.1, 413, DEV)
    A_log = W.normal((H,), 0.5, 414, DEV, dtype=torch.float32)
    dt = W.normal((H * K,), 0.5, 415, DEV, dtype=torch.float32)
    o_norm = W.normal((V,), 0.02, 416, DEV, mean=1.0)
    st1 = W.normal((1, H, K, V), 0.1, 417, DEV, dtype=torch.float32)
    st2 = st1.clone()
    sizes = (H * K, H * K, H * V)
    ws = tuple(t.clone() for t in torch.split(w_all, sizes, dim=0))
    cs = tuple(t.clone() for t in torch.split(c_all, sizes, dim=1))
    for t in range(2):
        pr = W.normal((1, C + 2 * R + H), 1.0, 420 + t, DEV)
        a = TA.kda_decode_step(pr, w_all, c_all, f_b, g_b, A_log, dt, st1, o_norm, heads=H)
        b = TA.kda_decode_step(pr, ws, cs, f_b, g_b, A_log, dt, st2, o_norm, heads=H)
        torch.cuda.synchronize()
        assert torch.equal(a, b) and torch.equal(st1, st2), t
        assert torch.equal(c_all, torch.cat(cs, dim=1)), t


# ------------------------------------------------------------------------ the two ends of a decode step

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_argmax_rows_matches_torch_argmax(dtype):
    """argmax_rows against torch.argmax on the CPU (the reference's logits.argmax(-1)): random rows of lengths that
    take the vector and the scalar paths (the LM head's 126464 among them), planted ties (the first index wins),
    NaN (above every number, the first one wins), rows of -inf, all-equal rows and a row offset by one element."""
    print(f"[argmax] {dtype}", flush=True)
    g = torch.Generator().manual_seed(11)
    for n in (1, 7, 8, 64, 1000, 1003, 126464):
        x = torch.randn(5, n, generator=g).to(dtype)
        if n > 1:
            x[1, n // 3] = x[1, n - 1] = x[1].max() + 1  # a tie: the first wins
            x[2, n // 2] = float("nan")
            x[2, n - 1] = float("nan")
        x[3] = float("-inf")
        x[4] = 0.5
        got = TA.argmax_rows(x.to(DEV)).cpu()
        assert torch.equal(got, x.argmax(-1)), (n, got, x.argmax(-1))
        ws = TA.argmax_workspace(5, n, dtype, DEV)  # the split form (one workgroup below 2 x 512 pieces)
        got = TA.argmax_rows(x.to(DEV), workspace=ws).cpu()
        assert torch.equal(got, x.argmax(-1)), (n, got, x.argmax(-1))
        if n > 8:  # rows not 16-byte aligned: the scalar path
            xv = x.to(DEV)[:, 1:]
            assert torch.equal(TA.argmax_rows(xv).cpu(), x[:, 1:].argmax(-1)), n
    tok = torch.zeros(1, 1, dtype=torch.long, device=DEV)
    x = torch.randn(1, 126464, generator=g).to(dtype)
    TA.argmax_rows(x.to(DEV), out=tok)
    assert int(tok) == int(x.argmax())
    # the split form: the maximum planted in each workgroup's range in turn and at both ends, ties across ranges
    ws = TA.argmax_workspace(1, 126464, dtype, DEV)
    for pos in (0, 4095, 4096, 4097, 60000, 126463):
        y = x.clone()
        y[0, pos] = 100.0
        y[0, (pos + 70001) % 126464] = 100.0  # a tie: the lower index wins
        TA.argmax_rows(y.to(DEV), out=tok, workspace=ws)
        assert int(tok) == int(y.argmax()), pos


@pytest.mark.parametrize("dtype,id_dtype", [(torch.bfloat16, torch.int64), (torch.float32, torch.int32)])
def test_embed_rows_matches_index_select(dtype, id_dtype):
    """embed_rows against index_select (word_embeddings of engine.py:686), bit for bit, with an id outside the
    table giving a row of zeros."""
    print(f"[embed] {dtype} {id_dtype}", flush=True)
    g = torch.Generator().manual_seed(12)
    V, H = 1000, 2048
    table = torch.randn(V, H, generator=g).to(dtype)
    ids = torch.tensor([[3], [999], [0], [3]], dtype=id_dtype)
    got = TA.embed_rows(table.to(DEV), ids.to(DEV)).cpu()
    assert got.shape == (4, 1, H) and torch.equal(got, table[ids.long()])
    bad = TA.embed_rows(table.to(DEV), torch.tensor([V, -1], dtype=id_dtype, device=DEV)).cpu()
    assert torch.equal(bad, torch.zeros(2, H, dtype=dtype))
    with pytest.raises(ValueError, match="int64 or int32"):
        TA.embed_rows(table.to(DEV), torch.zeros(1, device=DEV))


def test_fast_thinker_step_from_engine_objects_sigmoid_router_and_int8():
    """thinker_step.FastThinkerStep built from engine-shaped objects (model.model.layers[i].attention / .mlp / norms,
    _KDAState- and _MLAState-like caches, tok_buf, pos_buf) with the thinker's own router (sigmoid + expert bias, 8
    groups, top 4 groups, scale 2.5) and int8 experts (q_gu / q_d / s_gu / s_d, as engine._quantize_moe_int8 leaves a
    block) on one layer: each layer's MoE half equals rms_norm -> moe_route -> fused_moe_decode(residual) on the
    layer's own input bit for bit, and the step writes the argmax back and advances the position."""
    import fused_moe
    import fused_ops
    import thinker_step
    print("[thinker_step] engine objects, sigmoid router, int8 layer", flush=True)
    h = W.HybridThinkerStep(4, DEV, pos=50, seed=7300)
    E = W.EXPERTS
    for li, layer in enumerate(h.model.model.layers):
        g = layer.mlp.gate
        g.expert_bias = W.normal((E,), 0.05, 7400 + li, DEV, dtype=torch.float32)
        g.n_group, g.topk_group, g.routed_scaling_factor = 8, 4, 2.5
    int8_layer = h.model.model.layers[1]
    q_gu, s_gu = fused_moe.quantize_rows_int8(int8_layer.mlp.w_gu, scale_dtype=torch.float32)
    q_d, s_d = fused_moe.quantize_rows_int8(int8_layer.mlp.w_d, scale_dtype=torch.float32)
    int8_layer.mlp.w_gu = int8_layer.mlp.w_d = None
    int8_layer.mlp.q_gu, int8_layer.mlp.q_d, int8_layer.mlp.s_gu, int8_layer.mlp.s_d = q_gu, q_d, s_gu, s_d
    step = thinker_step.FastThinkerStep(h.model, h.cache_layers, h.tok, h.pos, scoring="sigmoid")
    trace, out, logits = step.trace()
    assert int(h.pos) == 51 and int(h.tok) == int(logits.float().cpu().argmax())
    for li, (layer, (h_in, hm, ids, wts)) in enumerate(zip(h.model.model.layers, trace)):
        mlp, g = layer.mlp, layer.mlp.gate
        xn = fused_ops.rms_norm(hm, layer.post_attention_layernorm.weight, W.EPS)
        lg = torch.empty(1, E, device=DEV)
        i2 = torch.empty(1, W.TOP_K + 1, device=DEV, dtype=torch.long)
        w2 = torch.empty(1, W.TOP_K + 1, device=DEV)
        fused_ops.moe_route(xn, g.w32, g.expert_bias, 8, 4, W.TOP_K, 2.5, lg, i2, w2)
        if mlp.w_gu is not None:
            y = fused_moe.fused_moe_decode(xn, mlp.w_gu, mlp.w_d, i2, w2, residual=hm)
        else:
            y = fused_moe.fused_moe_decode(xn, mlp.q_gu, mlp.q_d, i2, w2, s_gu=mlp.s_gu, s_d=mlp.s_d, residual=hm)
        assert torch.equal(ids, i2) and torch.equal(wts, w2), li
        nxt = trace[li + 1][0] if li + 1 < len(trace) else out
        assert torch.equal(nxt, y), li


def test_fast_thinker_prefill_from_engine_objects_sigmoid_router_and_int8():
    """FastThinkerStep.prefill on engine-shaped objects with the thinker's own router (sigmoid + expert bias, 8
    groups, top 4 groups, scale 2.5) and int8 experts on one layer, a 40-token prompt: each layer's MoE half equals
    rms_norm -> route -> fused_moe_prefill(residual) on the layer's own input bit for bit (ids, weights, outputs),
    and the prefill writes the last row's argmax back and advances the position by 40."""
    import fused_moe
    import fused_ops
    import thinker_step
    print("[thinker_step] prefill, engine objects, sigmoid router, int8 layer", flush=True)
    T = 40
    h = W.HybridThinkerStep(4, DEV, pos=50, seed=7600)
    E = W.EXPERTS
    for li, layer in enumerate(h.model.model.layers):
        g = layer.mlp.gate
        g.expert_bias = W.normal((E,), 0.05, 7700 + li, DEV, dtype=torch.float32)
        g.n_group, g.topk_group, g.routed_scaling_factor = 8, 4, 2.5
    int8_layer = h.model.model.layers[2]
    q_gu, s_gu = fused_moe.quantize_rows_int8(int8_layer.mlp.w_gu, scale_dtype=torch.float32)
    q_d, s_d = fused_moe.quantize_rows_int8(int8_layer.mlp.w_d, scale_dtype=torch.float32)
    int8_layer.mlp.w_gu = int8_layer.mlp.w_d = None
    int8_layer.mlp.q_gu, int8_layer.mlp.q_d, int8_layer.mlp.s_gu, int8_layer.mlp.s_d = q_gu, q_d, s_gu, s_d
    step = thinker_step.FastThinkerStep(h.model, h.cache_layers, h.tok, h.pos, scoring="sigmoid")
    ids = torch.randint(0, h.embed.shape[0], (T,), generator=torch.Generator().manual_seed(21)).to(DEV)
    logits, trace = step.prefill(ids, trace=True)
    assert int(h.pos) == 50 + T and int(h.tok) == int(logits.float().cpu().argmax())
    for li, (layer, (h_in, hm, rid, rw)) in enumerate(zip(h.model.model.layers, trace)):
        mlp, g = layer.mlp, layer.mlp.gate
        xn = fused_ops.rms_norm(hm, layer.post_attention_layernorm.weight, W.EPS)
        i2, w2, _ = fused_ops.route(xn, g.w32, g.expert_bias, top_k=W.TOP_K, scoring="sigmoid", n_group=8,
                                    topk_group=4, scale=2.5)
        assert torch.equal(rid, i2.long()) and torch.equal(rw, w2), li
        if mlp.w_gu is not None:
            y = fused_moe.fused_moe_prefill(xn, mlp.w_gu, mlp.w_d, i2, w2, residual=hm)
        else:
            y = fused_moe.fused_moe_prefill(xn, mlp.q_gu, mlp.q_d, i2, w2, s_gu=mlp.s_gu, s_d=mlp.s_d, residual=hm)
        if li + 1 < len(trace):
            assert torch.equal(trace[li + 1][0], y), li
    del h, step
    torch.cuda.empty_cache()
