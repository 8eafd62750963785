"""Pins of the thinker-attention oracle (oracle/thinker_attn_oracle.py) by what the mathematics fixes: closed forms,
the Householder matrix form of the KDA recurrence, step composition, torch library routines, planted mistakes.
Its equivalence to fla's own kernels (fla-core 0.5.2, absent) stays parity unpinned."""
import math

import torch
import torch.nn.functional as F

from oracle import thinker_attn_oracle as A

F64 = torch.float64


def _rand(*shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=F64) * scale


def _kda_inputs(T=5, H=3, K=8, V=6, seed=0):
    q, k, v = _rand(T, H, K, seed=seed), _rand(T, H, K, seed=seed + 1), _rand(T, H, V, seed=seed + 2)
    g = _rand(T, H, K, seed=seed + 3)
    beta = torch.sigmoid(_rand(T, H, seed=seed + 4))
    A_log = _rand(H, seed=seed + 5, scale=0.5)
    dt = _rand(H * K, seed=seed + 6, scale=0.5)
    S0 = _rand(H, K, V, seed=seed + 7, scale=0.3)
    return q, k, v, g, beta, A_log, dt, S0


def test_one_step_from_zero_state_is_beta_k_v():
    """From S = 0 the decay has nothing to act on: S1 = beta k^ v^T and o = beta (q^ . k^) scale v, k^ = l2norm(k)."""
    q, k, v, g, beta, A_log, dt, _ = _kda_inputs(T=1)
    o, S = A.kda_recurrent(q, k, v, g, beta, None, A_log=A_log, dt_bias=dt)
    kh, qh = A.l2norm(k[0]), A.l2norm(q[0])
    want_S = beta[0][:, None, None] * kh[:, :, None] * v[0][:, None, :]
    torch.testing.assert_close(S, want_S, rtol=1e-12, atol=1e-12)
    want_o = beta[0][:, None] * (qh * kh).sum(-1, keepdim=True) * 8 ** -0.5 * v[0]
    torch.testing.assert_close(o[0], want_o, rtol=1e-12, atol=1e-12)


def test_zero_write_strength_and_unit_decay_leave_the_state():
    """beta = 0 and a gate input of -1e30 (softplus 0, decay exp(0) = 1; the padded-prompt trick of engine.py:252-253):
    the state is unchanged and o = scale * S^T q^."""
    q, k, v, g, beta, A_log, dt, S0 = _kda_inputs(T=3)
    g = torch.full_like(g, -1e30)
    o, S = A.kda_recurrent(q, k, v, g, torch.zeros_like(beta), S0, A_log=A_log, dt_bias=dt)
    torch.testing.assert_close(S, S0, rtol=0, atol=0)
    want = torch.einsum("thk,hkv->thv", A.l2norm(q), S0) * 8 ** -0.5
    torch.testing.assert_close(o, want, rtol=1e-12, atol=1e-12)


def test_householder_form_of_the_recurrence():
    """The same recurrence as matrices: S_t = (I - beta_t k_t k_t^T) diag(alpha_t) S_{t-1} + beta_t k_t v_t^T,
    o_t = S_t^T q_t, alpha_t = exp(gate). Catches a decay applied after the update or a transposed state."""
    q, k, v, g, beta, A_log, dt, S0 = _kda_inputs(T=6, H=2, K=5, V=4, seed=10)
    o, S = A.kda_recurrent(q, k, v, g, beta, S0, A_log=A_log, dt_bias=dt, scale=0.7)
    alpha = torch.exp(A.kda_gate(g, A_log, dt))
    qh, kh = A.l2norm(q) * 0.7, A.l2norm(k)
    for h in range(2):
        Sm = S0[h].clone()
        for t in range(6):
            kk = kh[t, h][:, None]
            Sm = (torch.eye(5, dtype=F64) - beta[t, h] * kk @ kk.T) @ torch.diag(alpha[t, h]) @ Sm \
                + beta[t, h] * kk @ v[t, h][None, :]
            torch.testing.assert_close(o[t, h], Sm.T @ qh[t, h], rtol=1e-10, atol=1e-10)
        torch.testing.assert_close(S[h], Sm, rtol=1e-10, atol=1e-10)


def test_planted_decay_after_update_is_caught():
    """A restatement that decays after the delta update disagrees with the one-step closed form."""
    q, k, v, g, beta, A_log, dt, _ = _kda_inputs(T=1, seed=20)
    alpha = torch.exp(A.kda_gate(g, A_log, dt))[0]
    kh = A.l2norm(k[0])
    wrong = alpha[:, :, None] * (beta[0][:, None, None] * kh[:, :, None] * v[0][:, None, :])
    _, S = A.kda_recurrent(q, k, v, g, beta, None, A_log=A_log, dt_bias=dt)
    assert not torch.allclose(S, wrong, rtol=1e-3, atol=1e-6)


def test_t_steps_equal_t_single_steps():
    q, k, v, g, beta, A_log, dt, S0 = _kda_inputs(T=7, seed=30)
    o, S = A.kda_recurrent(q, k, v, g, beta, S0, A_log=A_log, dt_bias=dt)
    Si, outs = S0, []
    for t in range(7):
        ot, Si = A.kda_recurrent(q[t:t + 1], k[t:t + 1], v[t:t + 1], g[t:t + 1], beta[t:t + 1], Si, A_log=A_log,
                                 dt_bias=dt)
        outs.append(ot)
    torch.testing.assert_close(torch.cat(outs), o, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(Si, S, rtol=1e-12, atol=1e-12)


def test_gate_closed_forms():
    """exp(-softplus(x)) = 1 / (1 + e^x): with A_log = 0 the decay is sigmoid(-(g + dt)); with a lower bound lb the
    log decay is lb * sigmoid(e^A (g + dt)); softplus keeps x itself above 20."""
    g = _rand(2, 3, 4, seed=40, scale=3.0)
    dt = _rand(12, seed=41)
    x = g + dt.reshape(3, 4)
    torch.testing.assert_close(torch.exp(A.kda_gate(g, torch.zeros(3, dtype=F64), dt)), torch.sigmoid(-x),
                               rtol=1e-12, atol=1e-14)
    Al = _rand(3, seed=42)
    torch.testing.assert_close(A.kda_gate(g, Al, dt, lower_bound=-5.0),
                               -5.0 * torch.sigmoid(torch.exp(Al)[:, None] * x), rtol=1e-12, atol=1e-14)
    big = torch.tensor([25.0, 100.0], dtype=F64)
    assert torch.equal(A.softplus(big), big)
    torch.testing.assert_close(A.softplus(torch.tensor([0.0], dtype=F64)), torch.tensor([math.log(2.0)], dtype=F64))


def test_l2norm_epsilon():
    x = torch.tensor([[3.0, 4.0]], dtype=F64)
    torch.testing.assert_close(A.l2norm(x), x / math.sqrt(25.0 + 1e-6))


def test_short_conv_equals_conv1d_over_the_window():
    """The step form over T tokens equals torch's depthwise F.conv1d over [cache | x] (causal, no padding), and the
    cache ends as the last W inputs."""
    C, W, T = 10, 4, 6
    x, cache = _rand(T, C, seed=50), _rand(C, W, seed=51)
    w, b = _rand(C, W, seed=52, scale=0.5), _rand(C, seed=53)
    y, cache2 = A.short_conv(x, cache, w, b)
    seq = torch.cat([cache, x.T], 1)[None]  # [1, C, W + T]
    ref = F.conv1d(seq, w[:, None, :], b, groups=C)[0, :, 1:].T  # outputs ending at each new token
    torch.testing.assert_close(y, F.silu(ref), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(cache2, seq[0, :, -W:], rtol=0, atol=0)


def test_rms_norm_gated_equals_library():
    x, g, w = _rand(5, 16, seed=60), _rand(5, 16, seed=61), _rand(16, seed=62)
    ref = F.rms_norm(x, (16,), w, 1e-5) * torch.sigmoid(g)
    torch.testing.assert_close(A.rms_norm_gated(x, g, w, 1e-5), ref, rtol=1e-12, atol=1e-12)


def test_mla_decode_attn_equals_sdpa_and_edge_cases():
    nh, L, dq, dv, pos = 3, 12, 16, 8, 7
    q, kn, vn = _rand(nh, dq, seed=70), _rand(nh, dq, seed=71), _rand(nh, dv, seed=72)
    kc, vc = _rand(nh, L, dq, seed=73), _rand(nh, L, dv, seed=74)
    out, kc2, vc2 = A.mla_decode_attn(q, kn, vn, kc, vc, pos)
    kr, vr = kc.clone(), vc.clone()
    kr[:, pos], vr[:, pos] = kn, vn
    ref = F.scaled_dot_product_attention(q[:, None, :], kr[:, : pos + 1], vr[:, : pos + 1])[:, 0]
    torch.testing.assert_close(out, ref, rtol=1e-12, atol=1e-12)
    assert torch.equal(kc2, kr) and torch.equal(vc2, vr)
    assert torch.equal(kc2[:, pos + 1:], kc[:, pos + 1:])
    out0, _, _ = A.mla_decode_attn(q, kn, vn, kc, vc, 0)  # one position: the new value itself
    torch.testing.assert_close(out0, vn, rtol=1e-12, atol=1e-12)


def _mla_prompt(T, pos, nh=3, L=24, dq=16, dv=8, seed=80):
    return (_rand(T, nh, dq, seed=seed), _rand(T, nh, dq, seed=seed + 1), _rand(T, nh, dv, seed=seed + 2),
            _rand(nh, L, dq, seed=seed + 3), _rand(nh, L, dv, seed=seed + 4))


def test_mla_prefill_attn_equals_token_by_token_decode_and_sdpa():
    T, pos = 6, 9
    q, kn, vn, kc, vc = _mla_prompt(T, pos)
    out, kc2, vc2 = A.mla_prefill_attn(q, kn, vn, kc, vc, pos)
    # the same prompt one token at a time through the decode form
    kd, vd = kc.clone(), vc.clone()
    for t in range(T):
        o, kd, vd = A.mla_decode_attn(q[t], kn[t], vn[t], kd, vd, pos + t)
        torch.testing.assert_close(out[t], o, rtol=1e-12, atol=1e-12)
    assert torch.equal(kc2, kd) and torch.equal(vc2, vd)
    # torch's attention with the causal mask over the updated caches
    n = pos + T
    mask = torch.arange(n)[None, :] <= (pos + torch.arange(T))[:, None]
    ref = F.scaled_dot_product_attention(q.transpose(0, 1), kc2[:, :n], vc2[:, :n], attn_mask=mask)
    torch.testing.assert_close(out, ref.transpose(0, 1), rtol=1e-12, atol=1e-12)
    assert torch.equal(kc2[:, n:], kc[:, n:]) and torch.equal(kc2[:, :pos], kc[:, :pos])


def test_mla_prefill_attn_edges():
    q, kn, vn, kc, vc = _mla_prompt(1, 5, seed=90)
    out, _, _ = A.mla_prefill_attn(q, kn, vn, kc, vc, 5)  # one token: the decode form
    ref, _, _ = A.mla_decode_attn(q[0], kn[0], vn[0], kc, vc, 5)
    torch.testing.assert_close(out[0], ref, rtol=1e-12, atol=1e-12)
    q, kn, vn, kc, vc = _mla_prompt(4, 0, L=4, seed=95)  # a fresh cache filled to the end: token 0 sees itself
    out, kc2, _ = A.mla_prefill_attn(q, kn, vn, kc, vc, 0)
    torch.testing.assert_close(out[0], vn[0], rtol=1e-12, atol=1e-12)
    assert torch.equal(kc2.transpose(0, 1), kn)


def test_planted_mask_off_by_one_is_caught():
    """A mask that hides the token's own key (keys < pos + t) changes every output row."""
    T, pos = 5, 3
    q, kn, vn, kc, vc = _mla_prompt(T, pos, seed=100)
    out, kc2, vc2 = A.mla_prefill_attn(q, kn, vn, kc, vc, pos)
    n = pos + T
    wrong = torch.arange(n)[None, :] < (pos + torch.arange(T))[:, None]
    bad = F.scaled_dot_product_attention(q.transpose(0, 1), kc2[:, :n], vc2[:, :n], attn_mask=wrong).transpose(0, 1)
    assert all((out[t] - bad[t]).abs().max() > 1e-3 for t in range(T))
