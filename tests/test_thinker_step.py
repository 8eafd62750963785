"""CPU checks of thinker_step.FastThinkerStep's set-up: how it reads the engine's objects (attribute paths, fused
projections, router parameters, int8 stacks) and which layer forms it refuses. No kernel runs here."""
from types import SimpleNamespace as NS

import pytest
import torch

import thinker_step

H, KD, R, NH = 64, 32, 16, 2


def _lin(rows, cols=H, seed=0):
    return NS(weight=torch.randn(rows, cols, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16),
              bias=None)


def _norm(n=H):
    return NS(weight=torch.ones(n, dtype=torch.bfloat16), variance_epsilon=1e-6)


def _kda(seed):
    conv = lambda s: NS(weight=torch.zeros(KD, 1, 4, dtype=torch.bfloat16), bias=None, hidden_size=KD,  # noqa: E731
                        kernel_size=(4,))
    return NS(mode="fused_recurrent", q_proj=_lin(KD, seed=seed), k_proj=_lin(KD, seed=seed + 1),
              v_proj=_lin(KD, seed=seed + 2), f_a_proj=_lin(R, seed=seed + 3), g_a_proj=_lin(R, seed=seed + 4),
              b_proj=_lin(NH, seed=seed + 5), f_b_proj=_lin(KD, R), g_b_proj=_lin(KD, R), q_conv1d=conv(0),
              k_conv1d=conv(1), v_conv1d=conv(2), o_norm=NS(weight=torch.ones(KD // NH), eps=1e-5),
              o_proj=_lin(H, KD), A_log=torch.zeros(NH), dt_bias=torch.zeros(KD), lower_bound=-5.0, num_heads=NH,
              head_k_dim=KD // NH, head_dim=KD // NH, no_kda_lora=False)


def _mla():
    return NS(q_proj=_lin(NH * 24), k_proj=_lin(NH * 24), v_proj=_lin(NH * 16), o_proj=_lin(H, NH * 16), num_heads=NH,
              qk_head_dim=24, v_head_dim=16)


def _moe(int8=False, E=8, I=32):
    gate = NS(w32=torch.zeros(E, H), expert_bias=torch.arange(E, dtype=torch.bfloat16), top_k=2, n_group=2,
              topk_group=1, routed_scaling_factor=2.5)
    if int8:
        return NS(gate=gate, w_gu=None, w_d=None, q_gu=torch.zeros(E + 1, 2 * I, H, dtype=torch.int8),
                  q_d=torch.zeros(E + 1, H, I, dtype=torch.int8), s_gu=torch.ones(E + 1, 2 * I),
                  s_d=torch.ones(E + 1, H))
    return NS(gate=gate, w_gu=torch.zeros(E + 1, 2 * I, H, dtype=torch.bfloat16),
              w_d=torch.zeros(E + 1, H, I, dtype=torch.bfloat16))


def _model(layers):
    return NS(model=NS(word_embeddings=NS(weight=torch.zeros(100, H, dtype=torch.bfloat16)), layers=layers,
                       norm=_norm()), lm_head=_lin(100))


def _layer(attn, kind, mlp):
    return NS(attention=attn, attention_layer_type=kind, input_layernorm=_norm(), post_attention_layernorm=_norm(),
              mlp=mlp)


def _caches():
    kda = NS(keys=torch.zeros(1, NH, KD // NH, KD // NH), values=tuple(torch.zeros(1, KD, 4) for _ in range(3)))
    mla = NS(k=torch.zeros(1, NH, 10, 24), v=torch.zeros(1, NH, 10, 16))
    return kda, mla


def _bufs():
    return torch.zeros(1, 1, dtype=torch.long), torch.zeros(1, dtype=torch.long)


def test_reads_the_engine_objects():
    kda_c, mla_c = _caches()
    a = _kda(10)
    model = _model([_layer(a, "kda", _moe()), _layer(_mla(), "attention", _moe(int8=True))])
    st = thinker_step.FastThinkerStep(model, [kda_c, mla_c], *_bufs())
    p0, p1 = st.L
    assert p0["kind"] == "kda" and p1["kind"] == "mla"
    want = torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight, a.f_a_proj.weight, a.g_a_proj.weight,
                      a.b_proj.weight])
    assert torch.equal(p0["proj"], want) and p0["proj_b"] is None and p0["rank"] == R
    assert p0["state"] is kda_c.keys and p0["conv"] == kda_c.values and p0["lower_bound"] == -5.0
    assert p0["heads"] == NH and p0["K"] == KD // NH and p0["o_norm"][1] == 1e-5
    assert p1["kc"] is mla_c.k and p1["qkv"].shape == (NH * 64, H)
    b0, b1 = p0["blk"], p1["blk"]
    assert b0["w_gu"] is model.model.layers[0].mlp.w_gu and b0["s_gu"] is None
    assert b1["w_gu"] is model.model.layers[1].mlp.q_gu and b1["s_d"] is model.model.layers[1].mlp.s_d
    assert b0["top_k"] == 2 and b0["n_group"] == 2 and b0["topk_group"] == 1 and b0["scale"] == 2.5
    assert b0["bias"].dtype == torch.float32 and b0["eps"] == 1e-6
    assert st.logits.shape == (1, 8) and st.ids.shape == (1, 3) and st.a_buf.shape == (3, 32)


def test_projection_biases_are_fused():
    kda_c, _ = _caches()
    a = _kda(20)
    a.k_proj.bias = torch.ones(KD, dtype=torch.bfloat16)
    st = thinker_step.FastThinkerStep(_model([_layer(a, "kda", _moe())]), [kda_c], *_bufs())
    b = st.L[0]["proj_b"]
    assert b.shape == (3 * KD + 2 * R + NH,) and float(b[KD:2 * KD].sum()) == KD and float(b.sum()) == KD


def test_refuses_what_it_cannot_run():
    kda_c, mla_c = _caches()
    bare = _mla()
    del bare.q_proj
    with pytest.raises(ValueError, match="mla_qkv"):
        thinker_step.FastThinkerStep(_model([_layer(bare, "attention", _moe())]), [mla_c], *_bufs())
    st = thinker_step.FastThinkerStep(_model([_layer(bare, "attention", _moe())]), [mla_c], *_bufs(),
                                      mla_qkv=lambda li, p, h: None)
    assert "qkv" not in st.L[0]
    a = _kda(30)
    a.no_kda_lora = True
    with pytest.raises(ValueError, match="no_kda_lora"):
        thinker_step.FastThinkerStep(_model([_layer(a, "kda", _moe())]), [kda_c], *_bufs())
    a = _kda(31)
    a.q_conv1d.bias = torch.zeros(KD)
    with pytest.raises(ValueError, match="bias"):
        thinker_step.FastThinkerStep(_model([_layer(a, "kda", _moe())]), [kda_c], *_bufs())
    wrong = NS(k=torch.zeros(1, NH + 1, 10, 24), v=torch.zeros(1, NH + 1, 10, 16))
    with pytest.raises(ValueError, match="MLA cache"):
        thinker_step.FastThinkerStep(_model([_layer(_mla(), "attention", _moe())]), [wrong], *_bufs())
    no_experts = _moe()
    no_experts.w_gu = None
    with pytest.raises(ValueError, match="stacked experts"):
        thinker_step.FastThinkerStep(_model([_layer(_kda(32), "kda", no_experts)]), [kda_c], *_bufs())
    with pytest.raises(ValueError, match="scoring"):
        thinker_step.FastThinkerStep(_model([]), [], *_bufs(), scoring="relu")
    with pytest.raises(ValueError, match="cache layers"):
        thinker_step.FastThinkerStep(_model([_layer(_kda(33), "kda", _moe())]), [], *_bufs())


def test_prefill_refuses_bad_prompts():
    """The prompt checks of FastThinkerStep.prefill come before any kernel: ids or rows (one of them), their types,
    an empty prompt, and n_valid's form."""
    kda_c, _ = _caches()
    st = thinker_step.FastThinkerStep(_model([_layer(_kda(40), "kda", _moe())]), [kda_c], *_bufs())
    with pytest.raises(ValueError, match="ids or its input rows"):
        st.prefill()
    with pytest.raises(ValueError, match="ids or its input rows"):
        st.prefill(torch.zeros(3, dtype=torch.long), h=torch.zeros(3, H, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="h must be"):
        st.prefill(h=torch.zeros(3, H, dtype=torch.float32))
    with pytest.raises(ValueError, match="ids must be"):
        st.prefill(torch.zeros(3, dtype=torch.float32))
    with pytest.raises(ValueError, match="empty prompt"):
        st.prefill(h=torch.zeros(0, H, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="n_valid"):
        st.prefill(h=torch.zeros(4, H, dtype=torch.bfloat16), n_valid=torch.tensor([2], dtype=torch.int32))
    with pytest.raises(ValueError, match="n_valid"):
        st.prefill(h=torch.zeros(4, H, dtype=torch.bfloat16), n_valid=torch.tensor([1, 2]))
