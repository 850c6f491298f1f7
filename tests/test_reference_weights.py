"""Weights taken from a loaded reference model: ``TalkerWeights.from_reference_model`` and
``CodePredictorWeights.from_reference_model`` read the attribute paths of the reference's modules
(model/components.py:29-200, model/layers.py:103-294: ``model.layers[i].self_attn.qkv_proj.weight``,
``mlp.gate_up_proj.weight``, ...) and the reference's config fields (model/config.py:66-118).

The stand-in modules below hold the tensors of a random-init weight object at those paths; the
adapter must give back an object whose every tensor (FP8 codes, scales, interleaved rows and the
derived projection tables included) equals the original's, and whose config equals the original's.
A transposed weight, a swapped norm or a wrong config field fails."""

from __future__ import annotations

from dataclasses import asdict
from types import SimpleNamespace

import pytest
import torch


def _norm(w, eps):
    return SimpleNamespace(weight=torch.nn.Parameter(w.clone(), requires_grad=False), variance_epsilon=eps)


def _lin(w, b=None):
    return SimpleNamespace(weight=torch.nn.Parameter(w.clone(), requires_grad=False),
                           bias=None if b is None else torch.nn.Parameter(b.clone(), requires_grad=False))


def _layer(L, eps, q_norm, k_norm, rope_theta):
    return SimpleNamespace(
        input_layernorm=_norm(L.input_norm, eps),
        self_attn=SimpleNamespace(qkv_proj=_lin(L.qkv), o_proj=_lin(L.o), q_norm=_norm(q_norm, eps),
                                  k_norm=_norm(k_norm, eps), rope_theta=rope_theta),
        post_attention_layernorm=_norm(L.post_norm, eps),
        mlp=SimpleNamespace(gate_up_proj=_lin(L.gate_up), down_proj=_lin(L.down)),
    )


def _talker_module(W):
    c = W.config
    layers = [_layer(L, c.rms_eps, L.attention.q_norm.weight, L.attention.k_norm.weight, c.rope_theta)
              for L in W.layers]
    inner = SimpleNamespace(layers=layers, norm=_norm(W.final_norm, c.rms_eps),
                            codec_embedding=_lin(W.codec_embedding))
    return SimpleNamespace(model=inner, codec_head=_lin(W.codec_head),
                           get_projected_text_embedding_cache=lambda: W.text_embedding)


def _reference_config(tc, cc=None):
    cp = SimpleNamespace(hidden_size=0, intermediate_size=0, num_hidden_layers=0, num_attention_heads=0,
                         num_key_value_heads=0, head_dim=0, vocab_size=tc.codec_vocab, rms_norm_eps=0.0,
                         rope_theta=0.0)
    if cc is not None:
        cp = SimpleNamespace(hidden_size=cc.hidden, intermediate_size=cc.intermediate, num_hidden_layers=cc.num_layers,
                             num_attention_heads=cc.num_qo_heads, num_key_value_heads=cc.num_kv_heads,
                             head_dim=cc.head_dim, vocab_size=cc.vocab, rms_norm_eps=cc.rms_eps,
                             rope_theta=cc.rope_theta)
    talker = SimpleNamespace(num_hidden_layers=tc.num_layers, hidden_size=tc.hidden, num_attention_heads=tc.num_qo_heads,
                             num_key_value_heads=tc.num_kv_heads, head_dim=tc.head_dim, intermediate_size=tc.intermediate,
                             vocab_size=tc.vocab, text_vocab_size=tc.text_vocab, codec_eos_token_id=tc.eos_id,
                             rms_norm_eps=tc.rms_eps, rope_theta=tc.rope_theta,
                             num_code_groups=cc.num_code_groups if cc is not None else 16, code_predictor=cp)
    return SimpleNamespace(talker=talker)


def _talker_config():
    from nari_qwen3_tts_amd.talker import TalkerConfig

    return TalkerConfig(num_layers=2, hidden=256, num_qo_heads=2, num_kv_heads=1, head_dim=128, intermediate=384,
                        vocab=512, text_vocab=300, codec_vocab=448, eos_id=450, rms_eps=1e-5, rope_theta=5e5)


def _same_talker(a, b):
    assert asdict(a.config) == asdict(b.config)
    for x, y in zip(a.layers, b.layers):
        for name in ("input_norm", "qkv", "o", "post_norm", "gate_up", "down", "gate_up_q", "gate_up_scales",
                     "gate_up_packed"):
            u, v = getattr(x, name), getattr(y, name)
            assert (u is None) == (v is None), name
            if u is not None:
                assert u.dtype == v.dtype and torch.equal(u.view(torch.uint8), v.view(torch.uint8)), name
        for n in ("q_norm", "k_norm"):
            assert torch.equal(getattr(x.attention, n).weight, getattr(y.attention, n).weight)
            assert getattr(x.attention, n).variance_epsilon == getattr(y.attention, n).variance_epsilon
        assert x.attention.rope_theta == y.attention.rope_theta
    for name in ("final_norm", "codec_head", "text_embedding", "codec_embedding"):
        assert torch.equal(getattr(a, name), getattr(b, name)), name
    assert a.fp8_gate_up == b.fp8_gate_up


def test_talker_weights_from_reference_model_bf16(nq):
    from nari_qwen3_tts_amd.talker import TalkerWeights

    cfg = _talker_config()
    W = TalkerWeights(cfg, torch.device("cpu"), seed=3, fp8_gate_up=False)
    got = TalkerWeights.from_reference_model(_talker_module(W), _reference_config(cfg), fp8_gate_up=False)
    _same_talker(W, got)


def test_talker_weights_reject_a_transposed_projection(nq):
    from nari_qwen3_tts_amd.talker import TalkerWeights

    cfg = _talker_config()
    W = TalkerWeights(cfg, torch.device("cpu"), seed=4, fp8_gate_up=False)
    module = _talker_module(W)
    module.model.layers[1].mlp.down_proj.weight = torch.nn.Parameter(W.layers[1].down.t().contiguous())
    with pytest.raises(ValueError, match="shape"):
        TalkerWeights.from_reference_model(module, _reference_config(cfg), fp8_gate_up=False)


@pytest.mark.gpu
def test_fp8_talker_and_code_predictor_weights_from_reference_model(nq, device):
    from nari_qwen3_tts_amd.code_predictor import CodePredictorConfig, CodePredictorWeights
    from nari_qwen3_tts_amd.talker import TalkerWeights

    cfg = _talker_config()
    W = TalkerWeights(cfg, device, seed=5, fp8_gate_up=True)
    got = TalkerWeights.from_reference_model(_talker_module(W), _reference_config(cfg), fp8_gate_up=True)
    _same_talker(W, got)

    cc = CodePredictorConfig(num_layers=2, hidden=256, num_qo_heads=4, num_kv_heads=2, head_dim=64, intermediate=384,
                             vocab=128, talker_hidden=cfg.hidden, talker_vocab=cfg.vocab, num_code_groups=5,
                             rms_eps=1e-5, rope_theta=5e5)
    C = CodePredictorWeights(cc, device, seed=6)
    layers = [_layer(L, cc.rms_eps, L.q_norm, L.k_norm, cc.rope_theta) for L in C.layers]
    model = SimpleNamespace(
        model=SimpleNamespace(layers=layers, norm=_norm(C.final_norm, cc.rms_eps),
                              codec_embedding=[_lin(e) for e in C.codec_embedding]),
        lm_head=[_lin(h) for h in C.lm_head],
        small_to_mtp_projection=_lin(C.proj_w, C.proj_b),
    )
    got_c = CodePredictorWeights.from_reference_model(model, _lin(C.layer0_embedding), _reference_config(cfg, cc))
    assert asdict(got_c.config) == asdict(C.config)
    for x, y in zip(C.layers, got_c.layers):
        for name in ("input_norm", "qkv", "o", "post_norm", "gate_up", "down", "q_norm", "k_norm", "gate_up_packed"):
            assert torch.equal(getattr(x, name), getattr(y, name)), name
    for name in ("final_norm", "lm_head", "proj_w", "proj_b", "layer0_embedding", "codec_embedding",
                 "projected_layer0", "projected_residual"):
        assert torch.equal(getattr(C, name), getattr(got_c, name)), name
