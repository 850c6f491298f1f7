"""The code-predictor oracle's per-pass teacher forcing (CPU): forcing a pass with the oracle's own
cache changes nothing, and a change of the forced cache at position p reaches exactly the passes
after p (pass g reads positions < g), which pins the forcing index."""

from __future__ import annotations

import numpy as np

from oracle import bf16 as o_bf16
from oracle import code_predictor as o_cp


def _weights(rng, layers=2, hidden=64, hq=4, hkv=2, d=16, inter=96, vocab=32, talker_hidden=48, talker_vocab=40,
             groups=5):
    def r(*shape, s=0.1):
        return o_bf16.round_f32((rng.standard_normal(shape) * s).astype(np.float32))

    lay = [dict(input_norm=np.ones(hidden, np.float32), qkv=r((hq + 2 * hkv) * d, hidden), o=r(hidden, hq * d),
                post_norm=np.ones(hidden, np.float32), gate_up=r(2 * inter, hidden), down=r(hidden, inter),
                q_norm=np.ones(d, np.float32), k_norm=np.ones(d, np.float32)) for _ in range(layers)]
    w = dict(layers=lay, final_norm=np.ones(hidden, np.float32), lm_head=r(groups - 1, vocab, hidden),
             proj_w=r(hidden, talker_hidden), proj_b=r(hidden), layer0_embedding=r(talker_vocab, talker_hidden, s=1.0),
             codec_embedding=r(groups - 1, vocab, talker_hidden, s=1.0))
    w["projected_layer0"] = o_bf16.round_f32(w["layer0_embedding"] @ w["proj_w"].T + w["proj_b"])
    w["projected_residual"] = o_bf16.round_f32(np.einsum("gvt,ht->gvh", w["codec_embedding"][:-1], w["proj_w"])
                                               + w["proj_b"])
    cfg = dict(num_qo_heads=hq, num_kv_heads=hkv, head_dim=d, rms_eps=1e-6, rope_theta=10000.0,
               num_code_groups=groups)
    return w, cfg


def test_forcing_with_the_own_cache_is_the_identity_and_reaches_later_passes_only():
    rng = np.random.default_rng(5)
    w, cfg = _weights(rng)
    rows, groups = 3, cfg["num_code_groups"]
    layer0 = rng.integers(0, 40, size=rows)
    past = o_bf16.round_f32(rng.standard_normal((rows, 48)).astype(np.float32))
    tokens = rng.integers(0, 32, size=(groups - 1, rows))
    logits, csum, cache = o_cp.whole_frame(w, cfg, layer0, past, tokens)
    forced_logits, forced_sum, forced_cache = o_cp.whole_frame(w, cfg, layer0, past, tokens, forced_cache=cache)
    np.testing.assert_array_equal(forced_logits, logits)
    np.testing.assert_array_equal(forced_sum, csum)
    np.testing.assert_array_equal(forced_cache, cache)
    for p in range(groups - 1):
        bent = cache.copy()
        bent[:, :, :, p] += 0.5
        moved = o_cp.whole_frame(w, cfg, layer0, past, tokens, forced_cache=bent)[0]
        # logits[g - 1] come from pass g, which reads positions < g
        for g in range(1, groups):
            same = np.array_equal(moved[g - 1], logits[g - 1])
            assert same == (g <= p), (p, g)
