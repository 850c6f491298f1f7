"""Oracle for the code-predictor frame loop (test infrastructure only).

Restates CodePredictorExecutor.whole_frame (executor/code_predictor.py:
159-235) with the fused-branch layer of forward_depth_unrolled
(model/components.py:295-356) over the oracle's norms, q/k RoPE (no bf16
rounding before the rotation in the dense-cache variant, model/kernels.py:
335-405) and short-cache attention:

    pass 0:  h = bf16(past_hidden @ P^T + b); layers at cache position 0
    start:   codec_sum = E0[layer0]; h = P0[layer0]
    g=1..15: x = layers(h, position g) with the final norm
             logits[g-1] = bf16(x @ lm_head[g-1]^T); token = tokens[g-1]
             codec_sum = bf16(codec_sum + E[g-1][token]); h = P[g-1][token]

Layer: x = rmsnorm(h); q, k, v = x @ Wqkv^T; q, k = norm_rope(q, k);
cache[pos] = (k, v); a = attention over cache[:pos+1]; h = bf16(h + bf16(a
@ Wo^T)); x = rmsnorm(h); h = bf16(h + bf16(silu_mul(x @ Wgu^T) @ Wd^T)).

The loop is teacher-forced: the tokens are an input (the GPU's own draws), so
the logits of every group can be compared with the device's while the draw
itself is checked by the sampler oracle on the device's logits.
"""

from __future__ import annotations

import numpy as np

from . import attention, bf16, norms, qk_rope


def _mm(x: np.ndarray, w: np.ndarray, b: np.ndarray | None = None) -> np.ndarray:
    y = x.astype(np.float32) @ w.astype(np.float32).T
    if b is not None:
        y = y + b.astype(np.float32)
    return bf16.round_f32(y)


def layer(w: dict, cfg: dict, i: int, h: np.ndarray, cache: np.ndarray, pos: int, positions: np.ndarray) -> tuple:
    """Layer i at cache position ``pos`` on the residual stream h: writes its K/V at ``pos`` of
    cache[i] and attends over positions [0, pos]; returns (the next normalised input, h)."""

    hq, hkv, d = cfg["num_qo_heads"], cfg["num_kv_heads"], cfg["head_dim"]
    eps, theta = cfg["rms_eps"], cfg["rope_theta"]
    n = h.shape[0]
    L = w["layers"][i]
    x = norms.rmsnorm(h, L["input_norm"], eps)
    qkv = _mm(x, L["qkv"])
    q = qkv[:, : hq * d].reshape(n, hq, d)
    k = qkv[:, hq * d : (hq + hkv) * d].reshape(n, hkv, d)
    v = qkv[:, (hq + hkv) * d :].reshape(n, hkv, d)
    q = qk_rope.norm_rope(q, L["q_norm"], positions, eps, theta, False)
    k = qk_rope.norm_rope(k, L["k_norm"], positions, eps, theta, False)
    cache[i, :, 0, pos] = k
    cache[i, :, 1, pos] = v
    a = bf16.round_f32(attention.short_cache_attention(q, cache[i, :, 0], cache[i, :, 1], pos + 1))
    o = _mm(a.reshape(n, hq * d), L["o"])
    x, h = norms.add_rmsnorm(o, h, L["post_norm"], eps)
    act = norms.silu_mul(_mm(x, L["gate_up"]))
    down = _mm(act, L["down"])
    nxt = w["final_norm"] if i + 1 == len(w["layers"]) else w["layers"][i + 1]["input_norm"]
    return norms.add_rmsnorm(down, h, nxt, eps)


def _layers(w: dict, cfg: dict, h: np.ndarray, cache: np.ndarray, pos: int, positions: np.ndarray) -> tuple:
    x = None
    for i in range(len(w["layers"])):
        x, h = layer(w, cfg, i, h, cache, pos, positions)
    return x, h


def logits_of(w: dict, x: np.ndarray, group: int) -> np.ndarray:
    """Group ``group``'s logits (1-based) from the normalised hidden state x."""

    return _mm(x, w["lm_head"][group - 1])


def whole_frame(w: dict, cfg: dict, layer0_token: np.ndarray, past_hidden: np.ndarray, tokens: np.ndarray,
                positions: np.ndarray | None = None, forced_cache: np.ndarray | None = None):
    """Teacher-forced frame: returns (logits [G-1, R, V], codec_sum [R, talker_hidden], cache).

    ``forced_cache`` (the device's cache after the frame, [layers, R, 2, G, Hkv, D]): each pass g >= 1
    starts from it for positions < g (pass p writes only position p, so the device's final cache
    holds what each pass saw), so every pass is checked on its own and errors do not carry from pass
    to pass; the returned cache still holds the oracle's own K/V at every position.
    """

    groups = cfg["num_code_groups"]
    rows = layer0_token.shape[0]
    if positions is None:
        positions = np.tile(np.arange(groups, dtype=np.int64), (rows, 1))
    cache = np.zeros((len(w["layers"]), rows, 2, groups, cfg["num_kv_heads"], cfg["head_dim"]), dtype=np.float32)
    h = _mm(past_hidden, w["proj_w"], w["proj_b"])
    _layers(w, cfg, h, cache, 0, positions[:, 0])
    codec_sum = w["layer0_embedding"][layer0_token].astype(np.float32)
    h = w["projected_layer0"][layer0_token].astype(np.float32)
    logits = np.zeros((groups - 1, rows, w["lm_head"].shape[1]), dtype=np.float32)
    own = cache if forced_cache is None else cache.copy()
    for g in range(1, groups):
        if forced_cache is not None:
            own[:, :, :, g - 1] = cache[:, :, :, g - 1]  # keep the oracle's own K/V of the last pass
            cache[:, :, :, :g] = forced_cache[:, :, :, :g]
        x, _ = _layers(w, cfg, h, cache, g, positions[:, g])
        logits[g - 1] = _mm(x, w["lm_head"][g - 1])
        tok = tokens[g - 1]
        codec_sum = bf16.round_f32(codec_sum + w["codec_embedding"][g - 1][tok])
        if g < groups - 1:
            h = w["projected_residual"][g - 1][tok].astype(np.float32)
    if forced_cache is not None:
        own[:, :, :, groups - 1] = cache[:, :, :, groups - 1]
    return logits, codec_sum, own
