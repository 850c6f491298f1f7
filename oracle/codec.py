"""Oracle for the incremental codec-decoder step (test infrastructure only).

The reference adapter (model/incremental_codec.py:11-466) runs an upstream
decoder (qwen-tts 0.1.1, not in the reference tree) on fresh frames only,
carrying three kinds of boundary state per stream:

- causal Conv1d left histories: prepend the stored `pad` input columns, keep
  the last `pad` columns of [history, input] (:58-88);
- causal ConvTranspose1d overlaps: the expansion is computed bias-free, the
  stored overlap is added to its first `stride` positions, the first
  F*stride positions (plus bias) are emitted and the rest is stored (:90-138);
- the transformer's retained K/V: keys/values of the last
  `sliding_window - 1` frames, a validity count (`transformer_context_length`)
  and the frame position that RoPE uses (:193-381).

This module restates that adapter over a random-init synthetic decoder of the
same structure (the structure, not the upstream weights, is what the state
handling depends on): 16-codebook embedding sum, pre-conv, an 8-layer
sliding-window transformer with per-head q/k RMSNorm, RoPE and layer scales,
two transconv + ConvNeXt upsample stages, then decoder blocks of SnakeBeta +
transconv + three dilated residual units, SnakeBeta + final conv, clamp to
[-1, 1]; PCM16 = round(clamp * 32767) (executor/codec.py:236-238).

Everything is float32 numpy over channels-last arrays [T, C].  `decode_whole`
runs a full sequence with zero initial state; `decode_incremental` runs one
chunk against explicit state and returns the new state.  Pinned by the
invariant the reference's adapter docstring claims (:11-19): decoding a
sequence in chunks equals decoding it whole; by the PCM16 known answers of
tests/job_separation/test_codec.py:192-194; and primitive by primitive against
torch's CPU routines (conv1d, conv_transpose1d, scaled_dot_product_attention
with a band mask, layer_norm, rms_norm, gelu, complex-rotation RoPE and the
cosine form of SnakeBeta), whole-sequence against chunked.
"""

from __future__ import annotations

import math

import numpy as np

F32 = np.float32


# ---------------------------------------------------------------------------
# primitives


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = x.astype(F32)
    var = np.mean(x * x, axis=-1, keepdims=True, dtype=F32)
    return (x / np.sqrt(var + F32(eps))) * w


def layernorm(x: np.ndarray, w: np.ndarray, b: np.ndarray, eps: float) -> np.ndarray:
    mu = np.mean(x, axis=-1, keepdims=True, dtype=F32)
    var = np.mean((x - mu) ** 2, axis=-1, keepdims=True, dtype=F32)
    return (x - mu) / np.sqrt(var + F32(eps)) * w + b


def gelu(x: np.ndarray) -> np.ndarray:
    erf = np.vectorize(math.erf, otypes=[np.float64])
    return (0.5 * x.astype(np.float64) * (1.0 + erf(x.astype(np.float64) / math.sqrt(2.0)))).astype(F32)


def snake(x: np.ndarray, alpha: np.ndarray, beta: np.ndarray) -> np.ndarray:
    """SnakeBeta: x + 1/beta * sin(alpha x)^2 (per channel, log-scale parameters exponentiated)."""

    a = np.exp(alpha).astype(F32)
    b = np.exp(beta).astype(F32)
    return (x + (F32(1.0) / (b + F32(1e-9))) * np.sin(x * a) ** 2).astype(F32)


def causal_conv(x: np.ndarray, hist: np.ndarray, w: np.ndarray, b: np.ndarray | None, dilation: int,
                groups: int = 1):
    """x [F, Cin], hist [pad, Cin] with pad = (K-1)*dilation; w [Cout, Cin/groups, K].
    Returns (y [F, Cout], new_hist [pad, Cin])."""

    cout, cin_g, k = w.shape
    pad = (k - 1) * dilation
    full = np.concatenate([hist, x], axis=0).astype(F32)
    n = x.shape[0]
    y = np.zeros((n, cout), dtype=F32)
    for tap in range(k):
        seg = full[tap * dilation : tap * dilation + n]  # input at t - (K-1-tap)*dilation
        if groups == 1:
            y += seg @ w[:, :, tap].T
        else:  # depthwise
            y += seg * w[:, 0, tap][None, :]
    if b is not None:
        y += b
    new_hist = full[full.shape[0] - pad :] if pad else full[:0]
    return y.astype(F32), new_hist.astype(F32)


def causal_transconv(x: np.ndarray, overlap: np.ndarray, w: np.ndarray, b: np.ndarray, stride: int):
    """x [F, Cin], overlap [stride, Cout]; w [Cin, Cout, 2*stride].  Returns (y [F*stride, Cout], new_overlap)."""

    n = x.shape[0]
    cin, cout, k = w.shape
    assert k == 2 * stride
    full = np.zeros(((n + 1) * stride, cout), dtype=F32)
    for t in range(n):
        full[t * stride : t * stride + k] += (x[t] @ w.reshape(cin, cout * k)).reshape(cout, k).T
    full[:stride] += overlap
    y = full[: n * stride] + b
    return y.astype(F32), full[n * stride :].astype(F32)


def rope(x: np.ndarray, positions: np.ndarray, theta: float) -> np.ndarray:
    """x [T, H, D] rotate-half RoPE at integer positions [T]."""

    d = x.shape[-1]
    half = d // 2
    inv = (F32(1.0) / (F32(theta) ** (np.arange(0, d, 2, dtype=F32) / F32(d)))).astype(F32)
    ang = positions.astype(F32)[:, None] * inv[None, :]
    cos = np.cos(ang)[:, None, :].astype(F32)
    sin = np.sin(ang)[:, None, :].astype(F32)
    a, bb = x[..., :half], x[..., half:]
    return np.concatenate([a * cos - bb * sin, bb * cos + a * sin], axis=-1).astype(F32)


def window_attention(q: np.ndarray, keys: np.ndarray, vals: np.ndarray, p0: int, ctx: int,
                     window: int) -> np.ndarray:
    """Sliding-window attention of n fresh queries at positions p0 .. p0+n-1 over the r = window-1
    retained keys (positions p0-r .. p0-1, of which the last ``ctx`` are valid) followed by the n
    fresh keys: a query at position t sees valid keys at positions t-window < s <= t, scale 1/sqrt(D)
    (model/incremental_codec.py:227-262,318-326).  q [n, H, D], keys / vals [r + n, H, D]."""

    n, _, d = q.shape
    r = window - 1
    pos = p0 + np.arange(n)
    kpos = np.concatenate([p0 - r + np.arange(r), pos])
    kvalid = np.concatenate([np.arange(r) >= r - ctx, np.ones(n, dtype=bool)])
    att = np.zeros(q.shape, dtype=F32)
    scale = F32(1.0 / math.sqrt(d))
    for i in range(n):
        m = kvalid & (kpos <= pos[i]) & (kpos > pos[i] - window)
        s = np.einsum("hd,khd->hk", q[i], keys[m]) * scale
        s = s - s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        att[i] = np.einsum("hk,khd->hd", p, vals[m])
    return att


# ---------------------------------------------------------------------------
# the decoder


def empty_state(cfg: dict) -> dict:
    """Zero state of one stream (shapes from the config)."""

    st = {"frame_position": 0, "context": 0, "hist": {}, "overlap": {}}
    r = cfg["window"] - 1
    st["k"] = np.zeros((cfg["layers"], r, cfg["heads"], cfg["head_dim"]), dtype=F32)
    st["v"] = np.zeros_like(st["k"])
    for name, (cin, pad) in conv_histories(cfg).items():
        st["hist"][name] = np.zeros((pad, cin), dtype=F32)
    for name, (cout, s) in transconv_overlaps(cfg).items():
        st["overlap"][name] = np.zeros((s, cout), dtype=F32)
    return st


def conv_histories(cfg: dict) -> dict:
    """name -> (input channels, history length) of every causal conv."""

    out = {"pre_conv": (cfg["dim"], 2)}
    for u in range(len(cfg["up_strides"])):
        out[f"up{u}.dw"] = (cfg["dim"], 6)
    out["dec0"] = (cfg["dim"], 6)
    for i in range(len(cfg["dec_strides"])):
        c = cfg["dec_channels"][i + 1]
        for j, dil in enumerate(cfg["dilations"]):
            out[f"dec{i + 1}.res{j}.a"] = (c, 6 * dil)
    out["final"] = (cfg["dec_channels"][-1], 6)
    return out


def transconv_overlaps(cfg: dict) -> dict:
    out = {}
    for u, s in enumerate(cfg["up_strides"]):
        out[f"up{u}.tc"] = (cfg["dim"], s)
    for i, s in enumerate(cfg["dec_strides"]):
        out[f"dec{i + 1}.tc"] = (cfg["dec_channels"][i + 1], s)
    return out


def _transformer(w: dict, cfg: dict, x: np.ndarray, st: dict) -> np.ndarray:
    n = x.shape[0]
    h_, d = cfg["heads"], cfg["head_dim"]
    r = cfg["window"] - 1
    p0 = st["frame_position"]
    ctx = st["context"]
    pos = p0 + np.arange(n)
    h = x @ w["in_w"].T + w["in_b"]
    new_k = np.zeros_like(st["k"])
    new_v = np.zeros_like(st["v"])
    for li, L in enumerate(w["tf"]):
        y = rmsnorm(h, L["ln1"], cfg["eps"])
        q = (y @ L["wq"].T).reshape(n, h_, d)
        k = (y @ L["wk"].T).reshape(n, h_, d)
        v = (y @ L["wv"].T).reshape(n, h_, d)
        q = rope(rmsnorm(q, L["qn"], cfg["eps"]), pos, cfg["theta"])
        k = rope(rmsnorm(k, L["kn"], cfg["eps"]), pos, cfg["theta"])
        keys = np.concatenate([st["k"][li], k], axis=0)  # [r + n, H, D]
        vals = np.concatenate([st["v"][li], v], axis=0)
        att = window_attention(q, keys, vals, p0, ctx, cfg["window"])
        h = h + (att.reshape(n, h_ * d) @ L["wo"].T) * L["ls1"]
        y = rmsnorm(h, L["ln2"], cfg["eps"])
        h = h + (gelu(y @ L["w1"].T) @ L["w2"].T) * L["ls2"]
        new_k[li] = keys[keys.shape[0] - r :]
        new_v[li] = vals[vals.shape[0] - r :]
    st["k"], st["v"] = new_k, new_v
    st["frame_position"] = p0 + n
    st["context"] = min(r, ctx + n)
    h = rmsnorm(h, w["out_norm"], cfg["eps"])
    return (h @ w["out_w"].T + w["out_b"]).astype(F32)


def decode_incremental(w: dict, cfg: dict, codes: np.ndarray, st: dict) -> np.ndarray:
    """codes [F, Q] of one stream; ``st`` is updated in place.  Returns wav [F * upsample] in [-1, 1]."""

    x = np.zeros((codes.shape[0], cfg["dim"]), dtype=F32)
    for qi in range(codes.shape[1]):
        x += w["codebooks"][qi][codes[:, qi]]
    x, st["hist"]["pre_conv"] = causal_conv(x, st["hist"]["pre_conv"], w["pre_conv_w"], w["pre_conv_b"], 1)
    x = _transformer(w, cfg, x, st)
    for u, s in enumerate(cfg["up_strides"]):
        U = w["up"][u]
        x, st["overlap"][f"up{u}.tc"] = causal_transconv(x, st["overlap"][f"up{u}.tc"], U["tc_w"], U["tc_b"], s)
        res = x
        y, st["hist"][f"up{u}.dw"] = causal_conv(x, st["hist"][f"up{u}.dw"], U["dw_w"], U["dw_b"], 1,
                                                 groups=cfg["dim"])
        y = layernorm(y, U["ln_w"], U["ln_b"], 1e-6)
        y = gelu(y @ U["pw1_w"].T + U["pw1_b"]) @ U["pw2_w"].T + U["pw2_b"]
        x = res + U["gamma"] * y
    x, st["hist"]["dec0"] = causal_conv(x, st["hist"]["dec0"], w["dec0_w"], w["dec0_b"], 1)
    for i, s in enumerate(cfg["dec_strides"]):
        B = w["blocks"][i]
        x = snake(x, B["alpha"], B["beta"])
        x, st["overlap"][f"dec{i + 1}.tc"] = causal_transconv(x, st["overlap"][f"dec{i + 1}.tc"], B["tc_w"],
                                                              B["tc_b"], s)
        for j, dil in enumerate(cfg["dilations"]):
            R = B["res"][j]
            y = snake(x, R["a1"], R["b1"])
            y, st["hist"][f"dec{i + 1}.res{j}.a"] = causal_conv(y, st["hist"][f"dec{i + 1}.res{j}.a"], R["c1_w"],
                                                                R["c1_b"], dil)
            y = snake(y, R["a2"], R["b2"])
            y = y @ R["c2_w"][:, :, 0].T + R["c2_b"]
            x = x + y
    x = snake(x, w["final_alpha"], w["final_beta"])
    x, st["hist"]["final"] = causal_conv(x, st["hist"]["final"], w["final_w"], w["final_b"], 1)
    return np.clip(x[:, 0], -1.0, 1.0).astype(F32)


def decode_whole(w: dict, cfg: dict, codes: np.ndarray) -> np.ndarray:
    """A full causal pass from zero state."""

    return decode_incremental(w, cfg, codes, empty_state(cfg))


def pcm16(wav: np.ndarray) -> np.ndarray:
    """round(clamp(x, -1, 1) * 32767) with round-half-to-even, as int16."""

    return np.rint(np.clip(wav.astype(F32), -1.0, 1.0) * F32(32767.0)).astype(np.int16)
