"""Each codec oracle primitive against torch's CPU routines, whole-sequence against chunked.

The codec's upstream module tree is absent, so the oracle's arithmetic is pinned here by
independent formulations: ``F.conv1d`` (causal convs with history, dilation, depthwise),
``F.conv_transpose1d`` of the whole sequence (the bias-free overlap carry of
model/incremental_codec.py:90-138), ``F.scaled_dot_product_attention`` with a band mask built
from tril/triu (the sliding window with retained keys, :193-381), ``F.layer_norm``,
``F.rms_norm``, ``F.gelu``, RoPE as a complex rotation and SnakeBeta in its cosine form.  A
flipped tap, a misplaced overlap, an off-by-one window or a sign error in the rotation fails one
of them."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import codec as o_codec

RNG = np.random.default_rng(20)


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))


@pytest.mark.parametrize("cin,cout,k,dil,groups", [(6, 5, 7, 1, 1), (4, 3, 7, 3, 1), (8, 8, 7, 1, 8),
                                                     (5, 5, 3, 9, 5), (3, 2, 1, 1, 1)])
def test_causal_conv_equals_conv1d_over_the_whole_sequence(cin, cout, k, dil, groups):
    n_total = 23
    x = RNG.standard_normal((n_total, cin)).astype(np.float32)
    w = RNG.standard_normal((cout, cin // groups, k)).astype(np.float32)
    b = RNG.standard_normal(cout).astype(np.float32)
    pad = (k - 1) * dil
    # torch: left zero padding of the whole sequence, cross-correlation with the taps as stored
    want = F.conv1d(F.pad(_t(x.T)[None], (pad, 0)), _t(w), _t(b), dilation=dil, groups=groups)[0].T.numpy()
    hist = np.zeros((pad, cin), np.float32)
    parts = []
    for lo, hi in ((0, 5), (5, 6), (6, 17), (17, 23)):
        y, hist = o_codec.causal_conv(x[lo:hi], hist, w, b, dil, groups=groups)
        parts.append(y)
        # the carried history is the last pad input columns seen so far (zeros before the start)
        seen = np.concatenate([np.zeros((pad, cin), np.float32), x[:hi]])
        np.testing.assert_array_equal(hist, seen[seen.shape[0] - pad:] if pad else seen[:0])
    np.testing.assert_allclose(np.concatenate(parts), want, atol=2e-5, rtol=2e-5)


@pytest.mark.parametrize("cin,cout,stride", [(5, 4, 2), (3, 6, 5), (4, 4, 8)])
def test_causal_transconv_equals_conv_transpose1d_of_the_whole_sequence(cin, cout, stride):
    n_total = 13
    x = RNG.standard_normal((n_total, cin)).astype(np.float32)
    w = RNG.standard_normal((cin, cout, 2 * stride)).astype(np.float32)
    b = RNG.standard_normal(cout).astype(np.float32)
    # the whole causal transconv: bias-free expansion, first F*stride positions, plus bias
    full = F.conv_transpose1d(_t(x.T)[None], _t(w), None, stride=stride)[0]
    assert full.shape[-1] == (n_total + 1) * stride
    want = (full[:, : n_total * stride] + _t(b)[:, None]).T.numpy()
    overlap = np.zeros((stride, cout), np.float32)
    parts = []
    for lo, hi in ((0, 1), (1, 6), (6, 13)):
        y, overlap = o_codec.causal_transconv(x[lo:hi], overlap, w, b, stride)
        assert y.shape == ((hi - lo) * stride, cout)
        parts.append(y)
        # the carry is the bias-free tail the whole expansion of x[:hi] leaves past hi*stride
        tail = F.conv_transpose1d(_t(x[:hi].T)[None], _t(w), None, stride=stride)[0, :, hi * stride:].T.numpy()
        np.testing.assert_allclose(overlap, tail, atol=2e-5, rtol=2e-5)
    np.testing.assert_allclose(np.concatenate(parts), want, atol=2e-5, rtol=2e-5)


@pytest.mark.parametrize("window,chunks", [(6, [4, 1, 9, 3]), (26, [12, 30, 7]), (3, [1, 1, 5])])
def test_window_attention_equals_sdpa_with_a_band_mask(window, chunks):
    h, d = 3, 16
    n_total = sum(chunks)
    q = RNG.standard_normal((n_total, h, d)).astype(np.float32)
    k = RNG.standard_normal((n_total, h, d)).astype(np.float32)
    v = RNG.standard_normal((n_total, h, d)).astype(np.float32)
    # whole sequence: query i sees keys i-window+1 .. i (a band of width `window` on and below the diagonal)
    ones = torch.ones(n_total, n_total, dtype=torch.bool)
    band = torch.tril(ones) & torch.triu(ones, diagonal=-(window - 1))
    want = F.scaled_dot_product_attention(_t(q).transpose(0, 1), _t(k).transpose(0, 1), _t(v).transpose(0, 1),
                                          attn_mask=band).transpose(0, 1).numpy()
    r = window - 1
    keys_state = np.zeros((r, h, d), np.float32)
    vals_state = np.zeros((r, h, d), np.float32)
    p0, ctx, parts = 0, 0, []
    for n in chunks:
        keys = np.concatenate([keys_state, k[p0:p0 + n]])
        vals = np.concatenate([vals_state, v[p0:p0 + n]])
        parts.append(o_codec.window_attention(q[p0:p0 + n], keys, vals, p0, ctx, window))
        keys_state, vals_state = keys[keys.shape[0] - r:], vals[vals.shape[0] - r:]
        p0, ctx = p0 + n, min(r, ctx + n)
    np.testing.assert_allclose(np.concatenate(parts), want, atol=2e-5, rtol=2e-5)


def test_norms_gelu_rope_snake_against_torch():
    x = RNG.standard_normal((7, 3, 32)).astype(np.float32) * 3
    w = RNG.standard_normal(32).astype(np.float32)
    b = RNG.standard_normal(32).astype(np.float32)
    np.testing.assert_allclose(o_codec.rmsnorm(x, w, 1e-5), F.rms_norm(_t(x), (32,), _t(w), 1e-5).numpy(),
                               atol=2e-5, rtol=2e-5)
    np.testing.assert_allclose(o_codec.layernorm(x, w, b, 1e-6),
                               F.layer_norm(_t(x), (32,), _t(w), _t(b), 1e-6).numpy(), atol=2e-5, rtol=2e-5)
    np.testing.assert_allclose(o_codec.gelu(x), F.gelu(_t(x)).numpy(), atol=2e-6, rtol=2e-6)
    # RoPE as a complex rotation: (a + i b) * exp(i * pos * theta^(-2j/D)) on the two halves
    pos = np.array([0, 1, 5, 17, 300, 4095, 7, 2])[:7]
    theta = 10000.0
    inv = torch.tensor(theta, dtype=torch.float64) ** (-torch.arange(0, 32, 2, dtype=torch.float64) / 32)
    z = torch.complex(_t(x[..., :16]).double(), _t(x[..., 16:]).double())
    rot = z * torch.polar(torch.ones(7, 1, 16, dtype=torch.float64),
                          torch.from_numpy(pos).double()[:, None, None] * inv[None, None, :])
    want = torch.cat([rot.real, rot.imag], dim=-1).numpy()
    got = o_codec.rope(x, pos, theta)
    np.testing.assert_allclose(got, want, atol=3e-3 * np.abs(x).max(), rtol=0)  # fp32 angles at pos 4095
    np.testing.assert_allclose(o_codec.rope(x[:1], pos[:1], theta), x[:1])  # position 0: identity
    # SnakeBeta: x + sin^2(a x) / b  ==  x + (1 - cos(2 a x)) / (2 b)
    xs = RNG.standard_normal((9, 32)).astype(np.float32)
    la, lb = RNG.standard_normal(32).astype(np.float32) * 0.3, RNG.standard_normal(32).astype(np.float32) * 0.3
    a, bb = np.exp(la.astype(np.float64)), np.exp(lb.astype(np.float64))
    want = xs + (1.0 - np.cos(2.0 * a * xs)) / (2.0 * (bb + 1e-9))
    np.testing.assert_allclose(o_codec.snake(xs, la, lb), want, atol=2e-5, rtol=2e-5)
