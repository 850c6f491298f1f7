"""Pins the attention, q/k RoPE and norm oracles with closed forms and torch CPU routines."""

from __future__ import annotations

import numpy as np
import torch

from oracle import attention as o_att
from oracle import bf16 as o_bf16
from oracle import norms as o_norms
from oracle import qk_rope as o_rope


def test_bf16_rounding_matches_torch():
    x = np.random.default_rng(0).standard_normal(100000).astype(np.float32) * 100
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(o_bf16.round_f32(x), want)


def _cache(rng, pages, ps, hkv, d):
    return o_bf16.round_f32(rng.standard_normal((pages, 2, ps, hkv, d)).astype(np.float32))


def test_attention_matches_torch_sdpa_with_causal_rows():
    rng = np.random.default_rng(1)
    ps, hq, hkv, d = 16, 8, 2, 64
    cache = _cache(rng, 64, ps, hkv, d)
    kv_indptr = np.array([0, 5, 9, 10])
    kv_indices = rng.permutation(64)[:10]
    last = np.array([3, 16, 1])
    qo = np.array([0, 1, 8, 9])  # decode row, 7-query causal chunk, decode row
    q = o_bf16.round_f32(rng.standard_normal((9, hq, d)).astype(np.float32))
    got = o_att.paged_attention(q, cache, kv_indptr, kv_indices, last, qo)
    for r in range(3):
        pages = kv_indices[kv_indptr[r] : kv_indptr[r + 1]]
        kv_len = (len(pages) - 1) * ps + last[r]
        k, v = o_att.gather_row(cache, pages, kv_len)
        qr = torch.from_numpy(q[qo[r] : qo[r + 1]]).permute(1, 0, 2)  # [H, n, D]
        kt = torch.from_numpy(np.repeat(k, hq // hkv, axis=1)).permute(1, 0, 2)
        vt = torch.from_numpy(np.repeat(v, hq // hkv, axis=1)).permute(1, 0, 2)
        n = qo[r + 1] - qo[r]
        mask = torch.arange(kv_len)[None, :] < (kv_len - n + torch.arange(n) + 1)[:, None]
        want = torch.nn.functional.scaled_dot_product_attention(qr, kt, vt, attn_mask=mask).permute(1, 0, 2)
        np.testing.assert_allclose(got[qo[r] : qo[r + 1]], want.numpy(), atol=1e-5, rtol=1e-5)


def test_attention_closed_forms():
    rng = np.random.default_rng(2)
    ps, hq, hkv, d = 4, 4, 2, 8
    cache = _cache(rng, 8, ps, hkv, d)
    q = rng.standard_normal((1, hq, d)).astype(np.float32)
    one = o_att.paged_attention(q, cache, np.array([0, 1]), np.array([5]), np.array([1]))
    np.testing.assert_allclose(one[0], np.repeat(cache[5, 1, 0], 2, axis=0), atol=1e-6)
    cache[:, 0] = cache[0, 0, 0]
    eq = o_att.paged_attention(q, cache, np.array([0, 3]), np.array([1, 2, 3]), np.array([2]))
    v = np.concatenate([cache[p, 1] for p in (1, 2, 3)])[:10]
    np.testing.assert_allclose(eq[0], np.repeat(v.mean(0), 2, axis=0), atol=1e-5)


def _torch_rope(x, pos, theta):
    """The reference CPU formulation (model/components.py:213-233) in torch."""

    d = x.shape[-1]
    freqs = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    ang = pos.float().unsqueeze(-1) * freqs
    cos = torch.cat((ang.cos(), ang.cos()), -1).unsqueeze(1)
    sin = torch.cat((ang.sin(), ang.sin()), -1).unsqueeze(1)
    a, b = x.chunk(2, -1)
    return x * cos + torch.cat((-b, a), -1) * sin


def test_rope_matches_reference_cpu_formulation_and_invariants():
    rng = np.random.default_rng(3)
    x = o_bf16.round_f32(rng.standard_normal((12, 4, 128)).astype(np.float32))
    w = np.ones(128, np.float32)
    pos = rng.integers(0, 3000, size=12)
    got = o_rope.norm_rope(x, w, pos, 1e-6, 1e6, False)
    normed = x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6)
    want = _torch_rope(torch.from_numpy(normed), torch.from_numpy(pos), 1e6).numpy()
    np.testing.assert_allclose(got, want, atol=2e-2, rtol=1e-2)
    ident = o_rope.norm_rope(x, w, np.zeros(12), 1e-6, 1e6, True)
    np.testing.assert_array_equal(ident, o_bf16.round_f32(normed.astype(np.float32)))
    pair = lambda y: np.hypot(y[..., :64], y[..., 64:])
    np.testing.assert_allclose(pair(got), pair(normed), atol=3e-2, rtol=1e-2)


def test_norms_match_torch():
    rng = np.random.default_rng(4)
    x = o_bf16.round_f32(rng.standard_normal((5, 256)).astype(np.float32))
    r = o_bf16.round_f32(rng.standard_normal((5, 256)).astype(np.float32))
    w = o_bf16.round_f32((rng.random(256) + 0.5).astype(np.float32))
    xt, rt, wt = (torch.from_numpy(a).to(torch.bfloat16) for a in (x, r, w))
    res = rt + xt
    v = res.float()
    want = (v * torch.rsqrt(v.square().mean(-1, keepdim=True) + 1e-6) * wt.float()).to(torch.bfloat16)
    got_h, got_r = o_norms.add_rmsnorm(x, r, w, 1e-6)
    np.testing.assert_array_equal(got_r, res.float().numpy())
    np.testing.assert_allclose(got_h, want.float().numpy(), atol=1e-2, rtol=1e-2)
    gu = o_bf16.round_f32(rng.standard_normal((3, 64)).astype(np.float32))
    g, u = torch.from_numpy(gu).chunk(2, -1)
    np.testing.assert_allclose(o_norms.silu_mul(gu), (torch.nn.functional.silu(g) * u).numpy(), atol=2e-2, rtol=1e-2)
