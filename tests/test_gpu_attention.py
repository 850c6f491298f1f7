"""HIP paged attention vs the oracle (bf16 tolerance: max abs <= 2e-2, mean <= 2e-3)."""

from __future__ import annotations

import zlib

import numpy as np
import pytest
import torch

from helpers import DecodeKey, PrefillKey, adopt_random, attention_error, attention_module, make_kv, to_np
from oracle import attention as o_att
from oracle import qk_rope as o_rope

pytestmark = pytest.mark.gpu
MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def _run(nq, ctx, q, layer_index=0):
    out = ctx.run_attention(q, layer_index)
    torch.cuda.synchronize()
    assert int(ctx.attention_status.item()) == 0
    return out


def _oracle(ctx, q, layer_index=0):
    m = ctx.metadata
    return o_att.paged_attention(
        to_np(q), to_np(ctx.storage[layer_index]), to_np(m.paged_kv_indptr), to_np(m.paged_kv_indices),
        to_np(m.paged_kv_last_page_len), None if m.qo_indptr is None else to_np(m.qo_indptr),
    )


def _decode_case(nq, device, seed, lengths, *, hq=16, hkv=8, d=128, ps=16, pages=4096, capture=None):
    rng = np.random.default_rng(seed)
    rows = len(lengths)
    capture = capture or rows
    kv = make_kv(nq, device, hq=hq, hkv=hkv, d=d, pages=pages, ps=ps, scratch=capture)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    kv.storage.copy_(torch.randn(kv.storage.shape, generator=g, device=device).to(torch.bfloat16))
    rids = adopt_random(kv, rng, lengths)
    key = DecodeKey(capture)
    ctx = kv.create_decode(key, slot=0)
    pubs = kv.prepare_decode(ctx, key, tuple(rids))
    q = torch.randn(capture, hq, d, generator=g, device=device).to(torch.bfloat16)
    return kv, ctx, pubs, q


@pytest.mark.parametrize(
    "label,seed,rows,lo,hi,hq,hkv,d,ps,pages,capture",
    [
        ("cfg1", 1001, 8, 16, 512, 16, 8, 128, 16, 4096, 8),
        ("cfg2-layer", 1002, 64, 64, 2048, 16, 8, 128, 16, 32768, 64),
        ("padded-bucket", 3, 13, 1, 700, 16, 8, 128, 16, 4096, 16),
        ("gqa1", 4, 6, 1, 900, 8, 8, 128, 16, 2048, 6),
        ("gqa4", 5, 6, 1, 900, 32, 8, 128, 16, 2048, 6),
        ("d64", 6, 10, 1, 900, 16, 8, 64, 16, 2048, 10),
        ("ps128", 8, 5, 0, 3000, 16, 8, 128, 128, 512, 5),
        ("ps4", 9, 7, 0, 200, 16, 8, 128, 4, 4096, 7),
        ("long", 10, 3, 6000, 9000, 16, 8, 128, 16, 4096, 3),
    ],
)
def test_paged_decode_matches_oracle(nq, device, label, seed, rows, lo, hi, hq, hkv, d, ps, pages, capture):
    lengths = np.random.default_rng(seed + 100).integers(lo, hi + 1, size=rows)
    kv, ctx, pubs, q = _decode_case(nq, device, seed, lengths, hq=hq, hkv=hkv, d=d, ps=ps, pages=pages, capture=capture)
    out = _run(nq, ctx, q)
    mx, mean = attention_error(to_np(out), _oracle(ctx, q))
    assert mx <= MAX_ABS and mean <= MEAN_ABS, f"{label}: max {mx:.3g} mean {mean:.3g}"
    kv.abort(pubs)


def test_split_rows_identical_across_launches(nq, device):
    """Rows split over several waves are merged by whichever wave arrives last;
    the merge order is fixed, so every launch must give the same bits."""
    lengths = np.random.default_rng(77).integers(64, 2049, size=64)
    kv, ctx, pubs, q = _decode_case(nq, device, 77, lengths, pages=32768, capture=64)
    first = _run(nq, ctx, q).clone()
    mx, mean = attention_error(to_np(first), _oracle(ctx, q))
    assert mx <= MAX_ABS and mean <= MEAN_ABS
    outs = []
    for i in range(200):
        outs.append(ctx.run_attention(q, 0).clone())
    torch.cuda.synchronize()
    assert int(ctx.attention_status.item()) == 0
    for i, o in enumerate(outs):
        assert torch.equal(o, first), f"launch {i} differs"
    kv.abort(pubs)


def test_single_key_returns_value_exactly(nq, device):
    """kv_len = 1: softmax of one score is 1, so the output is V itself."""

    kv, ctx, pubs, q = _decode_case(nq, device, 21, [0] * 9)
    out = _run(nq, ctx, q)
    m = ctx.metadata
    pages = to_np(m.paged_kv_indices).astype(np.int64)
    storage = ctx.storage[0]
    for r in range(9):
        v = storage[int(pages[r]), 1, 0]  # [Hkv, D]
        want = v.repeat_interleave(2, dim=0)
        assert torch.equal(out[r], want), f"row {r}"
    kv.abort(pubs)


def test_equal_keys_give_mean_of_values(nq, device):
    kv, ctx, pubs, q = _decode_case(nq, device, 22, [300, 37, 1000])
    m = ctx.metadata
    indptr = to_np(m.paged_kv_indptr)
    pages = to_np(m.paged_kv_indices).astype(np.int64)
    layer = ctx.storage[0]
    layer[:, 0] = layer[int(pages[0]), 0, 0]  # every key of the pool equals one vector
    out = _run(nq, ctx, q)
    lens = [301, 38, 1001]
    for r in range(3):
        rows = torch.cat([layer[int(p), 1] for p in pages[indptr[r] : indptr[r + 1]]])[: lens[r]]
        want = rows.float().mean(0).repeat_interleave(2, dim=0)
        assert (out[r].float() - want).abs().max().item() <= 1e-2
    kv.abort(pubs)


def test_mixed_prefill_and_decode_rows(nq, device):
    """Reduced cfg3: causal prefill chunks (bottom-right) and decode rows in one launch."""

    rng = np.random.default_rng(1003)
    kv = make_kv(nq, device, pages=8192, ps=16, scratch=128)
    g = torch.Generator(device=device)
    g.manual_seed(1003)
    kv.storage.copy_(torch.randn(kv.storage.shape, generator=g, device=device).to(torch.bfloat16))
    pre_prior = rng.integers(0, 513, size=4)
    pre_adv = rng.integers(32, 257, size=4)
    dec_prior = rng.integers(64, 2049, size=12)
    rids = adopt_random(kv, rng, np.concatenate([pre_prior, dec_prior]))
    advances = tuple(int(a) for a in np.concatenate([pre_adv, np.ones(12, dtype=np.int64)]))
    key = PrefillKey(16, sum(advances) + 3)
    ctx = kv.create_prefill(key, slot=0, decode_rows=True)
    pubs = kv.prepare_prefill(ctx, key, tuple(rids), advances)
    q = torch.randn(key.token_capacity, 16, 128, generator=g, device=device).to(torch.bfloat16)
    out = _run(nq, ctx, q)
    n = sum(advances)
    mx, mean = attention_error(to_np(out)[:n], _oracle(ctx, q)[:n])
    assert mx <= MAX_ABS and mean <= MEAN_ABS, f"max {mx:.3g} mean {mean:.3g}"
    kv.abort(pubs)


def test_mixed_batch_full_config3(nq, device):
    """The mixed workload at full size: 16 prefill chunks (qo U{32..256} over prior context U{0..512})
    and 112 decode rows (KV U{64..2048}), page size 16, pages drawn from a randomly permuted pool,
    planned on the GPU; prefill tiles and decode bins run as the mixed bench leg runs them (two streams,
    fork/join) and every output row is checked against the oracle."""

    rng = np.random.default_rng(1003)
    kv = make_kv(nq, device, pages=16384, ps=16, scratch=256)
    g = torch.Generator(device=device)
    g.manual_seed(1003)
    kv.storage.copy_(torch.randn(kv.storage.shape, generator=g, device=device).to(torch.bfloat16))
    pre_prior = rng.integers(0, 513, size=16)
    pre_adv = rng.integers(32, 257, size=16)
    dec_prior = rng.integers(64, 2049, size=112)
    rids = adopt_random(kv, rng, np.concatenate([pre_prior, dec_prior]))
    advances = tuple(int(a) for a in np.concatenate([pre_adv, np.ones(112, dtype=np.int64)]))
    key = PrefillKey(128, sum(advances))
    ctx = kv.create_prefill(key, slot=0, decode_rows=True)
    pubs = kv.prepare_prefill(ctx, key, tuple(rids), advances)
    q = torch.randn(key.token_capacity, 16, 128, generator=g, device=device).to(torch.bfloat16)
    out = _run(nq, ctx, q)
    n = sum(advances)
    got, want = to_np(out)[:n], _oracle(ctx, q)[:n]
    mx, mean = attention_error(got, want)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, f"max {mx:.3g} mean {mean:.3g}"
    # the decode rows (the last 112 query tokens) on their own as well
    mx, mean = attention_error(got[-112:], want[-112:])
    assert mx <= MAX_ABS and mean <= MEAN_ABS, f"decode rows: max {mx:.3g} mean {mean:.3g}"
    kv.abort(pubs)


@pytest.mark.parametrize("ps,priors,advances", [
    (16, [0, 17, 300, 5], [2, 33, 64, 100]),
    (16, [512, 0], [256, 255]),
    (4, [9, 0, 40], [31, 2, 70]),
    (32, [100, 31, 0], [1, 45, 96]),
    # long causal ranges: tiles cut into key-range pieces, merged by the last to finish (a decode row
    # with decode_rows makes the plan use the wide 64-query tiles)
    (16, [3000, 1500], [40, 200]),
    (128, [2100, 0, 700], [70, 300, 1]),
    # four pieces (more than 48 key tiles), the merge's second pair: narrow tiles, then wide ones
    (16, [3200, 8], [64, 33]),
    (16, [3100, 40, 900], [100, 1, 64]),
])
@pytest.mark.parametrize("decode_rows", [False, True])
def test_prefill_rows_match_oracle(nq, device, ps, priors, advances, decode_rows):
    """Causal prefill rows (MFMA tile path for 16/8 heads of 128) at tile remainders, page sizes and
    prior lengths that straddle pages, with a decode row mixed in where an advance is 1: attended in
    the prefill launch as a one-query row, or (decode_rows) by a decode launch beside it, which
    makes the plan use the wide tiles."""

    rng = np.random.default_rng(sum(advances) + ps)
    scratch = max(32, -(-(sum(advances) + 5) // ps) + 4)  # padding tokens live in scratch slots
    kv = make_kv(nq, device, pages=4096, ps=ps, scratch=scratch)
    g = torch.Generator(device=device)
    g.manual_seed(ps)
    kv.storage.copy_(torch.randn(kv.storage.shape, generator=g, device=device).to(torch.bfloat16))
    rids = adopt_random(kv, rng, np.asarray(priors))
    key = PrefillKey(len(priors) + 2, sum(advances) + 5)
    ctx = kv.create_prefill(key, slot=0, decode_rows=decode_rows)
    pubs = kv.prepare_prefill(ctx, key, tuple(rids), tuple(advances))
    q = torch.randn(key.token_capacity, 16, 128, generator=g, device=device).to(torch.bfloat16)
    out = _run(nq, ctx, q)
    n = sum(advances)
    mx, mean = attention_error(to_np(out)[:n], _oracle(ctx, q)[:n])
    assert mx <= MAX_ABS and mean <= MEAN_ABS, f"max {mx:.3g} mean {mean:.3g}"
    kv.abort(pubs)


def test_attend_runs_rope_write_and_attention(nq, device):
    """TalkerAttentionContext.attend: K1-style q/k transform, paged write, then attention."""

    rng = np.random.default_rng(31)
    kv = make_kv(nq, device, layers=2, pages=1024, ps=16, scratch=8)
    g = torch.Generator(device=device)
    g.manual_seed(31)
    kv.storage.copy_(torch.randn(kv.storage.shape, generator=g, device=device).to(torch.bfloat16))
    rids = adopt_random(kv, rng, rng.integers(1, 400, size=6))
    key = DecodeKey(8)
    ctx = kv.create_decode(key, slot=0)
    pubs = kv.prepare_decode(ctx, key, tuple(rids))
    ctx.select_layer(1)
    qkv = torch.randn(8, (16 + 16) * 128, generator=g, device=device).to(torch.bfloat16)
    q = qkv[:, :2048].view(8, 16, 128)
    k = qkv[:, 2048:3072].view(8, 8, 128)
    v = qkv[:, 3072:].view(8, 8, 128)
    qw = torch.rand(128, generator=g, device=device) + 0.5
    kw = torch.rand(128, generator=g, device=device) + 0.5
    att = attention_module(128, weights=(qw, kw), device=device)
    q0, k0, v0 = to_np(q), to_np(k), to_np(v)
    before = to_np(ctx.storage[1])
    m = ctx.metadata
    pos, wp, wo = to_np(m.position_ids), to_np(m.write_pages), to_np(m.write_offsets)
    out = ctx.attend(att, q, k, v)
    torch.cuda.synchronize()
    q_want = o_rope.norm_rope(q0, to_np(att.q_norm.weight), pos, 1e-6, 1e6, True)
    k_want = o_rope.norm_rope(k0, to_np(att.k_norm.weight), pos, 1e-6, 1e6, True)
    np.testing.assert_allclose(to_np(q), q_want, atol=2e-2, rtol=1e-2)
    np.testing.assert_allclose(to_np(k), k_want, atol=2e-2, rtol=1e-2)
    cache_want = o_rope.paged_write(before, to_np(k), v0, wp, wo)
    np.testing.assert_array_equal(to_np(ctx.storage[1]), cache_want)
    want = o_att.paged_attention(to_np(q), cache_want, to_np(m.paged_kv_indptr), to_np(m.paged_kv_indices),
                                 to_np(m.paged_kv_last_page_len))
    mx, mean = attention_error(to_np(out), want)
    assert mx <= MAX_ABS and mean <= MEAN_ABS
    kv.abort(pubs)


@pytest.mark.parametrize("valid_length", [1, 2, 7, 16])
def test_code_predictor_short_cache(nq, device, valid_length):
    from nari_qwen3_tts_amd.kernels import decode_attn_nhd_short_cache

    g = torch.Generator(device=device)
    g.manual_seed(valid_length)
    rows, hq, hkv, d = 128, 16, 8, 64
    cache = torch.randn(5, rows, 2, 16, hkv, d, generator=g, device=device).to(torch.bfloat16)
    q = torch.randn(rows, 1, hq, d, generator=g, device=device).to(torch.bfloat16)
    out = decode_attn_nhd_short_cache(q, cache[3, :, 0], cache[3, :, 1], valid_length)
    torch.cuda.synchronize()
    want = o_att.short_cache_attention(to_np(q[:, 0]), to_np(cache[3, :, 0]), to_np(cache[3, :, 1]), valid_length)
    mx, mean = attention_error(to_np(out[:, 0]), want)
    assert out.shape == q.shape
    assert mx <= MAX_ABS and mean <= MEAN_ABS


def _fused_case(nq, device, seed, lengths, capture, pages, ps=16):
    rng = np.random.default_rng(seed)
    kv = make_kv(nq, device, layers=1, pages=pages, ps=ps, scratch=capture)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    kv.storage.copy_(torch.randn(kv.storage.shape, generator=g, device=device).to(torch.bfloat16))
    rids = adopt_random(kv, rng, lengths)
    key = DecodeKey(capture)
    ctx = kv.create_decode(key, slot=0)
    pubs = kv.prepare_decode(ctx, key, tuple(rids))
    splits, row = 4, (16 + 2 * 8) * 128
    planes = (torch.randn(splits * capture * row, generator=g, device=device) * 0.5).float()
    qw = torch.rand(128, generator=g, device=device) + 0.5
    kw = torch.rand(128, generator=g, device=device) + 0.5
    att = attention_module(128, weights=(qw, kw), device=device)
    return kv, ctx, pubs, planes, splits, att


def _lengths(kind, rng):
    if kind == "cfg2":
        return rng.integers(64, 2049, size=64), 64, 32768
    if kind == "small":
        return rng.integers(16, 513, size=8), 8, 4096
    if kind == "skewed":  # one row far beyond a bin's share: split across bins and merged
        return np.concatenate([[6000], rng.integers(10, 100, size=20)]), 21, 4096
    if kind == "tiny":  # bins of fewer than 16 blocks: waves with empty spans
        return rng.integers(1, 4, size=13), 16, 1024
    return rng.integers(1, 300, size=40), 40, 4096


@pytest.mark.parametrize("kind", ["cfg2", "small", "skewed", "tiny", "mixed-len"])
def test_fused_decode_rope_attention(nq, device, kind):
    """attend_partials on a decode binding: the fused bins kernel vs the two-kernel path (rope kernel,
    then stream + merge) on the same cache, and vs the oracle."""
    rng = np.random.default_rng(zlib.crc32(kind.encode()) % 1000)
    lengths, capture, pages = _lengths(kind, rng)
    kv, ctx, pubs, planes, splits, att = _fused_case(nq, device, 900 + len(kind), lengths, capture, pages)
    q_out = torch.zeros(capture, 16, 128, dtype=torch.bfloat16, device=device)
    before = kv.storage.clone()
    assert ctx.fused_decode
    out_f = ctx.attend_partials(att, planes, splits, q_out).clone()
    out_f2 = ctx.attend_partials(att, planes, splits, q_out).clone()  # the same K/V rewritten: same inputs
    torch.cuda.synchronize()
    assert int(ctx.attention_status.item()) == 0
    assert ctx.fused_decode, "the library declined the fused shape"
    meta = ctx.workspace[:64].view(torch.int32).cpu().numpy()
    if kind == "skewed":
        assert meta[9] > 0, "no row was split across bins"
    cache_f = kv.storage.clone()
    kv.storage.copy_(before)
    ctx.fused_decode = False
    out_u = ctx.attend_partials(att, planes, splits, q_out).clone()
    torch.cuda.synchronize()
    assert int(ctx.attention_status.item()) == 0
    # the new K/V come from the same norm + RoPE arithmetic: bit-exact
    assert torch.equal(cache_f, kv.storage)
    assert torch.equal(out_f, out_f2)
    m = ctx.metadata
    want = o_att.paged_attention(to_np(q_out), to_np(kv.storage[0]), to_np(m.paged_kv_indptr),
                                 to_np(m.paged_kv_indices), to_np(m.paged_kv_last_page_len))
    for got in (out_f, out_u):
        mx, mean = attention_error(to_np(got), want)
        assert mx <= MAX_ABS and mean <= MEAN_ABS, (kind, mx, mean)
    kv.abort(pubs)
