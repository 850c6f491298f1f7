"""HIP q/k RoPE, norm and SwiGLU kernels vs the oracle and torch fp32 references."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import to_np
from oracle import norms as o_norms
from oracle import qk_rope as o_rope

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("d,round_to_input", [(128, True), (64, False), (64, True)])
def test_qk_norm_rope_dense_cache_and_no_cache(nq, device, d, round_to_input):
    from nari_qwen3_tts_amd import kernels

    g = torch.Generator(device=device)
    g.manual_seed(d)
    rows, hq, hkv = 37, 16, 8
    qkv = torch.randn(rows, (hq + 2 * hkv) * d, generator=g, device=device).to(torch.bfloat16)
    q = qkv[:, : hq * d].view(rows, hq, d)
    k = qkv[:, hq * d : (hq + hkv) * d].view(rows, hkv, d)
    v = qkv[:, (hq + hkv) * d :].view(rows, hkv, d)
    qw = (torch.rand(d, generator=g, device=device) + 0.5).to(torch.bfloat16)
    kw = (torch.rand(d, generator=g, device=device) + 0.5).to(torch.bfloat16)
    pos = torch.randint(0, 4096, (rows, 16), generator=g, device=device)
    q0, k0, v0 = to_np(q), to_np(k), to_np(v)
    col = pos[:, 5]
    if round_to_input:
        kernels.paired_qk_norm_rope_(q, k, qw, kw, col, 1e-6, 1e6)
    else:
        cache = torch.zeros(rows, 2, 16, hkv, d, dtype=torch.bfloat16, device=device)
        kernels.paired_qk_norm_rope_dense_cache_(q, k, v, qw, kw, col, 1e-6, 1e6, cache[:, 0], cache[:, 1], 5)
    torch.cuda.synchronize()
    p = to_np(col)
    np.testing.assert_allclose(to_np(q), o_rope.norm_rope(q0, to_np(qw), p, 1e-6, 1e6, round_to_input), atol=2e-2, rtol=1e-2)
    np.testing.assert_allclose(to_np(k), o_rope.norm_rope(k0, to_np(kw), p, 1e-6, 1e6, round_to_input), atol=2e-2, rtol=1e-2)
    if not round_to_input:
        np.testing.assert_array_equal(to_np(cache[:, 0, 5]), to_np(k))
        np.testing.assert_array_equal(to_np(cache[:, 1, 5]), v0)
        assert torch.count_nonzero(cache[:, :, :5]) == 0 and torch.count_nonzero(cache[:, :, 6:]) == 0


def test_paged_cache_variant_writes_pages(nq, device):
    from nari_qwen3_tts_amd import kernels

    g = torch.Generator(device=device)
    g.manual_seed(3)
    rows, hq, hkv, d, pages, ps = 20, 16, 8, 128, 64, 16
    q = torch.randn(rows, hq, d, generator=g, device=device).to(torch.bfloat16)
    k = torch.randn(rows, hkv, d, generator=g, device=device).to(torch.bfloat16)
    v = torch.randn(rows, hkv, d, generator=g, device=device).to(torch.bfloat16)
    w = torch.ones(d, dtype=torch.bfloat16, device=device)
    layer = torch.zeros(pages, 2, ps, hkv, d, dtype=torch.bfloat16, device=device)
    wp = torch.randperm(pages, generator=g, device=device)[:rows]
    wo = torch.randint(0, ps, (rows,), generator=g, device=device)
    pos = torch.zeros(rows, dtype=torch.long, device=device)  # position 0: identity rotation
    q0, k0, v0 = to_np(q), to_np(k), to_np(v)
    kernels.paired_qk_norm_rope_paged_cache_(q, k, v, w, w, pos, 1e-6, 1e6, layer, wp, wo)
    torch.cuda.synchronize()
    want_k = o_rope.norm_rope(k0, np.ones(d, np.float32), np.zeros(rows), 1e-6, 1e6, True)
    np.testing.assert_allclose(to_np(k), want_k, atol=1e-2, rtol=1e-2)
    want = o_rope.paged_write(np.zeros(layer.shape, np.float32), to_np(k), v0, to_np(wp), to_np(wo))
    np.testing.assert_array_equal(to_np(layer), want)


def test_add_rmsnorm_rmsnorm_silu(nq, device):
    from nari_qwen3_tts_amd.layers import add_rmsnorm, rmsnorm, silu_mul

    g = torch.Generator(device=device)
    g.manual_seed(0)
    rows, width = 64, 2048
    hidden = torch.randn(rows, width, generator=g, device=device).to(torch.bfloat16)
    residual = torch.randn(rows, width, generator=g, device=device).to(torch.bfloat16)
    weight = (torch.rand(width, generator=g, device=device) + 0.5).to(torch.bfloat16)
    h0, r0 = to_np(hidden), to_np(residual)
    add_rmsnorm(hidden, residual, weight, 1e-6)
    want_h, want_r = o_norms.add_rmsnorm(h0, r0, to_np(weight), 1e-6)
    np.testing.assert_array_equal(to_np(residual), want_r)
    np.testing.assert_allclose(to_np(hidden), want_h, atol=2e-2, rtol=1e-2)
    # torch fp32 reference of RMSNorm (model/layers.py:110-115)
    x = torch.randn(rows, width, generator=g, device=device).to(torch.bfloat16)
    out = rmsnorm(x, weight, 1e-6)
    xf = x.float()
    ref = (xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + 1e-6) * weight.float()).to(torch.bfloat16)
    assert (out.float() - ref.float()).abs().max().item() <= 2e-2
    gu = torch.randn(rows, 2 * 6144, generator=g, device=device).to(torch.bfloat16)
    act = silu_mul(gu)
    gf, uf = gu.float().chunk(2, dim=-1)
    ref = torch.nn.functional.silu(gf) * uf
    assert (act.float() - ref).abs().max().item() <= 3e-2


def test_qk_rope_from_projection_partials_equals_bf16_path(nq, device):
    """q/k norm + RoPE + paged KV write fed by the QKV projection's split-K planes gives the same bits
    as the projection's bf16 output fed through the in-place kernel."""

    from nari_qwen3_tts_amd import _lib, kernels
    from nari_qwen3_tts_amd.layers import linear, linear_partials, linear_workspace_bytes

    g = torch.Generator(device=device)
    g.manual_seed(61)
    rows, hidden, hq, hkv, d, pages, ps = 64, 2048, 16, 8, 128, 96, 16
    x = torch.randn(rows, hidden, generator=g, device=device).to(torch.bfloat16)
    w = (torch.randn((hq + 2 * hkv) * d, hidden, generator=g, device=device) * 0.02).to(torch.bfloat16)
    qn = (torch.rand(d, generator=g, device=device) + 0.5).to(torch.bfloat16)
    kn = (torch.rand(d, generator=g, device=device) + 0.5).to(torch.bfloat16)
    pos = torch.randint(0, 5000, (rows,), generator=g, device=device)
    wp = torch.randperm(pages, generator=g, device=device)[:rows]
    wo = torch.randint(0, ps, (rows,), generator=g, device=device)
    cache_a = torch.zeros(pages, 2, ps, hkv, d, dtype=torch.bfloat16, device=device)
    cache_b = torch.zeros_like(cache_a)
    qkv = linear(x, w)
    q = qkv[:, : hq * d].view(rows, hq, d)
    k = qkv[:, hq * d : (hq + hkv) * d].view(rows, hkv, d)
    v = qkv[:, (hq + hkv) * d :].view(rows, hkv, d)
    kernels.paired_qk_norm_rope_paged_cache_(q, k, v, qn, kn, pos, 1e-6, 1e6, cache_a, wp, wo)
    ws = torch.empty(linear_workspace_bytes(rows, w.shape[0], hidden, _lib.NQ_EPI_PARTIALS), dtype=torch.uint8,
                     device=device)
    splits = linear_partials(x, w, ws)
    q_out = torch.empty(rows, hq, d, dtype=torch.bfloat16, device=device)
    _lib.call("nq_qkv_partials_norm_rope_kv_write", ws.data_ptr(), splits, rows, q_out.data_ptr(), q_out.stride(0),
              q_out.stride(1), None, 0, 0, qn.data_ptr(), kn.data_ptr(), pos.data_ptr(), 1, hq, hkv, d, 1e-6, 1e6, 1,
              cache_b.data_ptr(), cache_b.stride(0), cache_b.stride(1), cache_b.stride(2), cache_b.stride(3),
              wp.data_ptr(), wo.data_ptr(), 0, _lib.stream(device))
    torch.cuda.synchronize()
    assert torch.equal(q_out, q)
    assert torch.equal(cache_a, cache_b)


def test_embed_add_rmsnorm_equals_gather_add_then_norm(nq, device):
    """The talker step's input (executor/talker.py:256-262: step embedding + text embedding of the
    step's text token) and the first layer's input norm in one launch give the same bits as the
    gather, the bf16 add and the RMSNorm kernel run one after another; an id outside the table is
    reported in status."""
    import torch.nn.functional as F

    from nari_qwen3_tts_amd import _lib
    from nari_qwen3_tts_amd.layers import embed_add_rmsnorm, rmsnorm

    g = torch.Generator(device=device)
    g.manual_seed(3)
    vocab, width = 1000, 2048
    for rows in (1, 64, 37):
        table = torch.randn(vocab, width, generator=g, device=device).to(torch.bfloat16)
        # a strided addend: the first `width` columns of a wider buffer
        wide = torch.randn(rows, width + 64, generator=g, device=device).to(torch.bfloat16)
        addend = wide[:, :width]
        weight = (torch.rand(width, generator=g, device=device) + 0.5).to(torch.bfloat16)
        ids = torch.randint(0, vocab, (rows,), generator=g, device=device)
        residual = torch.empty(rows, width, dtype=torch.bfloat16, device=device)
        out = torch.empty_like(residual)
        status = torch.zeros(1, dtype=torch.int32, device=device)
        embed_add_rmsnorm(ids, table, addend, weight, 1e-6, residual, out, status)
        want_r = torch.add(addend, F.embedding(ids, table))
        want_o = rmsnorm(want_r, weight, 1e-6)
        assert torch.equal(residual, want_r)
        assert torch.equal(out, want_o)
        assert int(status.item()) == 0
        # fp32 restatement of the same math (model/layers.py:110-115)
        rf = want_r.float()
        ref = (rf * torch.rsqrt(rf.square().mean(-1, keepdim=True) + 1e-6) * weight.float()).to(torch.bfloat16)
        assert (out.float() - ref.float()).abs().max().item() <= 2e-2
    bad = ids.clone()
    bad[-1] = vocab
    embed_add_rmsnorm(bad, table, addend, weight, 1e-6, residual, out, status)
    assert int(status.item()) == _lib.NQ_ERR_INVALID_ARGUMENT
    # the rows with valid ids are unaffected
    assert torch.equal(residual[:-1], want_r[:-1])


def test_gather_sum_rows_and_gather_norm_equal_their_torch_steps(nq, device):
    """The code predictor's codec_sum (layer-0 embedding plus each group's codec embedding,
    executor/code_predictor.py:159-235) in one launch gives the bits of index_select followed by one
    bf16 add per group; the gathered-row norm (no addend) gives those of index_select + RMSNorm."""
    import torch.nn.functional as F

    from nari_qwen3_tts_amd import _lib
    from nari_qwen3_tts_amd.layers import embed_add_rmsnorm, gather_sum_rows, rmsnorm

    g = torch.Generator(device=device)
    g.manual_seed(9)
    rows, width, groups, v0, v = 128, 2048, 15, 3072, 2048
    first = torch.randn(v0, width, generator=g, device=device).to(torch.bfloat16)
    tables = torch.randn(groups + 1, v, width, generator=g, device=device).to(torch.bfloat16)
    first_ids = torch.randint(0, v0, (rows,), generator=g, device=device)
    ids = torch.randint(0, v, (groups, rows), generator=g, device=device)
    want = torch.index_select(first, 0, first_ids)
    for k in range(groups):
        want.add_(F.embedding(ids[k], tables[k]))
    out = torch.empty(rows, width, dtype=torch.bfloat16, device=device)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    gather_sum_rows(first_ids, first, ids, tables, out, status)
    assert torch.equal(out, want)
    assert int(status.item()) == 0
    # strided ids (a transposed view) give the same rows
    out2 = torch.empty_like(out)
    gather_sum_rows(first_ids, first, ids.t().contiguous().t(), tables, out2)
    assert torch.equal(out2, want)
    bad = ids.clone()
    bad[3, 5] = v
    gather_sum_rows(first_ids, first, bad, tables, out2, status)
    assert int(status.item()) == _lib.NQ_ERR_INVALID_ARGUMENT

    hidden = 1024
    proj = torch.randn(v, hidden, generator=g, device=device).to(torch.bfloat16)
    proj[7, :16] = -0.0  # signed zeros stay as they are (nothing is added)
    weight = (torch.rand(hidden, generator=g, device=device) + 0.5).to(torch.bfloat16)
    tok = ids[0].clone()
    tok[0] = 7
    h = torch.empty(rows, hidden, dtype=torch.bfloat16, device=device)
    x = torch.empty_like(h)
    embed_add_rmsnorm(tok, proj, None, weight, 1e-6, h, x)
    want_h = torch.index_select(proj, 0, tok)
    assert torch.equal(h.view(torch.int16), want_h.view(torch.int16))
    assert torch.equal(x, rmsnorm(want_h, weight, 1e-6))
