"""nq_paged_attention_noalloc (plan + attention in the library's static device scratch) against the
workspace entry points it stands for (nq_attention_plan + nq_paged_attention): the same plan over
the same metadata gives the same bits.  Two calls in a row, the second smaller, so stale scratch
contents of the first call must not leak into the second; then a batch whose plan exceeds the
scratch is refused before any launch."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import DecodeKey, PrefillKey, adopt_random, attention_error, make_kv, to_np
from oracle import attention as o_att

pytestmark = pytest.mark.gpu


def _mixed_case(nq, device, seed, pre_prior, pre_adv, dec_prior, pages):
    rng = np.random.default_rng(seed)
    rows = len(pre_prior) + len(dec_prior)
    kv = make_kv(nq, device, pages=pages, ps=16, scratch=max(rows, 64))
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    kv.storage.copy_(torch.randn(kv.storage.shape, generator=g, device=device).to(torch.bfloat16))
    rids = adopt_random(kv, rng, np.concatenate([pre_prior, dec_prior]).astype(np.int64))
    advances = tuple(int(a) for a in np.concatenate([pre_adv, np.ones(len(dec_prior), dtype=np.int64)]))
    if len(pre_prior):
        key = PrefillKey(rows, sum(advances) + 3)
        ctx = kv.create_prefill(key, slot=0, decode_rows=True)  # decode rows through the decode launch
        pubs = kv.prepare_prefill(ctx, key, tuple(rids), advances)
        tokens = key.token_capacity
    else:
        key = DecodeKey(rows)
        ctx = kv.create_decode(key, slot=0)
        pubs = kv.prepare_decode(ctx, key, tuple(rids))
        tokens = rows
    q = torch.randn(tokens, 16, 128, generator=g, device=device).to(torch.bfloat16)
    return kv, ctx, pubs, q, sum(advances)


def test_noalloc_attention_equals_the_workspace_path(nq, device):
    from nari_qwen3_tts_amd import _lib
    from nari_qwen3_tts_amd.kernels import paged_attention_noalloc

    cases = [
        # 4 causal prefill chunks + 12 decode rows over an 8192-page pool
        (1101, [0, 130, 512, 7], [32, 100, 256, 45], list(np.random.default_rng(5).integers(64, 2049, 12)), 8192),
        # then a smaller batch: 5 decode rows over a 2048-page pool
        (1102, [], [], [17, 300, 1000, 64, 2], 2048),
    ]
    for seed, pre_prior, pre_adv, dec_prior, pages in cases:
        print(f"case seed {seed}: {len(pre_prior)} prefill + {len(dec_prior)} decode rows, {pages} pages", flush=True)
        kv, ctx, pubs, q, n = _mixed_case(nq, device, seed, np.asarray(pre_prior, np.int64),
                                          np.asarray(pre_adv, np.int64), np.asarray(dec_prior, np.int64), pages)
        want = ctx.run_attention(q, 0).clone()
        status = torch.zeros(1, dtype=torch.int32, device=device)
        got = torch.full_like(q, 7.0)
        # the workspace path issues a mixed batch's decode rows with NQ_ATTN_BESIDE_PREFILL (their workgroup
        # size, hence their K/V span split, depends on it), so the comparison takes the same parts
        parts = _lib.NQ_ATTN_DECODE | _lib.NQ_ATTN_PREFILL | (_lib.NQ_ATTN_BESIDE_PREFILL if pre_prior else 0)
        paged_attention_noalloc(q, kv.storage[0], ctx.metadata, max_pages=ctx.index_capacity, parts=parts,
                                status=status, out=got)
        torch.cuda.synchronize()
        assert int(status.item()) == 0 and int(ctx.attention_status.item()) == 0
        assert torch.equal(got[:n], want[:n]), f"seed {seed}: no-allocation output differs from the workspace path"
        m = ctx.metadata
        ref = o_att.paged_attention(to_np(q), to_np(kv.storage[0]), to_np(m.paged_kv_indptr),
                                    to_np(m.paged_kv_indices), to_np(m.paged_kv_last_page_len),
                                    None if m.qo_indptr is None else to_np(m.qo_indptr))
        mx, mean = attention_error(to_np(got)[:n], ref[:n])
        assert mx <= 2e-2 and mean <= 2e-3, (seed, mx, mean)
        kv.abort(pubs)
        del kv, ctx
        torch.cuda.empty_cache()


def test_noalloc_attention_refuses_batches_beyond_its_scratch(nq, device):
    from nari_qwen3_tts_amd import _lib
    from nari_qwen3_tts_amd.kernels import paged_attention_noalloc

    kv, ctx, pubs, q, _ = _mixed_case(nq, device, 1103, np.asarray([], np.int64), np.asarray([], np.int64),
                                      np.asarray([40, 50], np.int64), 512)
    lib = _lib.load()
    big = 1 << 22  # a 4M-page pool: the plan would not fit the static scratch
    assert lib.nq_attention_workspace_bytes(q.shape[0], big, 16, 16, 8, 128) > _lib.NQ_NOALLOC_SCRATCH_BYTES
    out = torch.zeros_like(q)
    with pytest.raises(ValueError, match="scratch"):
        paged_attention_noalloc(q, kv.storage[0], ctx.metadata, max_pages=big, out=out)
    m = ctx.metadata
    rc = lib.nq_paged_attention_noalloc(
        None, m.paged_kv_indptr.data_ptr(), m.paged_kv_last_page_len.data_ptr(), m.paged_kv_indices.data_ptr(),
        2, q.data_ptr(), q.stride(0), q.stride(1), kv.storage[0].data_ptr(), *kv.storage[0].stride()[:4],
        kv.storage.shape[1], 16, 16, 8, 128, 128 ** -0.5, out.data_ptr(), out.stride(0), out.stride(1),
        q.shape[0], big, _lib.NQ_ATTN_DECODE, None, _lib.stream(device))
    assert rc == _lib.NQ_ERR_INVALID_ARGUMENT
    torch.cuda.synchronize()
    assert torch.count_nonzero(out).item() == 0  # nothing was launched
    kv.abort(pubs)
