"""One talker decode step (2 layers of the full-width talker, 8 ragged rows) vs the oracle step."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import DecodeKey, adopt_random, to_np
from oracle import planner as o_plan
from oracle import talker as o_talker

pytestmark = pytest.mark.gpu


def _host_layers(w):
    return [
        dict(input_norm=to_np(L.input_norm), qkv=to_np(L.qkv), o=to_np(L.o), post_norm=to_np(L.post_norm),
             gate_up=to_np(L.gate_up), down=to_np(L.down), q_norm=to_np(L.attention.q_norm.weight),
             k_norm=to_np(L.attention.k_norm.weight))
        for L in w.layers
    ]


@pytest.mark.parametrize("hip_linear", [True, False])
def test_decode_step_matches_oracle(nq, device, hip_linear):
    from nari_qwen3_tts_amd.talker import TalkerConfig, TalkerDecodeStep, TalkerWeights
    from nari_qwen3_tts_amd.talker_kv import PagedTalkerKV

    cfg = TalkerConfig(num_layers=2)
    rows, ps, pages = 8, 16, 512
    kv = PagedTalkerKV(num_layers=cfg.num_layers, num_kv_heads=cfg.num_kv_heads, num_qo_heads=cfg.num_qo_heads,
                       head_dim=cfg.head_dim, total_pages=pages, page_size=ps, scratch_page_count=rows,
                       workspace_bytes=0, device=device, dtype=torch.bfloat16)
    g = torch.Generator(device=device)
    g.manual_seed(77)
    kv.storage.copy_(torch.randn(kv.storage.shape, generator=g, device=device).to(torch.bfloat16))
    weights = TalkerWeights(cfg, device, seed=78)
    rng = np.random.default_rng(79)
    rids = adopt_random(kv, rng, rng.integers(16, 300, size=rows))
    key = DecodeKey(rows)
    ctx = kv.create_decode(key, slot=0)
    step = TalkerDecodeStep(weights, ctx, rows)
    step.use_hip_linear = step.use_hip_linear and hip_linear
    assert step.use_hip_linear == hip_linear
    step.step_embed.copy_((torch.randn(rows, cfg.hidden, generator=g, device=device) * 0.5).to(torch.bfloat16))
    step.text_ids.copy_(torch.randint(0, cfg.text_vocab, (rows,), generator=g, device=device))

    states = [kv.state(r) for r in rids]
    free_before = list(kv.allocator.free_list())
    cache_before = to_np(kv.storage)
    pubs = kv.prepare_decode(ctx, key, tuple(rids))
    step.forward()
    torch.cuda.synchronize()

    alloc = o_plan.Allocator(pages, ps)
    alloc.free = free_before
    meta = o_plan.metadata([(s.sequence_length, s.position_start, list(p.page_indices)) for s, p in zip(states, pubs)],
                           [1] * rows, capture_rows=rows, token_capacity=rows, prefill=False, page_size=ps,
                           scratch_pages=list(kv._scratch_pages))
    residual = to_np(step.step_embed) + to_np(weights.text_embedding)[to_np(step.text_ids)]
    residual = o_talker.bf16.round_f32(residual)
    hcfg = dict(num_qo_heads=cfg.num_qo_heads, num_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim,
                rms_eps=cfg.rms_eps, rope_theta=cfg.rope_theta)
    hidden, _ = o_talker.decode_layers(_host_layers(weights), hcfg, residual, cache_before, meta,
                                       final_norm=to_np(weights.final_norm))
    want = o_talker.logits(hidden, to_np(weights.codec_head))
    got = to_np(step.logits)
    err = np.abs(got - want)
    scale = float(np.abs(want).mean())
    # bf16 storage at every layer boundary: about one bf16 ulp of the logit on average
    assert err.max() <= 6e-2 and err.mean() <= 8e-3 * scale, (err.max(), err.mean(), scale)
    # the new tokens' K/V landed where the planner said (the oracle wrote its own
    # values into its copy of the cache at the same slots)
    stored = to_np(kv.storage)
    for t in range(rows):
        page, off = int(meta["write_pages"][t]), int(meta["write_offsets"][t])
        np.testing.assert_allclose(stored[:, page, :, off], cache_before[:, page, :, off], atol=3e-2, rtol=2e-2)
    kv.abort(pubs)
