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
             k_norm=to_np(L.attention.k_norm.weight), fp8_gate_up=w.fp8_gate_up)
        for L in w.layers
    ]


@pytest.mark.parametrize("fp8", [True, False])
def test_decode_step_matches_oracle(nq, device, fp8):
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
    weights = TalkerWeights(cfg, device, seed=78, fp8_gate_up=fp8)
    rng = np.random.default_rng(79)
    rids = adopt_random(kv, rng, rng.integers(16, 300, size=rows))
    key = DecodeKey(rows)
    ctx = kv.create_decode(key, slot=0)
    step = TalkerDecodeStep(weights, ctx, rows, use_counter_rng=False)
    step.uniforms.copy_(torch.rand(rows, generator=g, device=device))
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
    def oracle_logits(fp8_gate_up):
        """Logits of the oracle step and the oracle's copy of the cache with its K/V written."""
        layers = _host_layers(weights)
        for L in layers:
            L["fp8_gate_up"] = fp8_gate_up
        cache = cache_before.copy()
        hidden, _ = o_talker.decode_layers(layers, hcfg, residual, cache, meta, final_norm=to_np(weights.final_norm))
        return o_talker.logits(hidden, to_np(weights.codec_head)), cache

    want, oracle_cache = oracle_logits(fp8)
    got = to_np(step.logits)
    err = np.abs(got - want)
    scale = float(np.abs(want).mean())
    if not fp8:
        # bf16 storage at every layer boundary: about one bf16 ulp of the logit on average
        assert err.max() <= 6e-2 and err.mean() <= 8e-3 * scale, (err.max(), err.mean(), scale)
    else:
        # FP8 codes turn the bf16-level device/oracle differences of their inputs into whole e4m3
        # steps: an FP8 MLP moves about 3.3x as much as a bf16 one under one-ulp input noise
        # (1.8 % vs 0.54 % of its output), so the bound is 4x the bf16 one ...
        assert err.max() <= 0.25 and err.mean() <= 3.5e-2 * scale, (err.max(), err.mean(), scale)
        # ... while the FP8 and bf16 semantics differ by more: the step must sit clearly closer
        # to the FP8 oracle than to the bf16 one
        err_bf16 = np.abs(got - oracle_logits(False)[0]).mean()
        assert err.mean() < 0.75 * err_bf16, (err.mean(), err_bf16)
    # the new tokens' K/V landed where the planner said (the oracle wrote its own
    # values into its copy of the cache at the same slots)
    stored = to_np(kv.storage)
    for t in range(rows):
        page, off = int(meta["write_pages"][t]), int(meta["write_offsets"][t])
        got_kv, want_kv = stored[:, page, :, off], oracle_cache[:, page, :, off]
        if not fp8:
            np.testing.assert_allclose(got_kv, want_kv, atol=3e-2, rtol=2e-2)
        else:
            # layer 0's K/V depend only on the step input; later layers' carry the FP8 MLP's
            # amplified differences (normalised values of order 1)
            np.testing.assert_allclose(got_kv[0], want_kv[0], atol=3e-2, rtol=2e-2)
            d = np.abs(got_kv[1:] - want_kv[1:])
            assert d.mean() <= 4e-2 and d.max() <= 0.5, (d.mean(), d.max())
    kv.abort(pubs)


def test_decode_step_refuses_prefill_sized_buckets(nq, device):
    """A decode bucket above the skinny GEMM's 128 rows is refused, not sent to another GEMM backend."""
    from nari_qwen3_tts_amd.talker import TalkerConfig, TalkerDecodeStep, TalkerWeights

    cfg = TalkerConfig(num_layers=1)
    kv = _kv(cfg, device, rows=256)
    key = DecodeKey(256)
    with pytest.raises(ValueError, match="128 rows"):
        TalkerDecodeStep(TalkerWeights(cfg, device, seed=1, fp8_gate_up=False), kv.create_decode(key, slot=0), 256)


def _kv(cfg, device, rows):
    from nari_qwen3_tts_amd.talker_kv import PagedTalkerKV

    return PagedTalkerKV(num_layers=cfg.num_layers, num_kv_heads=cfg.num_kv_heads, num_qo_heads=cfg.num_qo_heads,
                         head_dim=cfg.head_dim, total_pages=1024, page_size=16, scratch_page_count=rows,
                         workspace_bytes=0, device=device, dtype=torch.bfloat16)
