"""Code-predictor frame loop on the GPU vs the teacher-forced oracle frame.

The device runs the whole 16-group frame; the oracle replays it with the
device's own tokens, so every group's logits are compared (bf16 tolerance),
every token is checked bit-exactly by the sampler oracle on the device's
logits, and codec_sum (bf16 adds of embedding rows) must match exactly.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import to_np
from oracle import code_predictor as o_cp
from oracle import sampler as o_samp

pytestmark = pytest.mark.gpu


def _host_weights(w):
    return dict(
        layers=[{k: to_np(v) for k, v in vars(L).items()} for L in w.layers],
        final_norm=to_np(w.final_norm), lm_head=to_np(w.lm_head), proj_w=to_np(w.proj_w), proj_b=to_np(w.proj_b),
        layer0_embedding=to_np(w.layer0_embedding), codec_embedding=to_np(w.codec_embedding),
        projected_layer0=to_np(w.projected_layer0), projected_residual=to_np(w.projected_residual),
    )


@pytest.mark.parametrize("rows,counter_rng", [(8, False), (5, True)])
def test_frame_matches_oracle(nq, device, rows, counter_rng):
    from nari_qwen3_tts_amd.code_predictor import CodePredictorConfig, CodePredictorFrame, CodePredictorWeights

    cfg = CodePredictorConfig(num_layers=2)
    w = CodePredictorWeights(cfg, device, seed=90 + rows)
    frame = CodePredictorFrame(w, rows, use_counter_rng=counter_rng)
    g = torch.Generator(device=device)
    g.manual_seed(91)
    frame.layer0_token.copy_(torch.randint(0, cfg.talker_vocab, (rows,), generator=g, device=device))
    frame.past_hidden.copy_(torch.randn(rows, cfg.talker_hidden, generator=g, device=device).to(torch.bfloat16))
    frame.temperature.copy_(torch.tensor([0.9, 0.0, 1.3, 0.7, 0.9, 0.5, 1.0, 0.9][:rows], device=device))
    frame.top_k.copy_(torch.tensor([50, 1, 0, 7, 50, 2048, 50, 64][:rows], dtype=torch.int32, device=device))
    frame.top_p.copy_(torch.tensor([0.95, 1.0, 0.8, 1.0, 0.5, 0.9, 1.0, 0.99][:rows], device=device))
    frame.seed.copy_(torch.arange(rows, device=device) * 31 + 5)
    frame.offsets.copy_(torch.arange(rows * 15, device=device).view(rows, 15) * 3)
    if not counter_rng:
        frame.uniforms.copy_(torch.rand(15, rows, generator=g, device=device))
    frames, codec_sum = frame.forward()
    torch.cuda.synchronize()

    hw = _host_weights(w)
    hcfg = dict(num_qo_heads=cfg.num_qo_heads, num_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim,
                rms_eps=cfg.rms_eps, rope_theta=cfg.rope_theta, num_code_groups=cfg.num_code_groups)
    tokens = to_np(frame.tokens)
    logits, csum, cache = o_cp.whole_frame(hw, hcfg, to_np(frame.layer0_token), to_np(frame.past_hidden), tokens)
    got = to_np(frame.logits)
    err = np.abs(got - logits)
    assert err.max() <= 5e-2 and err.mean() <= 2e-3, (err.max(), err.mean())
    # every draw, bit-exact on the device's own logits; with the counter RNG the sampler draws each
    # uniform from (seed, offset) in the same launch, so the oracle's Philox supplies them here
    uniforms = to_np(frame.uniforms)
    if counter_rng:
        seeds, offs = to_np(frame.seed), to_np(frame.offsets)
        uniforms = np.array([[o_samp.uniform_from_counter(int(seeds[r]), int(offs[r, k])) for r in range(rows)]
                             for k in range(15)], dtype=np.float32)
    for k in range(15):
        want_tok = o_samp.sample(got[k], to_np(frame.temperature), to_np(frame.top_k), to_np(frame.top_p), uniforms[k])
        np.testing.assert_array_equal(tokens[k], want_tok)
    np.testing.assert_array_equal(to_np(frames)[:, 0], to_np(frame.layer0_token))
    np.testing.assert_array_equal(to_np(frames)[:, 1:], tokens.T)
    np.testing.assert_array_equal(to_np(codec_sum), csum)
    np.testing.assert_allclose(to_np(frame.kv_cache), cache, atol=3e-2, rtol=2e-2)


def test_frame_replays_in_a_graph(nq, device):
    from nari_qwen3_tts_amd.code_predictor import CodePredictorConfig, CodePredictorFrame, CodePredictorWeights
    from nari_qwen3_tts_amd.graphs import HipGraphCaptureDriver

    cfg = CodePredictorConfig(num_layers=2)
    w = CodePredictorWeights(cfg, device, seed=7)
    rows = 16
    frame = CodePredictorFrame(w, rows, use_counter_rng=True)
    frame.temperature.fill_(0.9)
    frame.top_k.fill_(50)
    frame.top_p.fill_(0.95)
    call = HipGraphCaptureDriver(device=device).capture(frame.forward)
    g = torch.Generator(device=device)
    for trial in range(3):
        g.manual_seed(100 + trial)
        frame.layer0_token.copy_(torch.randint(0, cfg.talker_vocab, (rows,), generator=g, device=device))
        frame.past_hidden.copy_(torch.randn(rows, cfg.talker_hidden, generator=g, device=device).to(torch.bfloat16))
        frame.seed.copy_(torch.randint(0, 1 << 40, (rows,), generator=g, device=device))
        call.replay()
        torch.cuda.synchronize()
        graph_frames, graph_sum = frame.frames.clone(), frame.codec_sum.clone()
        frame.forward()
        torch.cuda.synchronize()
        assert torch.equal(graph_frames, frame.frames)
        assert torch.equal(graph_sum, frame.codec_sum)


@pytest.mark.timeout(300)
def test_bench_frame_b128_matches_oracle(nq, device):
    """The frame batch bench.py replays (5 layers, 128 rows, counter RNG, hipGraph) vs the oracle:

    - two replays give the same bits, and an eager run of the same frame (recording the residual
      stream of every pass and layer) gives them too;
    - teacher-forced per layer: every layer of every pass runs in the oracle on the device's own
      input and the device's K/V of the earlier positions; its residual update within a relative L2
      of 1e-2 and its K/V at the pass's position within bf16 tolerance;
    - each group's logits from the device's own final hidden state held to the bf16 bound (mean
      2e-3, max 2e-2), every draw bit-exact on the device's logits, codec_sum exact;
    - teacher-forced per pass (the device's cache of the earlier positions and its tokens, errors
      then compound through the pass's 5 layers only): mean 2e-3 per group, max 3e-2 (about two bf16
      ulps of the largest logits, |x| < 4)."""
    import bench

    cfg, w, frame, call = bench.build_code_predictor(torch)
    rows = frame.tokens.shape[1]
    groups, layers = cfg.num_code_groups, cfg.num_layers
    call.replay()
    torch.cuda.synchronize()
    first = [frame.frames.clone(), frame.codec_sum.clone(), frame.logits.clone()]
    call.replay()
    torch.cuda.synchronize()
    assert torch.equal(first[0], frame.frames) and torch.equal(first[1], frame.codec_sum)
    assert torch.equal(first[2], frame.logits)
    frame.trace = torch.zeros(groups, layers + 2, rows, cfg.hidden, dtype=torch.bfloat16, device=device)
    frame.forward()
    torch.cuda.synchronize()
    assert torch.equal(first[0], frame.frames) and torch.equal(first[2], frame.logits)

    hw = _host_weights(w)
    hcfg = dict(num_qo_heads=cfg.num_qo_heads, num_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim,
                rms_eps=cfg.rms_eps, rope_theta=cfg.rope_theta, num_code_groups=cfg.num_code_groups)
    tokens = to_np(frame.tokens)
    got = to_np(frame.logits)
    trace = to_np(frame.trace)
    device_cache = to_np(frame.kv_cache)
    positions = to_np(frame.position_ids)
    worst, kv_worst = 0.0, 0.0
    for g in range(groups):
        for i in range(layers):
            cache = device_cache.copy()
            _, h = o_cp.layer(hw, hcfg, i, trace[g, i], cache, g, positions[:, g])
            want, dev = h - trace[g, i], trace[g, i + 1] - trace[g, i]
            worst = max(worst, float(np.linalg.norm(dev - want) / np.linalg.norm(want)))
            kv_worst = max(kv_worst, float(np.abs(cache[i, :, :, g] - device_cache[i, :, :, g]).max()))
    print(f"per-layer rel L2 worst {worst:.2e}, K/V max err {kv_worst:.2e}", flush=True)
    assert worst <= 1e-2 and kv_worst <= 3e-2, (worst, kv_worst)
    head = [(float(e.mean()), float(e.max())) for e in
            (np.abs(got[g - 1] - o_cp.logits_of(hw, trace[g, layers + 1], g)) for g in range(1, groups))]
    print("per-group head logit error (mean, max):", ["%.1e/%.1e" % m for m in head], flush=True)
    assert all(mean <= 2e-3 and mx <= 2e-2 for mean, mx in head), head

    logits, csum, _ = o_cp.whole_frame(hw, hcfg, to_np(frame.layer0_token), to_np(frame.past_hidden), tokens,
                                       forced_cache=device_cache)
    err = np.abs(got - logits)
    per_group = [(float(e.mean()), float(e.max())) for e in err]
    print("per-pass logit error (mean, max):", ["%.1e/%.1e" % m for m in per_group], flush=True)
    assert all(mean <= 2e-3 and mx <= 3e-2 for mean, mx in per_group), per_group
    seeds, offs = to_np(frame.seed), to_np(frame.offsets)
    for k in range(15):
        u = np.array([o_samp.uniform_from_counter(int(seeds[r]), int(offs[r, k])) for r in range(rows)], np.float32)
        want_tok = o_samp.sample(got[k], to_np(frame.temperature), to_np(frame.top_k), to_np(frame.top_p), u)
        np.testing.assert_array_equal(tokens[k], want_tok)
    np.testing.assert_array_equal(to_np(frame.frames)[:, 1:], tokens.T)
    np.testing.assert_array_equal(to_np(frame.codec_sum), csum)
