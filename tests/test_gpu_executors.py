"""The HIP executors at the reference's executor seams, driven the way Executor._replay_stage
(executor/executor.py:252-285) drives TalkerExecutor and CodePredictorExecutor: typed capture keys,
capture at startup (largest first, executor/executor.py:215-250), then replay(key, values) with the
reference's row inputs (tests/reference_rows.py restates their fields).

- Talker decode: 45 rows lowered onto the captured buckets (planner/catalog.py:43-71), each part
  replayed; logits against the oracle step, tokens bit-exact against the oracle sampler on the
  replay's own logits (counter uniforms from each row's seed and offset), next seen masks, next RNG
  offsets (+ 16 x 32), end-of-speech flags; the second decision rotates to the next capture slot.
- Talker prefill: three prompts (host and device row tensors) in one 128-token capture, checked the
  same way against the oracle prefill.
- Code predictor: both captured sampler routes against whole_frame on the same values (identical
  bits), the whole frame against the teacher-forced oracle, and the route rule (contract/rng.py:20-29).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import reference_rows as R
from helpers import adopt_random, to_np
from oracle import code_predictor as o_cp
from oracle import sampler as o_samp
from test_gpu_catalog import _oracle_part
from test_gpu_code_predictor import _host_weights
from test_gpu_prefill import _oracle_prefill_part

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]


def _kv(cfg, device, pages=2048, scratch=64, seed=401):
    from nari_qwen3_tts_amd.talker_kv import PagedTalkerKV

    kv = PagedTalkerKV(num_layers=cfg.num_layers, num_kv_heads=cfg.num_kv_heads, num_qo_heads=cfg.num_qo_heads,
                       head_dim=cfg.head_dim, total_pages=pages, page_size=16, scratch_page_count=scratch,
                       workspace_bytes=0, device=device, dtype=torch.bfloat16)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    kv.storage.copy_(torch.randn(kv.storage.shape, generator=g, device=device).to(torch.bfloat16))
    return kv


def _sampling_rows(n, vocab, codec_vocab, device, gen, offset=512):
    rows = []
    for i in range(n):
        mask = None
        if i % 3:
            mask = torch.zeros(vocab, dtype=torch.bool)
            mask[torch.randint(0, codec_vocab, (16,), generator=gen)] = True
            mask = mask.to(device)
        rows.append(R.TalkerSamplingExecutionRow(temperature=0.9 if i % 5 else 0.0, top_k=50, top_p=0.95,
                                                 repetition_penalty=1.05, seed=7919 * i + 17, offset=offset + i,
                                                 seen_token_mask=mask))
    return rows


def _want_tokens(logits, sampling, cfg, suppress):
    n = len(sampling)
    seen = np.stack([np.zeros(cfg.vocab, bool) if s.seen_token_mask is None else to_np(s.seen_token_mask)
                     for s in sampling])
    u = np.array([o_samp.uniform_from_counter(s.seed, s.offset) for s in sampling], np.float32)
    tok = o_samp.sample(logits, np.array([s.temperature for s in sampling], np.float32),
                        np.array([s.top_k for s in sampling], np.int32),
                        np.array([s.top_p for s in sampling], np.float32), u,
                        penalty=np.array([s.repetition_penalty for s in sampling], np.float32), seen=seen,
                        mask_from=cfg.codec_vocab, eos_id=cfg.eos_id, suppress_eos=np.asarray(suppress, bool))
    want_seen = seen.copy()
    want_seen[np.arange(n), tok] = True
    return tok, want_seen


def test_talker_executor_decode_through_the_replay_stage(nq, device):
    from nari_qwen3_tts_amd.executors import TALKER_FRAME_OFFSET_STRIDE, HipTalkerExecutor
    from nari_qwen3_tts_amd.graphs import lower_rows
    from nari_qwen3_tts_amd.talker import TalkerConfig, TalkerWeights

    cfg = TalkerConfig(num_layers=2)
    kv = _kv(cfg, device)
    weights = TalkerWeights(cfg, device, seed=402, fp8_gate_up=False)
    exe = HipTalkerExecutor(weights=weights, cache=kv, capture_slots=2)
    sizes = (8, 16, 32, 48)
    for size in sorted(sizes, reverse=True):  # the Executor captures the largest keys first
        exe.capture(R.TalkerDecodeCaptureKey(size))
    exe.capture(R.TalkerDecodeCaptureKey(8))  # a second capture of a key is a no-op
    assert exe.captured_cuda_graph_instances == 2 * len(sizes)

    n = 45
    rng = np.random.default_rng(403)
    rids = tuple(adopt_random(kv, rng, rng.integers(16, 300, size=n)))
    gen = torch.Generator(device="cpu").manual_seed(404)
    step_embed = (torch.randn(n, cfg.hidden, generator=gen) * 0.5).to(torch.bfloat16).to(device)
    text_ids = torch.randint(0, cfg.text_vocab, (n,), generator=gen)
    suppress = [i % 2 == 0 for i in range(n)]
    sampling = _sampling_rows(n, cfg.vocab, cfg.codec_vocab, device, gen)
    scratch = list(kv._scratch_pages)
    for decision in range(2):
        parts = lower_rows(n, sizes)
        assert [(p.start, p.stop, p.capture_rows) for p in parts] == [(0, 45, 48)]
        states = [kv.state(r) for r in rids]
        cache_before = to_np(kv.storage)
        rows = tuple(R.TalkerDecodeExecutionRow(
            talker_step_embed=step_embed[i],
            # text ids arrive from the host and from the device, as the engine stages them
            text_token_id=text_ids[i].clone() if i % 2 else text_ids[i].to(device),
            suppress_eos=suppress[i], sampling=sampling[i]) for i in range(n))
        values = R.TalkerDecodeRowsExecutionInput(request_ids=rids, rows=rows)
        key = R.TalkerDecodeCaptureKey(parts[0].capture_rows)
        result = R.replay_stage(exe, R.TalkerDecodeCaptureKey, key, values)
        torch.cuda.synchronize()
        assert exe._next_decode[key] == (decision + 1) % 2
        logits = to_np(result.result.logits)
        pubs = result.kv_publications
        want = _oracle_part(weights, cfg, cache_before, states, pubs, to_np(step_embed), text_ids.numpy(), 48,
                            scratch, 16)
        err = np.abs(logits - want)
        scale = float(np.abs(want).mean())
        assert err.max() <= 6e-2 and err.mean() <= 8e-3 * scale, (decision, err.max(), err.mean(), scale)
        want_tok, want_seen = _want_tokens(logits, sampling, cfg, suppress)
        np.testing.assert_array_equal(to_np(result.result.tokens), want_tok)
        np.testing.assert_array_equal(to_np(result.next_seen_token_masks), want_seen)
        np.testing.assert_array_equal(to_np(result.next_sampling_offsets),
                                      np.array([s.offset for s in sampling]) + TALKER_FRAME_OFFSET_STRIDE)
        np.testing.assert_array_equal(result.end_of_speech(), want_tok == cfg.eos_id)
        assert tuple(result.result.last_hidden.shape) == (n, cfg.hidden)
        for p in pubs:
            p.publish()
        sampling = [R.TalkerSamplingExecutionRow(s.temperature, s.top_k, s.top_p, s.repetition_penalty, s.seed,
                                                 int(o), result.next_seen_token_masks[i])
                    for i, (s, o) in enumerate(zip(sampling, to_np(result.next_sampling_offsets)))]
    # the replay stage refuses a key of the wrong type; the executor refuses a prefill input on a decode key
    with pytest.raises(TypeError):
        R.replay_stage(exe, R.TalkerPrefillCaptureKey, R.TalkerDecodeCaptureKey(48), values)
    with pytest.raises(RuntimeError, match="not been captured"):
        exe.replay(R.TalkerDecodeCaptureKey(64), values)
    with pytest.raises(ValueError, match="exceed the captured shape"):
        exe.replay(R.TalkerDecodeCaptureKey(16), values)
    assert not kv.allocator._inflight


@pytest.mark.parametrize("source", ["cpu", "cuda"])
def test_talker_executor_prefill_through_the_replay_stage(nq, device, source):
    from nari_qwen3_tts_amd.catalog import PrefillKey
    from nari_qwen3_tts_amd.executors import HipTalkerExecutor
    from nari_qwen3_tts_amd.talker import TalkerConfig, TalkerWeights

    cfg = TalkerConfig(num_layers=2)
    kv = _kv(cfg, device, pages=1024, seed=411)
    weights = TalkerWeights(cfg, device, seed=412, fp8_gate_up=False)
    weights.text_embedding.mul_(32)
    weights.codec_embedding.mul_(32)
    exe = HipTalkerExecutor(weights=weights, cache=kv, capture_slots=1)
    key = R.TalkerPrefillCaptureKey(4, 128, None)
    exe.capture(key)
    rng = np.random.default_rng(413)
    gen = torch.Generator(device="cpu").manual_seed(414)
    lengths = (20, 37, 9)
    rids = tuple(adopt_random(kv, rng, (0, 45, 130), prefix="x"))
    total = sum(lengths)
    text = torch.randint(0, cfg.text_vocab, (total,), generator=gen)
    codec = torch.randint(0, cfg.vocab, (total,), generator=gen)
    mask = torch.rand(total, generator=gen) < 0.6
    starts = np.concatenate([[0], np.cumsum(lengths)])
    sampling = _sampling_rows(3, cfg.vocab, cfg.codec_vocab, device, gen, offset=0)
    suppress = [True, False, True]
    dev = torch.device(source) if source == "cpu" else device
    rows = tuple(R.TalkerPrefillExecutionRow(
        text_token_ids=text[starts[i]:starts[i + 1]].to(dev), codec_token_ids=codec[starts[i]:starts[i + 1]].to(dev),
        codec_token_mask=mask[starts[i]:starts[i + 1]].to(dev), suppress_eos=suppress[i], sampling=sampling[i])
        for i in range(3))
    states = [kv.state(r) for r in rids]
    cache = to_np(kv.storage)
    result = R.replay_stage(exe, R.TalkerPrefillCaptureKey, key,
                            R.TalkerPrefillRowsExecutionInput(request_ids=rids, rows=rows))
    torch.cuda.synchronize()
    logits = to_np(result.result.logits)
    want, want_h = _oracle_prefill_part(weights, cfg, cache, states, result.kv_publications, lengths, text.numpy(),
                                        codec.numpy(), mask.numpy(), PrefillKey(4, 128), list(kv._scratch_pages), 16)
    err = np.abs(logits - want)
    scale = float(np.abs(want).mean())
    assert err.max() <= 6e-2 and err.mean() <= 8e-3 * scale, (err.max(), err.mean(), scale)
    got_h = to_np(result.result.last_hidden)
    assert float(np.linalg.norm(got_h - want_h) / np.linalg.norm(want_h)) <= 2e-2
    want_tok, want_seen = _want_tokens(logits, sampling, cfg, suppress)
    np.testing.assert_array_equal(to_np(result.result.tokens), want_tok)
    np.testing.assert_array_equal(to_np(result.next_seen_token_masks), want_seen)
    np.testing.assert_array_equal(result.end_of_speech(), want_tok == cfg.eos_id)
    assert [p.sequence_advance for p in result.kv_publications] == list(lengths)
    kv.abort(result.kv_publications)
    with pytest.raises(TypeError, match="prefill"):
        exe.replay(key, R.TalkerDecodeRowsExecutionInput(request_ids=rids[:1], rows=()))


def _cp_rows(n, cfg, device, gen, temperature, top_k):
    return tuple(R.CodePredictorExecutionRow(
        layer0_token=torch.randint(0, cfg.talker_vocab, (1,), generator=gen).to(device),
        past_hidden=torch.randn(cfg.talker_hidden, generator=gen).to(torch.bfloat16).to(device),
        temperature=temperature, top_k=top_k, top_p=0.95, seed=31 * i + 5,
        offsets=tuple(range(100 * i, 100 * i + 15))) for i in range(n))


def _cp_input(rows, cfg, device):
    return R.CodePredictorInput(
        layer0_token=torch.cat([r.layer0_token.reshape(1) for r in rows]),
        past_hidden=torch.stack([r.past_hidden for r in rows]),
        temperature=torch.tensor([r.temperature for r in rows], dtype=torch.float32, device=device),
        top_k=torch.tensor([r.top_k for r in rows], dtype=torch.int32, device=device),
        top_p=torch.tensor([r.top_p for r in rows], dtype=torch.float32, device=device),
        seed=torch.tensor([r.seed for r in rows], dtype=torch.long, device=device),
        offsets=torch.tensor([r.offsets for r in rows], dtype=torch.long, device=device),
        num_code_groups=cfg.num_code_groups)


def test_code_predictor_executor_routes_and_whole_frame(nq, device):
    from nari_qwen3_tts_amd.code_predictor import CodePredictorConfig, CodePredictorWeights
    from nari_qwen3_tts_amd.executors import HipCodePredictorExecutor
    from nari_qwen3_tts_amd.sampling import sample_logits_cuda_graph

    cfg = CodePredictorConfig(num_layers=2)
    weights = CodePredictorWeights(cfg, device, seed=421)
    exe = HipCodePredictorExecutor(weights=weights, max_batch_size=16)
    key = R.CodePredictorCaptureKey(16)
    exe.capture(key)
    assert exe.captured_cuda_graph_instances == 2
    gen = torch.Generator(device="cpu").manual_seed(422)
    hcfg = dict(num_qo_heads=cfg.num_qo_heads, num_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim,
                rms_eps=cfg.rms_eps, rope_theta=cfg.rope_theta, num_code_groups=cfg.num_code_groups)
    hw = _host_weights(weights)
    for route, temperature, top_k, sampler in (("fused", 0.9, 50, None),
                                                ("general", 0.9, 0, sample_logits_cuda_graph)):
        rows = _cp_rows(12, cfg, device, gen, temperature, top_k)
        values = R.CodePredictorRowsExecutionInput(rows=rows, sampler_route=R.CodePredictorSamplerRoute(route))
        got = R.replay_stage(exe, R.CodePredictorCaptureKey, key, values)
        direct = exe.whole_frame(_cp_input(rows, cfg, device), capture_sampler=sampler)
        torch.cuda.synchronize()
        assert torch.equal(got.frames, direct.frames), route
        assert torch.equal(got.codec_sum, direct.codec_sum), route
        # the direct frame against the teacher-forced oracle: logits within bf16 tolerance, every draw
        # bit-exact on the device's own logits, codec_sum exact
        frame = exe._eager[12]
        tokens = to_np(frame.tokens)
        logits, csum, _ = o_cp.whole_frame(hw, hcfg, to_np(frame.layer0_token), to_np(frame.past_hidden), tokens)
        dev_logits = to_np(frame.logits)
        err = np.abs(dev_logits - logits)
        assert err.max() <= 5e-2 and err.mean() <= 2e-3, (route, err.max(), err.mean())
        for g in range(15):
            u = np.array([o_samp.uniform_from_counter(r.seed, r.offsets[g]) for r in rows], np.float32)
            want = o_samp.sample(dev_logits[g], np.full(12, temperature, np.float32), np.full(12, top_k, np.int32),
                                 np.full(12, 0.95, np.float32), u)
            np.testing.assert_array_equal(tokens[g], want)
        np.testing.assert_array_equal(to_np(direct.frames)[:, 1:], tokens.T)
        np.testing.assert_array_equal(to_np(direct.codec_sum), csum)
    # rows whose route differs from the input's route are refused (contract/rng.py:20-29)
    mixed = _cp_rows(2, cfg, device, gen, 0.9, 50)[:1] + _cp_rows(1, cfg, device, gen, 0.9, 100)
    with pytest.raises(ValueError, match="homogeneous"):
        exe.replay(key, R.CodePredictorRowsExecutionInput(rows=mixed, sampler_route=R.CodePredictorSamplerRoute.FUSED))
    with pytest.raises(ValueError, match="captured shape"):
        exe.replay(key, R.CodePredictorRowsExecutionInput(rows=_cp_rows(17, cfg, device, gen, 0.9, 50)))
    with pytest.raises(RuntimeError, match="not been captured"):
        exe.replay(R.CodePredictorCaptureKey(8), R.CodePredictorRowsExecutionInput(rows=rows[:2]))
