"""Fused HIP sampler vs the oracle: token ids bit-exact given the same logits and uniforms."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import to_np
from oracle import sampler as o_samp

pytestmark = pytest.mark.gpu


def _inputs(device, seed, rows, vocab, *, dtype=torch.float32, temperature=0.9, top_k=50, top_p=0.95, penalty=1.05,
            history=64):
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    logits = torch.randn(rows, vocab, generator=g).to(dtype)
    seen = torch.zeros(rows, vocab, dtype=torch.bool)
    if history:
        ids = torch.randint(0, vocab, (rows, history), generator=g)
        seen.scatter_(1, ids, True)
    u = torch.rand(rows, generator=g)
    t = torch.full((rows,), float(temperature))
    k = torch.full((rows,), int(top_k), dtype=torch.int32)
    p = torch.full((rows,), float(top_p))
    r = torch.full((rows,), float(penalty))
    return [x.to(device) for x in (logits, t, k, p, u, r, seen)]


def _check(logits, t, k, p, u, r, seen, **kw):
    from nari_qwen3_tts_amd.sampling import sample_with_uniforms

    got = sample_with_uniforms(logits, t, k, p, u, repetition_penalty=r, seen_token_mask=seen, **kw)
    torch.cuda.synchronize()
    want = o_samp.sample(
        to_np(logits), to_np(t), to_np(k), to_np(p), to_np(u), penalty=to_np(r), seen=to_np(seen),
        mask_from=kw.get("mask_from"), eos_id=kw.get("eos_id", -1),
        suppress_eos=None if kw.get("suppress_eos") is None else to_np(kw["suppress_eos"]),
    )
    np.testing.assert_array_equal(to_np(got), want)
    return got


def test_cfg1_sampler_bit_exact(nq, device):
    _check(*_inputs(device, 1001, 8, 3072))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_batch64_talker_sampler_bit_exact(nq, device, dtype):
    _check(*_inputs(device, 1002, 64, 3072, dtype=dtype))


@pytest.mark.parametrize(
    "top_k,top_p,temperature",
    [(1, 0.95, 0.9), (64, 1.0, 0.7), (0, 0.9, 1.0), (100, 0.8, 1.3), (3072, 1.0, 0.5), (5000, 0.5, 0.9), (17, 1e-6, 0.9)],
)
def test_topk_topp_variants_bit_exact(nq, device, top_k, top_p, temperature):
    _check(*_inputs(device, 7 + top_k, 16, 3072, top_k=top_k, top_p=top_p, temperature=temperature))


def test_greedy_rows_and_masks(nq, device):
    logits, t, k, p, u, r, seen = _inputs(device, 3, 32, 3072)
    t[::3] = 0.0
    sup = torch.zeros(32, dtype=torch.bool, device=device)
    sup[::2] = True
    got = _check(logits, t, k, p, u, r, seen, mask_from=2048, eos_id=2150, suppress_eos=sup)
    toks = to_np(got)
    assert np.all((toks < 2048) | (toks == 2150))
    assert not np.any(toks[::2] == 2150)


def test_ties_resolve_to_lowest_id(nq, device):
    rows, vocab = 8, 2048
    logits = torch.zeros(rows, vocab, device=device)
    logits[:, 100:200] = 5.0  # a plateau of 100 equal maxima
    u = torch.linspace(0, 0.999, rows, device=device)
    t = torch.full((rows,), 1.0, device=device)
    k = torch.full((rows,), 50, dtype=torch.int32, device=device)
    p = torch.ones(rows, device=device)
    r = torch.ones(rows, device=device)
    seen = torch.zeros(rows, vocab, dtype=torch.bool, device=device)
    got = to_np(_check(logits, t, k, p, u, r, seen))
    assert np.all((got >= 100) & (got < 150))  # top-50 of the plateau are its 50 lowest ids
    t.zero_()
    assert np.all(to_np(_check(logits, t, k, p, u, r, seen)) == 100)


def test_update_seen_marks_sampled_token(nq, device):
    from nari_qwen3_tts_amd.sampling import sample_with_uniforms

    logits, t, k, p, u, r, seen = _inputs(device, 5, 16, 3072, history=0)
    before = seen.clone()
    tok = sample_with_uniforms(logits, t, k, p, u, repetition_penalty=r, seen_token_mask=seen, update_seen=True)
    torch.cuda.synchronize()
    after = seen.clone()
    after_expected = before.clone()
    after_expected[torch.arange(16, device=device), tok] = True
    assert torch.equal(after, after_expected)


def test_code_predictor_vocab_15_steps_bit_exact(nq, device):
    g = torch.Generator(device="cpu")
    g.manual_seed(1004)
    rows, vocab = 128, 2048
    for step in range(15):
        logits = torch.randn(rows, vocab, generator=g).to(torch.bfloat16).to(device)
        u = torch.rand(rows, generator=g).to(device)
        t = torch.full((rows,), 0.9, device=device)
        k = torch.full((rows,), 50, dtype=torch.int32, device=device)
        p = torch.ones(rows, device=device)
        r = torch.ones(rows, device=device)
        seen = torch.zeros(rows, vocab, dtype=torch.bool, device=device)
        _check(logits, t, k, p, u, r, seen)


def test_uniforms_from_counter_match_philox(nq, device):
    from nari_qwen3_tts_amd.sampling import uniforms_from_counter

    seeds = torch.tensor([0, 1, 7, 2**40 + 3, 123456789, 2**62], dtype=torch.long)
    offsets = torch.tensor([0, 512, 544, 1 << 33, 15 * 32, 999], dtype=torch.long)
    got = to_np(uniforms_from_counter(seeds.to(device), offsets.to(device)))
    want = np.array([o_samp.uniform_from_counter(int(s), int(o)) for s, o in zip(seeds, offsets)], dtype=np.float32)
    np.testing.assert_array_equal(got, want)
    # Strided offset column, as the code predictor passes offsets[:, group - 1].
    table = torch.arange(6 * 15, dtype=torch.long).view(6, 15) * 32
    got = to_np(uniforms_from_counter(seeds.to(device), table.to(device)[:, 4]))
    want = np.array([o_samp.uniform_from_counter(int(s), int(o)) for s, o in zip(seeds, table[:, 4])], dtype=np.float32)
    np.testing.assert_array_equal(got, want)


def test_reference_signatures_are_row_local(nq, device):
    """A row's draw depends only on its own (seed, offset): batch == singleton == permuted."""

    from nari_qwen3_tts_amd.sampling import sample_code_predictor_cuda_graph, sample_talker_cuda_graph

    logits, t, k, p, _, r, seen = _inputs(device, 9, 12, 3072)
    seed = torch.arange(12, dtype=torch.long, device=device) * 7 + 1
    off = torch.arange(12, dtype=torch.long, device=device) * 512
    batch = sample_talker_cuda_graph(logits, t, k, p, seed, off, r, seen)
    perm = torch.randperm(12, device=device)
    permuted = sample_talker_cuda_graph(logits[perm], t[perm], k[perm], p[perm], seed[perm], off[perm], r[perm], seen[perm])
    assert torch.equal(batch[perm], permuted)
    single = torch.cat([sample_talker_cuda_graph(logits[i : i + 1], t[i : i + 1], k[i : i + 1], p[i : i + 1],
                                                 seed[i : i + 1], off[i : i + 1], r[i : i + 1], seen[i : i + 1])
                        for i in range(12)])
    assert torch.equal(batch, single)
    cp = sample_code_predictor_cuda_graph(logits, t, k, p, seed, off)
    assert cp.dtype == torch.long and cp.shape == (12,)


def test_counter_draw_equals_uniforms_then_sample(nq, device):
    """One launch with the in-kernel Philox draw gives the tokens of uniforms_from_counter followed by
    sample_with_uniforms, including a strided offset column and the seen-mask update."""

    from nari_qwen3_tts_amd.sampling import sample_with_counter, sample_with_uniforms, uniforms_from_counter

    logits, t, k, p, _, r, seen = _inputs(device, 21, 40, 3072)
    seed = torch.arange(40, dtype=torch.long, device=device) * 7919 + 3
    table = (torch.arange(40 * 15, dtype=torch.long, device=device).view(40, 15) * 97) % 100003
    for off in (table[:, 0].contiguous(), table[:, 6]):
        u = uniforms_from_counter(seed, off)
        seen_a, seen_b = seen.clone(), seen.clone()
        want = sample_with_uniforms(logits, t, k, p, u, repetition_penalty=r, seen_token_mask=seen_a, mask_from=2048,
                                    eos_id=2150, update_seen=True)
        got = sample_with_counter(logits, t, k, p, seed, off, repetition_penalty=r, seen_token_mask=seen_b,
                                  mask_from=2048, eos_id=2150, update_seen=True)
        assert torch.equal(got, want)
        assert torch.equal(seen_a, seen_b)


@pytest.mark.parametrize("rows", [64, 7])
def test_draw_from_projection_planes_equals_projection_then_draw(nq, device, rows):
    """The codec head's split-K planes summed, rounded and drawn from in the sampling launch give the
    logits and tokens of the bf16 projection followed by sample_with_counter (the talker step's head,
    executor/talker.py:173-183, 240-243, 373), seen update included."""

    from nari_qwen3_tts_amd.layers import linear, linear_partials, linear_workspace_bytes
    from nari_qwen3_tts_amd.sampling import sample_with_counter, sample_with_counter_from_planes

    g = torch.Generator(device=device)
    g.manual_seed(5)
    hidden, vocab = 2048, 3072
    x = torch.randn(rows, hidden, generator=g, device=device).to(torch.bfloat16)
    w = (torch.randn(vocab, hidden, generator=g, device=device) * 0.05).to(torch.bfloat16)
    ws = torch.empty(max(16, linear_workspace_bytes(rows, vocab, hidden, nq._lib.NQ_EPI_PARTIALS)), dtype=torch.uint8,
                     device=device)
    t = torch.full((rows,), 0.9, device=device)
    k = torch.full((rows,), 50, dtype=torch.int32, device=device)
    p = torch.full((rows,), 0.95, device=device)
    r = torch.full((rows,), 1.05, device=device)
    seed = torch.arange(rows, dtype=torch.long, device=device) * 7919 + 11
    off = torch.arange(rows, dtype=torch.long, device=device) * 3 + 512
    seen = torch.rand(rows, vocab, generator=g, device=device) < 0.02
    want_logits = linear(x, w, workspace=ws)
    seen_a, seen_b = seen.clone(), seen.clone()
    want = sample_with_counter(want_logits, t, k, p, seed, off, repetition_penalty=r, seen_token_mask=seen_a,
                               mask_from=2048, eos_id=2150, update_seen=True)
    splits = linear_partials(x, w, ws)
    assert splits > 1
    planes = ws[: splits * rows * vocab * 4].view(torch.float32).view(splits, rows, vocab)
    got_logits = torch.zeros(rows, vocab, dtype=torch.bfloat16, device=device)
    got = sample_with_counter_from_planes(planes, t, k, p, seed, off, logits_out=got_logits, repetition_penalty=r,
                                          seen_token_mask=seen_b, mask_from=2048, eos_id=2150, update_seen=True)
    assert torch.equal(got_logits, want_logits)
    assert torch.equal(got, want)
    assert torch.equal(seen_a, seen_b)
    # without a logits output
    got2 = sample_with_counter_from_planes(planes, t, k, p, seed, off, repetition_penalty=r,
                                           seen_token_mask=seen.clone(), mask_from=2048, eos_id=2150)
    assert torch.equal(got2, want)
