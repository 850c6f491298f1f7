"""The capture catalog: every decode bucket of a profile x 4 capture slots, a 45-row decision
lowered onto them and each part replayed from its captured graph, checked against the oracle step;
the next decision rotates to the next capture slots; leases and the pool fence fail closed.

- balanced profile (profiles/balanced.yaml:10-12,33): all 19 buckets up to 64, 45 rows -> one
  48-row bucket with 3 padding rows;
- ttfa profile (profiles/ttfa.yaml:10-12): buckets up to 32, 45 rows -> [(32 rows, bucket 32),
  (13 rows, bucket 16, 3 padding)], the lowering of tests/model_optimization/test_config_catalog.py:
  208-216."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import adopt_random, to_np
from oracle import bf16 as o_bf16
from oracle import planner as o_plan
from oracle import sampler as o_samp
from oracle import talker as o_talker

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]


def _oracle_part(weights, cfg, cache_before, states, pubs, step_embed, text_ids, capture, scratch, ps):
    """Oracle logits of one lowered part (its real rows, then padding rows)."""
    meta = o_plan.metadata([(s.sequence_length, s.position_start, list(p.page_indices)) for s, p in zip(states, pubs)],
                           [1] * len(states), capture_rows=capture, token_capacity=capture, prefill=False,
                           page_size=ps, scratch_pages=scratch)
    k = len(states)
    emb = np.zeros((capture, cfg.hidden), np.float32)
    ids = np.zeros(capture, np.int64)
    emb[:k], ids[:k] = step_embed, text_ids
    residual = o_bf16.round_f32(emb + to_np(weights.text_embedding)[ids])
    layers = [dict(input_norm=to_np(L.input_norm), qkv=to_np(L.qkv), o=to_np(L.o), post_norm=to_np(L.post_norm),
                   gate_up=to_np(L.gate_up), down=to_np(L.down), q_norm=to_np(L.attention.q_norm.weight),
                   k_norm=to_np(L.attention.k_norm.weight), fp8_gate_up=False) for L in weights.layers]
    hcfg = dict(num_qo_heads=cfg.num_qo_heads, num_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim,
                rms_eps=cfg.rms_eps, rope_theta=cfg.rope_theta)
    hidden, _ = o_talker.decode_layers(layers, hcfg, residual, cache_before.copy(), meta,
                                       final_norm=to_np(weights.final_norm))
    return o_talker.logits(hidden, to_np(weights.codec_head))[:k]


TTFA_BUCKETS = (1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 16, 24, 32)


@pytest.mark.parametrize("profile", ["balanced", "ttfa"])
def test_catalog_lowers_rotates_and_matches_oracle(nq, device, profile):
    from nari_qwen3_tts_amd.catalog import CAPTURE_SLOTS, DECODE_BUCKETS, DecodeRows, TalkerDecodeCatalog
    from nari_qwen3_tts_amd.errors import SlotBusyError
    from nari_qwen3_tts_amd.talker import TalkerConfig, TalkerWeights
    from nari_qwen3_tts_amd.talker_kv import PagedTalkerKV

    assert DECODE_BUCKETS == (1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 16, 24, 32, 40, 48, 56, 64)
    assert CAPTURE_SLOTS == 4
    cfg = TalkerConfig(num_layers=2)
    ps, pages = 16, 2048
    kv = PagedTalkerKV(num_layers=cfg.num_layers, num_kv_heads=cfg.num_kv_heads, num_qo_heads=cfg.num_qo_heads,
                       head_dim=cfg.head_dim, total_pages=pages, page_size=ps, scratch_page_count=64,
                       workspace_bytes=0, device=device, dtype=torch.bfloat16)
    g = torch.Generator(device=device)
    g.manual_seed(201)
    kv.storage.copy_(torch.randn(kv.storage.shape, generator=g, device=device).to(torch.bfloat16))
    weights = TalkerWeights(cfg, device, seed=202, fp8_gate_up=False)
    buckets = DECODE_BUCKETS if profile == "balanced" else TTFA_BUCKETS
    catalog = TalkerDecodeCatalog(weights, kv, buckets=buckets)
    assert all(len(catalog._slots[b]) == 4 for b in buckets)
    # one attention workspace per capture slot index, shared by every bucket's binding of that slot
    assert len({s.context.workspace.data_ptr() for b in buckets for s in catalog._slots[b]}) == 4

    n = 45
    rng = np.random.default_rng(203)
    rids = tuple(adopt_random(kv, rng, rng.integers(16, 300, size=n)))
    lowered = [(p.logical_rows, p.capture_rows, p.padding) for p in catalog.lower(n)]
    parts = [(0, 45, 48)] if profile == "balanced" else [(0, 32, 32), (32, 45, 16)]
    assert lowered == ([(45, 48, 3)] if profile == "balanced" else [(32, 32, 0), (13, 16, 3)])
    gen = torch.Generator(device="cpu").manual_seed(204)
    seen = torch.zeros(n, cfg.vocab, dtype=torch.bool)
    seen.scatter_(1, torch.randint(0, cfg.codec_vocab, (n, 16), generator=gen), True)
    rows = DecodeRows(
        request_ids=rids,
        step_embed=(torch.randn(n, cfg.hidden, generator=gen) * 0.5).to(torch.bfloat16).to(device),
        text_ids=torch.randint(0, cfg.text_vocab, (n,), generator=gen).to(device),
        temperature=torch.full((n,), 0.9, device=device),
        top_k=torch.full((n,), 50, dtype=torch.int32, device=device),
        top_p=torch.full((n,), 0.95, device=device),
        repetition_penalty=torch.full((n,), 1.05, device=device),
        seed=(torch.arange(n) * 7919 + 17).to(device),
        offsets=torch.full((n,), 512, dtype=torch.long, device=device),
        seen=seen.to(device),
        suppress_eos=(torch.arange(n) % 2 == 0).to(device),
    )
    scratch = list(kv._scratch_pages)
    for decision in range(2):
        states = [kv.state(r) for r in rids]
        cache_before = to_np(kv.storage)
        seen0 = to_np(rows.seen)
        result = catalog.decode(rows)
        torch.cuda.synchronize()
        # the second decision takes the next capture slot of each bucket
        assert result.parts == tuple((capture, decision) for _, _, capture in parts)
        logits = to_np(result.logits)
        pubs = result.publications
        for a, b, capture in parts:
            want = _oracle_part(weights, cfg, cache_before, states[a:b], pubs[a:b], to_np(rows.step_embed)[a:b],
                                to_np(rows.text_ids)[a:b], capture, scratch, ps)
            err = np.abs(logits[a:b] - want)
            scale = float(np.abs(want).mean())
            assert err.max() <= 6e-2 and err.mean() <= 8e-3 * scale, (decision, a, err.max(), err.mean(), scale)
        u = np.array([o_samp.uniform_from_counter(int(s), int(o)) for s, o in
                      zip(to_np(rows.seed), to_np(rows.offsets))], np.float32)
        want_tok = o_samp.sample(logits, to_np(rows.temperature), to_np(rows.top_k), to_np(rows.top_p), u,
                                 penalty=to_np(rows.repetition_penalty), seen=seen0, mask_from=cfg.codec_vocab,
                                 eos_id=cfg.eos_id, suppress_eos=to_np(rows.suppress_eos))
        np.testing.assert_array_equal(to_np(result.tokens), want_tok)
        want_seen = seen0.copy()
        want_seen[np.arange(n), want_tok] = True
        np.testing.assert_array_equal(to_np(result.seen), want_seen)
        np.testing.assert_array_equal(result.end_of_speech(), want_tok == cfg.eos_id)
        assert result.completion_fence.ready()
        for p in pubs:
            p.publish()
        rows = DecodeRows(**{**rows.__dict__, "seen": result.seen.clone(), "offsets": rows.offsets + 512})

    # fail closed: a busy slot lease or an open pool fence refuses the next decision
    first = parts[0][2]
    busy = catalog._slots[first][catalog._next[first]].leases.reserve()
    with pytest.raises(SlotBusyError):
        catalog.decode(rows)
    catalog._slots[first][(catalog._next[first] - 1) % 4].leases.release(busy)
    ticket = catalog.fence.reserve()
    with pytest.raises(SlotBusyError):
        catalog.decode(rows)
    catalog.fence.release(ticket)
    assert all(kv.allocator._inflight.get(r) is None for r in rids)  # nothing left in flight


@pytest.mark.timeout(900)
def test_fp8_28_layer_catalog_replay_matches_oracle(nq, device):
    """The serving build's shape through the catalog: 28 layers with the FP8 gate/up, buckets 16, 32
    and 48 x 4 capture slots; a 45-row decision replayed on a 48-row bucket slot, then the same
    slot's step run eagerly on the same plan with its residual stream recorded: the eager logits
    equal the replay's bit for bit, the oracle checks each of the 28 layers on the recorded input
    (relative L2 of the residual update <= 1.5e-2, the bound of the batch-64 step test), the codec
    head on the final hidden state within 2 bf16 ulps, and the replay's tokens bit-exact against the
    oracle sampler on the replay's own logits."""
    from nari_qwen3_tts_amd.catalog import DecodeRows, TalkerDecodeCatalog
    from nari_qwen3_tts_amd.talker import TalkerConfig, TalkerWeights
    from nari_qwen3_tts_amd.talker_kv import PagedTalkerKV

    cfg = TalkerConfig()
    ps, pages = 16, 4096
    kv = PagedTalkerKV(num_layers=cfg.num_layers, num_kv_heads=cfg.num_kv_heads, num_qo_heads=cfg.num_qo_heads,
                       head_dim=cfg.head_dim, total_pages=pages, page_size=ps, scratch_page_count=64,
                       workspace_bytes=0, device=device, dtype=torch.bfloat16)
    g = torch.Generator(device=device)
    g.manual_seed(211)
    for layer in range(cfg.num_layers):
        kv.storage[layer].normal_(generator=g)
    weights = TalkerWeights(cfg, device, seed=212, fp8_gate_up=True)
    catalog = TalkerDecodeCatalog(weights, kv, buckets=(16, 32, 48))
    n = 45
    rng = np.random.default_rng(213)
    rids = tuple(adopt_random(kv, rng, rng.integers(64, 1024, size=n)))
    gen = torch.Generator(device="cpu").manual_seed(214)
    seen = torch.zeros(n, cfg.vocab, dtype=torch.bool)
    seen.scatter_(1, torch.randint(0, cfg.codec_vocab, (n, 64), generator=gen), True)
    rows = DecodeRows(
        request_ids=rids,
        step_embed=(torch.randn(n, cfg.hidden, generator=gen) * 0.5).to(torch.bfloat16).to(device),
        text_ids=torch.randint(0, cfg.text_vocab, (n,), generator=gen).to(device),
        temperature=torch.full((n,), 0.9, device=device), top_k=torch.full((n,), 50, dtype=torch.int32, device=device),
        top_p=torch.full((n,), 0.95, device=device), repetition_penalty=torch.full((n,), 1.05, device=device),
        seed=(torch.arange(n) * 7919 + 17).to(device), offsets=torch.full((n,), 512, dtype=torch.long, device=device),
        seen=seen.to(device), suppress_eos=(torch.arange(n) % 2 == 0).to(device))
    states = [kv.state(r) for r in rids]
    seen0 = to_np(rows.seen)
    result = catalog.decode(rows)
    torch.cuda.synchronize()
    assert result.parts == ((48, 0),)
    logits = to_np(result.logits)
    u = np.array([o_samp.uniform_from_counter(int(s), int(o)) for s, o in zip(to_np(rows.seed), to_np(rows.offsets))],
                 np.float32)
    want_tok = o_samp.sample(logits, to_np(rows.temperature), to_np(rows.top_k), to_np(rows.top_p), u,
                             penalty=to_np(rows.repetition_penalty), seen=seen0, mask_from=cfg.codec_vocab,
                             eos_id=cfg.eos_id, suppress_eos=to_np(rows.suppress_eos))
    np.testing.assert_array_equal(to_np(result.tokens), want_tok)
    result.end_of_speech()

    # the same slot's step, eagerly, on the same plan, with the residual stream recorded
    step = catalog._slots[48][0].step
    step.trace = torch.zeros(cfg.num_layers + 1, 48, cfg.hidden, dtype=torch.bfloat16, device=device)
    step.seen[:n].copy_(rows.seen)
    step.forward()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_np(step.logits)[:n], logits)
    trace = to_np(step.trace)
    pubs = result.publications
    pages_used = [p for pub in pubs for p in pub.page_indices]
    remap = {p: i for i, p in enumerate(pages_used)}
    scratch = list(range(len(pages_used), len(pages_used) + 48))
    meta = o_plan.metadata([(s.sequence_length, s.position_start, [remap[p] for p in pub.page_indices])
                            for s, pub in zip(states, pubs)], [1] * n, capture_rows=48, token_capacity=48,
                           prefill=False, page_size=ps, scratch_pages=scratch)
    idx = torch.tensor(pages_used, dtype=torch.long, device=device)
    hcfg = dict(num_qo_heads=cfg.num_qo_heads, num_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim,
                rms_eps=cfg.rms_eps, rope_theta=cfg.rope_theta)
    final_norm = to_np(weights.final_norm)
    rels = []
    for li, L in enumerate(weights.layers):
        layer = dict(input_norm=to_np(L.input_norm), qkv=to_np(L.qkv), o=to_np(L.o), post_norm=to_np(L.post_norm),
                     gate_up=to_np(L.gate_up), down=to_np(L.down), q_norm=to_np(L.attention.q_norm.weight),
                     k_norm=to_np(L.attention.k_norm.weight), fp8_gate_up=True,
                     gate_up_q=L.gate_up_q.view(torch.uint8).cpu().numpy(), gate_up_s=L.gate_up_scales.cpu().numpy())
        nxt = final_norm if li + 1 == cfg.num_layers else to_np(weights.layers[li + 1].input_norm)
        cache = np.zeros((1, len(pages_used) + 48, 2, ps, cfg.num_kv_heads, cfg.head_dim), np.float32)
        cache[0, : len(pages_used)] = to_np(kv.storage[li].index_select(0, idx))
        _, res = o_talker.decode_layers([layer], hcfg, trace[li], cache, meta, range(0, 1), final_norm=nxt)
        want_update, got_update = (res - trace[li])[:n], (trace[li + 1] - trace[li])[:n]
        rels.append(float(np.linalg.norm(got_update - want_update) / np.linalg.norm(want_update)))
    print("per-layer rel L2", ["%.1e" % r for r in rels], flush=True)
    assert max(rels) <= 1.5e-2, rels
    from oracle import norms as o_norms

    hidden = to_np(step.hidden)[:n]
    np.testing.assert_allclose(hidden, o_norms.rmsnorm(trace[-1][:n], final_norm, cfg.rms_eps), atol=3e-2,
                               rtol=1e-2)
    want_logits = o_talker.logits(hidden, to_np(weights.codec_head))
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want_logits), 1e-30))) - 7)
    assert np.all(np.abs(logits - want_logits) <= 2 * ulp + 1e-6), "codec head beyond 2 bf16 ulps"
    kv.abort(result.publications)
