"""GPU ragged planner vs the oracle and the reference's literal vectors (bit-exact)."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import DecodeKey, PrefillKey, adopt_random, make_kv
from oracle import planner as o_plan

pytestmark = pytest.mark.gpu
LITERALS = json.loads((Path(__file__).parent / "golden" / "reference_literals.json").read_text())


def _np(t):
    return t.detach().cpu().numpy()


def _oracle_for(kv, priors, pubs, advances, capture_rows, token_capacity, prefill):
    rows = [(s.sequence_length, s.position_start, list(p.page_indices)) for s, p in zip(priors, pubs)]
    return o_plan.metadata(rows, list(advances), capture_rows=capture_rows, token_capacity=token_capacity,
                           prefill=prefill, page_size=kv.page_size, scratch_pages=list(kv._scratch_pages))


def _assert_matches(ctx, want, label):
    m = ctx.metadata
    got = {
        "kv_indptr": m.paged_kv_indptr, "kv_indices": m.paged_kv_indices, "last_page_len": m.paged_kv_last_page_len,
        "position_ids": m.position_ids, "write_pages": m.write_pages, "write_offsets": m.write_offsets,
    }
    if "qo_indptr" in want:
        got["qo_indptr"] = m.qo_indptr
    for name, tensor in got.items():
        np.testing.assert_array_equal(_np(tensor), want[name], err_msg=f"{label}: {name}")
    status = _np(ctx.buffers.status)
    assert status[0] == 0, f"{label}: planner status {status}"


def test_prefill_literals_of_reference(nq, device):
    lit = LITERALS["prefill_metadata"]
    pool = lit["pool"]
    kv = make_kv(nq, device, layers=pool["num_layers"], hq=pool["num_qo_heads"], hkv=pool["num_kv_heads"],
                 d=pool["head_dim"], pages=pool["total_pages"], ps=pool["page_size"], scratch=pool["scratch_page_count"])
    for rid in lit["requests"]:
        kv.add_request(rid)
    key = PrefillKey(lit["capture"]["capture_batch_size"], lit["capture"]["token_capacity"])
    ctx = kv.create_prefill(key, slot=0)
    priors = [kv.state(r) for r in lit["requests"]]
    pubs = kv.prepare_prefill(ctx, key, tuple(lit["requests"]), tuple(lit["advances"]))
    m = ctx.metadata
    assert _np(m.qo_indptr).tolist() == lit["qo_indptr"]
    assert _np(m.position_ids).tolist() == lit["position_ids"]
    assert _np(m.write_pages)[:5].tolist() == [pubs[r].page_indices[0] for r in lit["write_pages_rows"]]
    assert _np(m.write_offsets)[:5].tolist() == lit["write_offsets_head"]
    assert len(_np(m.paged_kv_last_page_len)) == lit["last_page_len_count"]
    assert len(set(m.padding_pages)) == lit["unique_padding_pages"]
    assert len(set(_np(m.paged_kv_indices)[-2:].tolist())) == lit["unique_tail_indices"]
    wp, wo = _np(m.write_pages).tolist(), _np(m.write_offsets).tolist()
    padding = set(zip(wp[5:], wo[5:]))
    assert len(padding) == lit["unique_padding_writes"]
    assert not padding & set(zip(wp[:5], wo[:5]))
    _assert_matches(ctx, _oracle_for(kv, priors, pubs, lit["advances"], key.capture_batch_size, key.token_capacity,
                                     True), "prefill literal")
    kv.abort(pubs)


def test_decode_after_prefill_literals_of_reference(nq, device):
    lit = LITERALS["decode_after_prefill"]
    pool = lit["pool"]
    kv = make_kv(nq, device, layers=pool["num_layers"], hq=pool["num_qo_heads"], hkv=pool["num_kv_heads"],
                 d=pool["head_dim"], pages=pool["total_pages"], ps=pool["page_size"], scratch=pool["scratch_page_count"])
    kv.add_request("a")
    pkey = PrefillKey(lit["prefill_capture"]["capture_batch_size"], lit["prefill_capture"]["token_capacity"])
    initial = kv.prepare_prefill(kv.create_prefill(pkey, slot=0), pkey, ("a",), (lit["prefill_advance"],))
    initial[0].publish()
    key = DecodeKey(lit["decode_capture"]["capture_batch_size"])
    ctx = kv.create_decode(key, slot=0)
    pubs = kv.prepare_decode(ctx, key, ("a",))
    m = ctx.metadata
    assert _np(m.position_ids).tolist() == lit["position_ids"]
    assert int(_np(m.write_pages)[0]) == pubs[0].page_indices[0]
    assert int(_np(m.write_offsets)[0]) == lit["write_offset0"]
    assert int(_np(m.write_pages)[1]) == m.padding_pages[lit["padding_write_page_index"]]
    assert kv.state("a").sequence_length == lit["sequence_length_after_abort"]
    kv.abort(pubs)
    assert kv.state("a").sequence_length == lit["sequence_length_after_abort"]


def test_scratch_capacity_errors_of_reference(nq, device):
    lit = LITERALS["scratch_capacity_errors"]
    kv = make_kv(nq, device, layers=2, hq=4, hkv=2, d=8, pages=16, ps=4, scratch=lit["scratch_page_count"])
    kv.add_request("a")
    dkey = DecodeKey(lit["decode_capture"])
    with pytest.raises(ValueError, match=lit["decode_error"]):
        kv.prepare_decode(kv.create_decode(dkey, slot=0), dkey, ("a",))
    pkey = PrefillKey(lit["prefill_capture"]["capture_batch_size"], lit["prefill_capture"]["token_capacity"])
    with pytest.raises(ValueError, match=lit["prefill_error"]):
        kv.prepare_prefill(kv.create_prefill(pkey, slot=1), pkey, ("a",), (1,))
    assert kv.state("a").sequence_length == 0


def test_pool_exhaustion_raises_before_launch(nq, device):
    from nari_qwen3_tts_amd.errors import KVAllocationError

    kv = make_kv(nq, device, layers=1, hq=4, hkv=2, d=64, pages=10, ps=4, scratch=5)
    kv.add_request("a")
    kv.add_request("b")
    key = PrefillKey(2, 18)
    with pytest.raises(KVAllocationError):
        kv.prepare_prefill(kv.create_prefill(key, slot=0), key, ("a", "b"), (1, 17))
    assert kv.allocator.free_pages == 5
    assert kv.state("a").sequence_length == 0


@pytest.mark.parametrize(
    "label,seed,rows,capture,prior_lo,prior_hi,pool,ps",
    [
        ("cfg1", 1001, 8, 8, 16, 512, 4096, 16),
        ("cfg2", 1002, 64, 64, 64, 2048, 32768, 16),
        ("padded", 7, 45, 48, 1, 300, 4096, 16),
        ("ps128", 11, 5, 8, 0, 1000, 512, 128),
        ("ps4", 12, 9, 12, 0, 60, 1024, 4),
    ],
)
def test_decode_metadata_matches_oracle(nq, device, label, seed, rows, capture, prior_lo, prior_hi, pool, ps):
    rng = np.random.default_rng(seed)
    kv = make_kv(nq, device, pages=pool, ps=ps, scratch=capture)
    prior = rng.integers(prior_lo, prior_hi + 1, size=rows)
    rids = adopt_random(kv, rng, prior)
    key = DecodeKey(capture)
    ctx = kv.create_decode(key, slot=0)
    priors = [kv.state(r) for r in rids]
    pubs = kv.prepare_decode(ctx, key, tuple(rids))
    want = _oracle_for(kv, priors, pubs, [1] * rows, capture, capture, False)
    _assert_matches(ctx, want, label)
    taken = sum(len(p.page_indices) - len(s.page_indices) for p, s in zip(pubs, priors))
    assert int(_np(ctx.buffers.status)[1]) == taken
    for rid, pub in zip(rids, pubs):
        row = kv.allocator.slot(rid)
        np.testing.assert_array_equal(_np(kv._table[row, : len(pub.page_indices)]), np.asarray(pub.page_indices))
    kv.abort(pubs)


def test_mixed_prefill_and_decode_rows_match_oracle(nq, device):
    """cfg3 shape: 16 prefill chunks (prior U[0,512], advance U[32,256]) + 112 decode rows."""

    rng = np.random.default_rng(1003)
    kv = make_kv(nq, device, pages=32768, ps=16, scratch=300)
    pre_prior = rng.integers(0, 513, size=16)
    pre_adv = rng.integers(32, 257, size=16)
    dec_prior = rng.integers(64, 2049, size=112)
    rids = adopt_random(kv, rng, np.concatenate([pre_prior, dec_prior]))
    advances = tuple(int(a) for a in np.concatenate([pre_adv, np.ones(112, dtype=np.int64)]))
    tokens = sum(advances)
    key = PrefillKey(128, tokens + 5)
    ctx = kv.create_prefill(key, slot=0)
    priors = [kv.state(r) for r in rids]
    pubs = kv.prepare_prefill(ctx, key, tuple(rids), advances)
    want = _oracle_for(kv, priors, pubs, advances, 128, tokens + 5, True)
    _assert_matches(ctx, want, "cfg3")
    kv.abort(pubs)


def test_multi_step_lifecycle_tracks_oracle_allocator(nq, device):
    """Publish / discard / remove over several steps; pages come back and are re-taken lowest first."""

    rng = np.random.default_rng(5)
    pages, ps = 96, 4
    kv = make_kv(nq, device, layers=1, hq=4, hkv=2, d=64, pages=pages, ps=ps, scratch=12)
    oracle = o_plan.Allocator(pages, ps)
    assert oracle.claim_scratch(12) == list(kv._scratch_pages)
    live = []
    for step in range(12):
        if len(live) < 5:
            rid = f"q{step}"
            kv.add_request(rid)
            oracle.add(rid)
            live.append(rid)
        rows = list(live)
        prefill = step % 3 == 0
        advances = [int(rng.integers(1, 9)) if prefill else 1 for _ in rows]
        capture = 6
        key = PrefillKey(capture, sum(advances) + 2) if prefill else DecodeKey(capture)
        ctx = kv.create_prefill(key, slot=0) if prefill else kv.create_decode(key, slot=0)
        priors = [kv.state(r) for r in rows]
        news, proposed = oracle.reserve(rows, advances)
        pubs = (kv.prepare_prefill(ctx, key, tuple(rows), tuple(advances)) if prefill
                else kv.prepare_decode(ctx, key, tuple(rows)))
        assert [list(p.page_indices) for p in pubs] == proposed
        tokens = key.token_capacity if prefill else capture
        _assert_matches(ctx, _oracle_for(kv, priors, pubs, advances, capture, tokens, prefill), f"step {step}")
        discard = step % 4 == 1
        for rid, pub, new, adv in zip(rows, pubs, news, advances):
            if discard:
                pub.discard()
                oracle.discard(new)
            else:
                pub.publish()
                oracle.publish(rid, pub.page_indices, adv)
        if step % 5 == 4:
            gone = live.pop(0)
            kv.remove_request(gone)
            oracle.remove(gone)
        assert list(kv.allocator.free_list()) == oracle.free
        # the device copy, kept by front moves and GPU merges only, equals the ledger's list
        assert kv.device_free_list().cpu().tolist() == oracle.free
        assert int(kv.free_list_status.item()) == 0
