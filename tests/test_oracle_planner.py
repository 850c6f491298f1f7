"""Pins the planner oracle: reference literal vectors and an independent token-by-token simulation."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import planner as o_plan

LITERALS = json.loads((Path(__file__).parent / "golden" / "reference_literals.json").read_text())


def test_prefill_literals():
    lit = LITERALS["prefill_metadata"]
    pool = lit["pool"]
    alloc = o_plan.Allocator(pool["total_pages"], pool["page_size"])
    scratch = alloc.claim_scratch(pool["scratch_page_count"])
    for rid in lit["requests"]:
        alloc.add(rid)
    news, proposed = alloc.reserve(lit["requests"], lit["advances"])
    rows = [(0, 0, p) for p in proposed]
    m = o_plan.metadata(rows, lit["advances"], capture_rows=4, token_capacity=8, prefill=True,
                        page_size=pool["page_size"], scratch_pages=scratch)
    assert m["qo_indptr"].tolist() == lit["qo_indptr"]
    assert m["position_ids"].tolist() == lit["position_ids"]
    assert m["write_pages"][:5].tolist() == [proposed[r][0] for r in lit["write_pages_rows"]]
    assert m["write_offsets"][:5].tolist() == lit["write_offsets_head"]
    assert len(m["last_page_len"]) == lit["last_page_len_count"]
    assert len(set(scratch)) == lit["unique_padding_pages"]
    assert len(set(m["kv_indices"][-2:].tolist())) == lit["unique_tail_indices"]
    padding = set(zip(m["write_pages"][5:].tolist(), m["write_offsets"][5:].tolist()))
    assert len(padding) == lit["unique_padding_writes"]
    assert not padding & set(zip(m["write_pages"][:5].tolist(), m["write_offsets"][:5].tolist()))


def test_decode_after_prefill_literals():
    lit = LITERALS["decode_after_prefill"]
    pool = lit["pool"]
    alloc = o_plan.Allocator(pool["total_pages"], pool["page_size"])
    scratch = alloc.claim_scratch(pool["scratch_page_count"])
    alloc.add("a")
    _, proposed = alloc.reserve(["a"], [lit["prefill_advance"]])
    alloc.publish("a", proposed[0], lit["prefill_advance"])
    st = alloc.states["a"]
    _, proposed = alloc.reserve(["a"], [1])
    m = o_plan.metadata([(st.sequence_length, st.position_start, proposed[0])], [1], capture_rows=2,
                        token_capacity=2, prefill=False, page_size=pool["page_size"], scratch_pages=scratch)
    assert m["position_ids"].tolist() == lit["position_ids"]
    assert int(m["write_offsets"][0]) == lit["write_offset0"]
    assert int(m["write_pages"][1]) == scratch[lit["padding_write_page_index"]]


def test_scratch_capacity_errors():
    lit = LITERALS["scratch_capacity_errors"]
    with pytest.raises(ValueError, match=lit["decode_error"]):
        o_plan.metadata([(0, 0, [5])], [1], capture_rows=2, token_capacity=2, prefill=False, page_size=4,
                        scratch_pages=[0])
    with pytest.raises(ValueError, match=lit["prefill_error"]):
        o_plan.metadata([(0, 0, [5])], [1], capture_rows=1, token_capacity=8, prefill=True, page_size=4,
                        scratch_pages=[0])


def test_allocator_literals():
    lit = LITERALS["allocator_publication"]
    a = o_plan.Allocator(lit["total_pages"], lit["page_size"])
    a.add("a")
    news, proposed = a.reserve(["a"], [lit["advance"]])
    assert len(proposed[0]) == lit["pages"]
    a.publish("a", proposed[0], lit["advance"])
    assert a.states["a"].sequence_length == lit["length_after_publish"]
    lit = LITERALS["allocator_rollback"]
    a = o_plan.Allocator(lit["total_pages"], lit["page_size"])
    a.add("a")
    a.add("b")
    with pytest.raises(MemoryError):
        a.reserve(["a", "b"], lit["advances"])
    assert len(a.free) == lit["free_after_failure"]
    lit = LITERALS["allocator_recycle"]
    a = o_plan.Allocator(lit["total_pages"], lit["page_size"])
    for i in range(lit["requests"]):
        a.add(f"r{i}")
        _, proposed = a.reserve([f"r{i}"], [lit["advance"]])
        a.publish(f"r{i}", proposed[0], lit["advance"])
        assert not a.free
        a.remove(f"r{i}")
        assert len(a.free) == lit["total_pages"]


def _simulate(rows, advances, page_size):
    """Independent statement: walk every token and look up which page/slot holds it."""

    out = []
    for (seq, pos0, pages), adv in zip(rows, advances):
        slots = [(p, s) for p in pages for s in range(page_size)]
        for off in range(adv):
            page, slot = slots[seq + off]
            out.append((page, slot, pos0 + off))
    return out


@pytest.mark.parametrize("seed,ps,prefill", [(0, 16, False), (1, 16, True), (2, 4, True), (3, 128, False)])
def test_metadata_agrees_with_token_walk(seed, ps, prefill):
    rng = np.random.default_rng(seed)
    n = 9
    prior = rng.integers(0, 200, size=n)
    adv = rng.integers(1, 40, size=n) if prefill else np.ones(n, dtype=np.int64)
    alloc, scratch, rids = o_plan.synthetic_batch(rng, n_rows=n, prior_lengths=prior, advances=adv,
                                                  total_pages=2048, page_size=ps, scratch_count=64)
    states = [alloc.states[r] for r in rids]
    news, proposed = alloc.reserve(rids, adv.tolist())
    rows = [(s.sequence_length, s.position_start, p) for s, p in zip(states, proposed)]
    cap = 12
    tokens = int(adv.sum()) + (0 if prefill else cap - n) + 3 if prefill else cap
    m = o_plan.metadata(rows, adv.tolist(), capture_rows=cap, token_capacity=tokens, prefill=prefill, page_size=ps,
                        scratch_pages=scratch)
    walk = _simulate(rows, adv.tolist(), ps)
    got = list(zip(m["write_pages"].tolist(), m["write_offsets"].tolist(), m["position_ids"].tolist()))
    assert got[: len(walk)] == walk
    # page lists: each row owns exactly ceil(len/ps) distinct pages, never shared
    indptr = m["kv_indptr"]
    real = [m["kv_indices"][indptr[r] : indptr[r + 1]].tolist() for r in range(n)]
    for r in range(n):
        assert len(real[r]) == -(-(int(prior[r]) + int(adv[r])) // ps)
    flat = [p for row in real for p in row]
    assert len(flat) == len(set(flat))
    # new pages are the lowest free pages, handed out in row order
    new_flat = [p for row in news for p in row]
    assert new_flat == sorted(new_flat)
    for r in range(n):
        total = int(prior[r] + adv[r])
        assert m["last_page_len"][r] == (total % ps or ps)
    # padding rows own their scratch page
    for r in range(n, cap):
        assert m["kv_indices"][indptr[r]] == scratch[r] and m["last_page_len"][r] == 1
