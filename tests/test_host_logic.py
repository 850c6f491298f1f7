"""Host-side logic of the product package that needs no GPU: allocator transactions, bucket lowering."""

from __future__ import annotations

import json
from pathlib import Path

import pytest

LITERALS = json.loads((Path(__file__).parent / "golden" / "reference_literals.json").read_text())


def test_publication_is_pending_stale_safe_and_discardable(nq):
    from nari_qwen3_tts_amd.cache import PagedKVAllocator, StaleKVPublicationError

    lit = LITERALS["allocator_publication"]
    a = PagedKVAllocator(total_pages=lit["total_pages"], page_size=lit["page_size"])
    a.add_request("a")
    pub = a.reserve(("a",), (lit["advance"],)).publications[0]
    assert a.state("a").sequence_length == 0
    assert len(pub.page_indices) == lit["pages"]
    assert pub.proposal().length == lit["advance"]
    pub.publish()
    assert a.state("a").sequence_length == lit["length_after_publish"]
    assert a.state("a").version == lit["version_after_publish"]
    with pytest.raises(StaleKVPublicationError):
        pub.publish()
    discarded = a.reserve(("a",), (1,)).publications[0]
    discarded.discard()
    assert a.state("a").sequence_length == lit["length_after_publish"]
    with pytest.raises(StaleKVPublicationError):
        discarded.publish()


def test_duplicate_rows_and_inflight_aliasing(nq):
    from nari_qwen3_tts_amd.cache import PagedKVAllocator
    from nari_qwen3_tts_amd.errors import SlotBusyError

    a = PagedKVAllocator(total_pages=12, page_size=4)
    a.add_request("a")
    a.add_request("b")
    with pytest.raises(ValueError, match="unique"):
        a.reserve(("a", "a"), (1, 1))
    res = a.reserve(("a", "b"), (1, 2))
    with pytest.raises(SlotBusyError, match="in flight"):
        a.reserve(("a",), (1,))
    with pytest.raises(SlotBusyError):
        a.remove_request("a")
    for pub in res.publications:
        pub.discard()


def test_failed_multirow_reservation_rolls_back(nq):
    from nari_qwen3_tts_amd.cache import PagedKVAllocator
    from nari_qwen3_tts_amd.errors import KVAllocationError

    lit = LITERALS["allocator_rollback"]
    a = PagedKVAllocator(total_pages=lit["total_pages"], page_size=lit["page_size"])
    a.add_request("a")
    a.add_request("b")
    with pytest.raises(KVAllocationError):
        a.reserve(("a", "b"), tuple(lit["advances"]))
    assert a.free_pages == lit["free_after_failure"]
    successor = a.reserve(("b",), (lit["retry_advance"],))
    successor.publications[0].discard()
    assert a.free_pages == lit["free_after_failure"]


def test_capacity_recycles_across_more_requests_than_pages(nq):
    from nari_qwen3_tts_amd.cache import PagedKVAllocator

    lit = LITERALS["allocator_recycle"]
    a = PagedKVAllocator(total_pages=lit["total_pages"], page_size=lit["page_size"])
    for i in range(lit["requests"]):
        a.add_request(f"r{i}")
        a.reserve((f"r{i}",), (lit["advance"],)).publications[0].publish()
        assert a.free_pages == 0
        a.remove_request(f"r{i}")
        assert a.free_pages == lit["total_pages"]


def test_lowest_pages_in_row_order_and_free_list_log(nq):
    """Reservations take the lowest free pages in row order; every change of the free list is logged
    in order (takes, sorted returns) for the device copy to replay."""
    from nari_qwen3_tts_amd.cache import PagedKVAllocator

    a = PagedKVAllocator(total_pages=20, page_size=2)
    scratch = a.claim_scratch_pages(3)
    assert scratch == (0, 1, 2)
    for r in "abc":
        a.add_request(r)
    a.drain_log()
    res = a.reserve(("a", "b", "c"), (3, 1, 4))
    assert [p.page_indices for p in res.publications] == [(3, 4), (5,), (6, 7)]
    assert res.pages_taken == 5
    for p in res.publications:
        p.publish()
    assert a.drain_log() == [("take", 5)]  # publishing returns nothing
    a.remove_request("b")
    res = a.reserve(("c",), (2,))
    res.publications[0].discard()
    log = a.drain_log()
    assert [k for k, _ in log] == ["return", "take", "return"]
    assert log[0][1].tolist() == [5] and log[1][1] == 1 and log[2][1].tolist() == [5]
    assert a.free_list()[0] == 5
    # the slots of removed requests are reused lowest first
    assert a.slot("a") == 0 and a.slot("c") == 2
    a.add_request("d")
    assert a.slot("d") == 1


def test_free_list_log_replayed_on_a_copy_equals_the_ledger(nq):
    """Replaying the log (front moves, sorted merges) on a second array reproduces the ledger's
    free list exactly, over random reserve / publish / discard / remove traffic."""
    import numpy as np

    from nari_qwen3_tts_amd.cache import PagedKVAllocator

    rng = np.random.default_rng(3)
    a = PagedKVAllocator(total_pages=300, page_size=4)
    a.claim_scratch_pages(4)
    copy, front = np.asarray(a.free_list(), dtype=np.int32), 0
    a.drain_log()
    live = []
    for step in range(200):
        if len(live) < 12 and rng.random() < 0.5:
            rid = f"r{step}"
            a.add_request(rid)
            live.append(rid)
        if live:
            rows = tuple(rng.choice(live, size=min(len(live), int(rng.integers(1, 6))), replace=False).tolist())
            try:
                pubs = a.reserve(rows, tuple(int(x) for x in rng.integers(1, 9, size=len(rows)))).publications
            except Exception:  # noqa: BLE001 - pool exhausted: nothing taken
                pubs = ()
            for p in pubs:
                (p.publish if rng.random() < 0.7 else p.discard)()
            if rng.random() < 0.2:
                a.remove_request(live.pop(int(rng.integers(len(live)))))
        for kind, value in a.drain_log():
            if kind == "take":
                front += value
            else:
                rest = copy[front:]
                copy = np.sort(np.concatenate([rest, value]))  # a different formulation of the merge
                front = 0
        assert copy[front:].tolist() == list(a.free_list())


def test_adopt_installs_scattered_pages(nq):
    from nari_qwen3_tts_amd.cache import PagedKVAllocator
    from nari_qwen3_tts_amd.errors import KVAllocationError

    a = PagedKVAllocator(total_pages=16, page_size=4)
    a.add_request("a")
    a.adopt("a", (9, 3, 12), 10, 10)
    assert a.state("a").page_indices == (9, 3, 12)
    assert 9 not in a.free_list()
    a.add_request("b")
    with pytest.raises(KVAllocationError):
        a.adopt("b", (9,), 2, 2)
    pub = a.reserve(("a",), (3,)).publications[0]
    assert pub.page_indices == (9, 3, 12, 0)


def test_bucket_lowering_literal(nq):
    from nari_qwen3_tts_amd.graphs import lower_rows

    lit = LITERALS["bucket_lowering"]
    parts = lower_rows(lit["logical_rows"], tuple(lit["buckets"]))
    assert [[p.logical_rows, p.capture_rows, p.padding] for p in parts] == lit["expected"]
    with pytest.raises(ValueError):
        lower_rows(0, (1, 2))


def test_product_fails_loudly_without_gpu_tensors(nq):
    import torch

    from nari_qwen3_tts_amd.sampling import sample_with_uniforms

    cpu = torch.zeros(2, 8)
    with pytest.raises(ValueError, match="GPU"):
        sample_with_uniforms(cpu, torch.zeros(2), torch.ones(2, dtype=torch.int32), torch.ones(2), torch.zeros(2))


def test_slot_leases_fail_closed(nq):
    from nari_qwen3_tts_amd.errors import SlotBusyError
    from nari_qwen3_tts_amd.graphs import SlotLeases

    leases = SlotLeases()
    first = leases.reserve()
    assert not leases.available
    with pytest.raises(SlotBusyError, match="in flight"):
        leases.reserve()
    with pytest.raises(SlotBusyError, match="stale"):
        leases.release(first + 1)
    leases.release(first)
    second = leases.reserve()
    assert second != first
    leases.release(second)
    with pytest.raises(SlotBusyError):
        leases.release(second)


@pytest.mark.parametrize("rows", [3, 40])
def test_reservation_counts_pages_alike_for_few_and_many_rows(nq, monkeypatch, rows):
    """Reservations of a few rows count their new pages in plain integers, larger ones in numpy:
    both give the same pages per row, the same committed states and the same error message."""

    import numpy as np

    from nari_qwen3_tts_amd import cache
    from nari_qwen3_tts_amd.errors import KVAllocationError

    rng = np.random.default_rng(rows)
    prior = rng.integers(0, 70, size=rows).tolist()
    advances = tuple(int(x) for x in rng.integers(1, 40, size=rows))

    def run(small: int):
        monkeypatch.setattr(cache, "_SMALL_RESERVATION", small)
        a = cache.PagedKVAllocator(total_pages=4096, page_size=16)
        rids = tuple(f"r{i}" for i in range(rows))
        for rid, n in zip(rids, prior):
            a.add_request(rid)
            if n:
                a.reserve((rid,), (n,)).publications[0].publish()
        res = a.reserve(rids, advances)
        pages = [tuple(p.new_pages.tolist()) for p in res.publications]
        for p in res.publications:
            p.publish()
        states = [a.state(rid) for rid in rids]
        with pytest.raises(KVAllocationError) as err:
            a.reserve(rids, tuple(16 * a.free_pages for _ in rids))  # every free page per row, or more
        return res.pages_taken, pages, states, str(err.value)

    plain, numeric = run(10**6), run(0)
    assert plain == numeric
    assert plain[0] == sum(len(p) for p in plain[1]) > 0
