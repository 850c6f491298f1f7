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


def test_lowest_pages_in_row_order_and_epoch_tracking(nq):
    from nari_qwen3_tts_amd.cache import PagedKVAllocator

    a = PagedKVAllocator(total_pages=20, page_size=2)
    scratch = a.claim_scratch_pages(3)
    assert scratch == (0, 1, 2)
    for r in "abc":
        a.add_request(r)
    res = a.reserve(("a", "b", "c"), (3, 1, 4))
    assert [p.page_indices for p in res.publications] == [(3, 4), (5,), (6, 7)]
    assert res.pages_taken == 5
    epoch = a.free_list_epoch
    for p in res.publications:
        p.publish()
    assert a.free_list_epoch == epoch  # publishing returns nothing
    a.remove_request("b")
    assert a.free_list_epoch == epoch + 1
    assert a.free_list()[0] == 5


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
