"""Host-side page ownership with pending / publish / discard KV transactions.

Mirrors the behaviour of the reference allocator (executor/cache.py:19-212):
a sorted free list whose lowest pages are handed out in row order (:153-162),
publications that become the request's committed state only on publish
(:186-207), discards that return the proposed new pages (:208-211), stale
publications rejected with StaleKVPublicationError (:62-75), rollback of a
failed multi-row reservation (:178-183).

On top of that, the allocator counts how many free pages a reservation took
from the front of the free list and flags when pages came back, so the
device copy of the free list (read by the GPU planner) can follow it with an
upload only when pages are returned.
"""

from __future__ import annotations

import bisect
from dataclasses import dataclass

from .errors import KVAllocationError, SlotBusyError, StaleKVPublicationError


@dataclass(frozen=True, slots=True)
class RequestKVState:
    request_id: str
    page_indices: tuple[int, ...] = ()
    sequence_length: int = 0
    position_start: int = 0
    version: int = 0


@dataclass(frozen=True, slots=True)
class KVPublicationProposal:
    """Engine-facing view of a pending publication (contract/result.py KVPublication)."""

    request_id: str
    pages: tuple[int, ...]
    length: int


@dataclass(slots=True)
class _Pending:
    token: int
    prior: RequestKVState
    proposed_pages: tuple[int, ...]
    new_pages: tuple[int, ...]
    sequence_advance: int
    status: str = "pending"


@dataclass(slots=True)
class PendingKVPublication:
    _allocator: "PagedKVAllocator"
    request_id: str
    token: int
    prior_version: int
    page_indices: tuple[int, ...]
    sequence_advance: int

    def proposal(self) -> KVPublicationProposal:
        current = self._allocator.state(self.request_id)
        return KVPublicationProposal(self.request_id, self.page_indices, current.sequence_length + self.sequence_advance)

    def validate(self) -> None:
        self._allocator._check_live(self)
        if self.sequence_advance < 1:
            raise StaleKVPublicationError("Talker KV publication is stale or no longer pending")

    def publish(self) -> None:
        self.validate()
        self._allocator._finish(self, publish=True)

    def discard(self) -> None:
        self.validate()
        self._allocator._finish(self, publish=False)


@dataclass(frozen=True, slots=True)
class KVReservation:
    publications: tuple[PendingKVPublication, ...]
    pages_taken: int = 0


class PagedKVAllocator:
    """Fixed-capacity page allocator; no scheduling, no transfers."""

    def __init__(self, *, total_pages: int, page_size: int) -> None:
        if total_pages < 1 or page_size < 1:
            raise ValueError("paged KV capacity must be positive")
        self.total_pages = total_pages
        self.page_size = page_size
        self._free: list[int] = list(range(total_pages))
        self._states: dict[str, RequestKVState] = {}
        self._pending: dict[str, _Pending] = {}
        self._tokens = 0
        # Incremented whenever pages return to the free list (device copy is stale).
        self.free_list_epoch = 0

    @property
    def free_pages(self) -> int:
        return len(self._free)

    def free_list(self) -> tuple[int, ...]:
        return tuple(self._free)

    def claim_scratch_pages(self, count: int) -> tuple[int, ...]:
        if isinstance(count, bool) or not isinstance(count, int) or count < 1:
            raise ValueError("scratch page count must be a positive integer")
        if count > len(self._free):
            raise KVAllocationError(f"cannot reserve {count} Talker scratch pages")
        taken = tuple(self._free[:count])
        self._free = self._free[count:]
        self.free_list_epoch += 1
        return taken

    def add_request(self, request_id: str) -> None:
        if not isinstance(request_id, str) or not request_id:
            raise ValueError("request_id must be a non-empty string")
        if request_id in self._states:
            raise ValueError(f"request {request_id!r} already owns KV state")
        self._states[request_id] = RequestKVState(request_id)

    def state(self, request_id: str) -> RequestKVState:
        state = self._states.get(request_id)
        if state is None:
            raise KeyError(f"unknown Talker KV request {request_id!r}")
        return state

    def remove_request(self, request_id: str) -> None:
        if request_id in self._pending:
            raise SlotBusyError(f"request {request_id!r} KV is in flight")
        state = self.state(request_id)
        self._return_pages(state.page_indices)
        del self._states[request_id]

    def adopt(self, request_id: str, pages: tuple[int, ...], sequence_length: int, position_start: int) -> None:
        """Install a committed state that owns ``pages`` (benchmark and test setup).

        Lets a workload start from pages scattered over the pool, which the
        lowest-free-page policy never produces by itself.
        """

        state = self.state(request_id)
        if state.page_indices or request_id in self._pending:
            raise ValueError(f"request {request_id!r} already owns pages")
        needed = -(-sequence_length // self.page_size)
        if len(pages) != needed:
            raise ValueError("adopted pages do not match the sequence length")
        free = set(self._free)
        if len(set(pages)) != len(pages) or any(p not in free for p in pages):
            raise KVAllocationError("adopted pages must be distinct free pages")
        taken = set(pages)
        self._free = [p for p in self._free if p not in taken]
        self.free_list_epoch += 1
        self._states[request_id] = RequestKVState(
            request_id, tuple(pages), sequence_length, position_start, state.version + 1
        )

    def _return_pages(self, pages) -> None:
        if not pages:
            return
        for page in pages:
            bisect.insort(self._free, page)
        self.free_list_epoch += 1

    def reserve(self, request_ids: tuple[str, ...], advances: tuple[int, ...]) -> KVReservation:
        if not request_ids or len(request_ids) != len(advances):
            raise ValueError("KV reservation rows must be non-empty and aligned")
        if len(set(request_ids)) != len(request_ids):
            raise ValueError("KV reservation request rows must be unique")
        states = [self.state(rid) for rid in request_ids]
        for rid, advance in zip(request_ids, advances):
            if rid in self._pending:
                raise SlotBusyError(f"request {rid!r} KV is already in flight")
            if isinstance(advance, bool) or not isinstance(advance, int) or advance < 1:
                raise ValueError("KV sequence advances must be positive integers")
        # Page demand of every row first, so a failure leaves nothing behind.
        missing = []
        for rid, state, advance in zip(request_ids, states, advances):
            needed = -(-(state.sequence_length + advance) // self.page_size)
            missing.append(needed - len(state.page_indices))
        taken = 0
        for rid, miss in zip(request_ids, missing):
            if miss > len(self._free) - taken:
                raise KVAllocationError(
                    f"Talker KV needs {miss} pages for {rid!r}, only {len(self._free) - taken} remain"
                )
            taken += max(miss, 0)
        publications = []
        cursor = 0
        for rid, state, advance, miss in zip(request_ids, states, advances, missing):
            new = tuple(self._free[cursor : cursor + max(miss, 0)])
            cursor += len(new)
            self._tokens += 1
            proposed = state.page_indices + new
            self._pending[rid] = _Pending(self._tokens, state, proposed, new, advance)
            publications.append(
                PendingKVPublication(self, rid, self._tokens, state.version, proposed, advance)
            )
        self._free = self._free[cursor:]
        return KVReservation(tuple(publications), cursor)

    def _check_live(self, publication: PendingKVPublication) -> _Pending:
        pending = self._pending.get(publication.request_id)
        current = self._states.get(publication.request_id)
        if (
            pending is None
            or current is None
            or pending.status != "pending"
            or pending.token != publication.token
            or pending.prior.version != publication.prior_version
            or current != pending.prior
            or pending.proposed_pages != publication.page_indices
        ):
            raise StaleKVPublicationError("Talker KV publication is stale or no longer pending")
        return pending

    def _finish(self, publication: PendingKVPublication, *, publish: bool) -> None:
        pending = self._check_live(publication)
        current = self._states[publication.request_id]
        if publish:
            self._states[publication.request_id] = RequestKVState(
                request_id=publication.request_id,
                page_indices=pending.proposed_pages,
                sequence_length=current.sequence_length + pending.sequence_advance,
                position_start=current.position_start + pending.sequence_advance,
                version=current.version + 1,
            )
            pending.status = "published"
        else:
            self._return_pages(pending.new_pages)
            pending.status = "discarded"
        del self._pending[publication.request_id]


__all__ = [
    "KVAllocationError",
    "KVPublicationProposal",
    "KVReservation",
    "PagedKVAllocator",
    "PendingKVPublication",
    "RequestKVState",
    "StaleKVPublicationError",
]
