"""Host ledger of KV page ownership for the paged talker KV.

Every live request owns a ledger slot, a small integer that is also the request's row of the
device page table.  The committed numbers of each request (sequence length, RoPE position start,
page count) sit in numpy arrays indexed by slot, so the planner's per-row inputs are array
gathers; the page ids are kept as one tuple per request because the engine-facing proposal
carries them as a tuple.  The free pages are one sorted numpy array with a consumed front: a
reservation hands out the lowest free pages in row order by moving the front, a return inserts
the pages back in sorted position.

The device copy of the free list is not uploaded from here.  Every change to the free list is
also appended to an ordered log (pages taken from the front, sorted pages returned); the owner of
the device copy replays the log on the GPU before its next planner launch (front offset moves,
``nq_free_list_merge`` for returns), so both copies stay equal.

Contract kept from the reference allocator (executor/cache.py:43-212), with its messages: a
reservation is all-or-nothing and returns one pending publication per row; a publication becomes
the request's committed state only when published, and a discard gives its new pages back; a
publication whose request has since changed, or that was already published or discarded, is stale
(``StaleKVPublicationError``); a request with a reservation in flight can neither reserve again
nor be removed (``SlotBusyError``); running out of pages raises ``KVAllocationError`` before
anything is taken.
"""

from __future__ import annotations

import heapq
from dataclasses import dataclass

import numpy as np

from .errors import KVAllocationError, SlotBusyError, StaleKVPublicationError

_STALE = "Talker KV publication is stale or no longer pending"
# reservations of at most this many rows count their pages in plain integers, larger ones in numpy
_SMALL_RESERVATION = 32


@dataclass(frozen=True, slots=True)
class RequestKVState:
    """Committed KV of one request (field names of executor/cache.py:25-31)."""

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


class _ReservedRows:
    """What one reservation decided, shared by its rows' publications (row i of each field)."""

    __slots__ = ("ledger", "request_ids", "serial", "priors", "taken", "lo", "hi", "advances")

    def __init__(self, ledger, request_ids, serial, priors, taken, lo, hi, advances) -> None:
        self.ledger, self.request_ids, self.serial, self.priors = ledger, request_ids, serial, priors
        self.taken, self.lo, self.hi, self.advances = taken, lo, hi, advances


class PendingKVPublication:
    """One row of a reservation: publish() commits it, discard() gives its new pages back.  The
    ledger keeps this object as the request's in-flight entry; it stays live while it is that
    entry and the request's committed state is still the one it was made against.  The row's
    fields (request_id, token, prior_version, sequence_advance, page_indices) are read from the
    reservation it belongs to."""

    __slots__ = ("_rows", "_i", "_pages")

    def __init__(self, rows: _ReservedRows, i: int) -> None:
        self._rows = rows
        self._i = i
        self._pages: tuple[int, ...] | None = None

    @property
    def _ledger(self) -> "PagedKVAllocator":
        return self._rows.ledger

    @property
    def request_id(self) -> str:
        return self._rows.request_ids[self._i]

    @property
    def token(self) -> int:
        return self._rows.serial + self._i + 1

    @property
    def _prior(self) -> RequestKVState:
        return self._rows.priors[self._i]

    @property
    def prior_version(self) -> int:
        return self._rows.priors[self._i].version

    @property
    def sequence_advance(self) -> int:
        return self._rows.advances[self._i]

    _advance = sequence_advance

    @property
    def new_pages(self) -> np.ndarray:
        r = self._rows
        return r.taken[r.lo[self._i]: r.hi[self._i]]

    @property
    def page_indices(self) -> tuple[int, ...]:
        """The request's pages if published: its committed pages, then the new ones."""

        if self._pages is None:
            r, i = self._rows, self._i
            lo, hi = r.lo[i], r.hi[i]
            prior = r.priors[i].page_indices
            self._pages = prior if lo == hi else prior + tuple(r.taken[lo:hi].tolist())
        return self._pages

    def proposal(self) -> KVPublicationProposal:
        current = self._ledger.state(self.request_id)
        return KVPublicationProposal(self.request_id, self.page_indices, current.sequence_length + self.sequence_advance)

    def validate(self) -> None:
        self._ledger._live(self)

    def publish(self) -> None:
        self._ledger._settle(self, commit=True)

    def discard(self) -> None:
        self._ledger._settle(self, commit=False)

    def __repr__(self) -> str:
        return f"PendingKVPublication({self.request_id!r}, token={self.token}, advance={self.sequence_advance})"


@dataclass(frozen=True, slots=True)
class KVReservation:
    publications: tuple[PendingKVPublication, ...]
    pages_taken: int = 0
    # the pages taken from the front of the free list, in row order (what the device planner must take)
    taken: np.ndarray | None = None


class PagedKVAllocator:
    """Fixed-capacity page ledger; no scheduling, no transfers, no device memory."""

    def __init__(self, *, total_pages: int, page_size: int) -> None:
        if total_pages < 1 or page_size < 1:
            raise ValueError("paged KV capacity must be positive")
        self.total_pages = total_pages
        self.page_size = page_size
        self._free = np.arange(total_pages, dtype=np.int32)
        self._front = 0
        self._states: dict[str, RequestKVState] = {}
        self._slot_of: dict[str, int] = {}
        self._spare: list[int] = []
        self._capacity = 0
        self.length = np.zeros(0, dtype=np.int32)
        self.position = np.zeros(0, dtype=np.int32)
        self.page_count = np.zeros(0, dtype=np.int32)
        self._grow(64)
        self._inflight: dict[str, PendingKVPublication] = {}
        self._serial = 0
        # ordered changes of the free list the device copy has not seen: ("take", n) / ("return", pages)
        self._log: list[tuple[str, object]] = []
        self._returning: list[np.ndarray] = []
        # set when the free list changed in a way the log does not describe (device copy must be re-sent)
        self.resend_free_list = False

    # -- capacity --------------------------------------------------------------
    def _grow(self, capacity: int) -> None:
        for name in ("length", "position", "page_count"):
            old = getattr(self, name)
            grown = np.zeros(capacity, dtype=np.int32)
            grown[: old.shape[0]] = old
            setattr(self, name, grown)
        heapq.heapify(self._spare)
        for slot in range(self._capacity, capacity):
            heapq.heappush(self._spare, slot)
        self._capacity = capacity

    @property
    def slot_capacity(self) -> int:
        return self._capacity

    @property
    def free_pages(self) -> int:
        self._merge_returns()
        return int(self._free.shape[0] - self._front)

    def free_list(self) -> tuple[int, ...]:
        self._merge_returns()
        return tuple(self._free[self._front:].tolist())

    def free_array(self) -> np.ndarray:
        """The sorted free pages (a read-only view)."""

        self._merge_returns()
        view = self._free[self._front:]
        view.flags.writeable = False
        return view

    def _take_front(self, count: int) -> np.ndarray:
        self._merge_returns()
        # a copy: the consumed front of the array is reused when pages below it come back
        taken = self._free[self._front: self._front + count].copy()
        self._front += count
        if count:
            self._log.append(("take", count))
        return taken

    def _give_back(self, pages: np.ndarray) -> None:
        """Queue pages for return; they join the free list (in one merge) before it is next read."""

        if pages.shape[0]:
            self._returning.append(pages)

    def _merge_returns(self) -> None:
        if not self._returning:
            return
        ret = self._returning[0] if len(self._returning) == 1 else np.concatenate(self._returning)
        self._returning = []
        ret = np.sort(ret.astype(np.int32, copy=False))
        m = ret.shape[0]
        if m > 1 and np.any(ret[1:] == ret[:-1]):
            raise RuntimeError("a KV page was returned while already free")
        live = self._free[self._front:]
        if m <= self._front and (live.shape[0] == 0 or ret[-1] < live[0]):
            # every returned page sorts below the free list (a discard of recent reservations, which
            # took the lowest pages): they go back into the consumed front, no copy of the list
            self._front -= m
            self._free[self._front: self._front + m] = ret
        else:
            at = np.searchsorted(live, ret)
            if live.shape[0] and np.any(live[np.minimum(at, live.shape[0] - 1)] == ret):
                raise RuntimeError("a KV page was returned while already free")
            self._free = np.insert(live, at, ret)
            self._front = 0
        self._log.append(("return", ret))

    def has_log(self) -> bool:
        """Whether the free list changed since the last drain (taken pages or pending returns)."""

        return bool(self._log or self._returning)

    def drain_log(self) -> list[tuple[str, object]]:
        """The free-list changes since the last drain, in order (for the device copy)."""

        self._merge_returns()
        log, self._log = self._log, []
        return log

    def claim_scratch_pages(self, count: int) -> tuple[int, ...]:
        if isinstance(count, bool) or not isinstance(count, int) or count < 1:
            raise ValueError("scratch page count must be a positive integer")
        if count > self.free_pages:
            raise KVAllocationError(f"cannot reserve {count} Talker scratch pages")
        return tuple(self._take_front(count).tolist())

    # -- requests --------------------------------------------------------------
    def add_request(self, request_id: str) -> None:
        if not isinstance(request_id, str) or not request_id:
            raise ValueError("request_id must be a non-empty string")
        if request_id in self._states:
            raise ValueError(f"request {request_id!r} already owns KV state")
        if not self._spare:
            self._grow(2 * self._capacity)
        slot = heapq.heappop(self._spare)
        self.length[slot] = self.position[slot] = self.page_count[slot] = 0
        self._slot_of[request_id] = slot
        self._states[request_id] = RequestKVState(request_id)

    def slot(self, request_id: str) -> int:
        """The request's ledger slot (its row of the device page table)."""

        slot = self._slot_of.get(request_id)
        if slot is None:
            raise KeyError(f"unknown Talker KV request {request_id!r}")
        return slot

    def state(self, request_id: str) -> RequestKVState:
        state = self._states.get(request_id)
        if state is None:
            raise KeyError(f"unknown Talker KV request {request_id!r}")
        return state

    def remove_request(self, request_id: str) -> None:
        if request_id in self._inflight:
            raise SlotBusyError(f"request {request_id!r} KV is in flight")
        state = self.state(request_id)
        self._give_back(np.asarray(state.page_indices, dtype=np.int32))
        del self._states[request_id]
        heapq.heappush(self._spare, self._slot_of.pop(request_id))

    def adopt(self, request_id: str, pages: tuple[int, ...], sequence_length: int, position_start: int) -> None:
        """Install a committed state that owns ``pages`` (benchmark and test setup).

        Lets a workload start from pages scattered over the pool, which the lowest-free-page policy
        never produces by itself; the device copy of the free list is then re-sent once.
        """

        state = self.state(request_id)
        if state.page_indices or request_id in self._inflight:
            raise ValueError(f"request {request_id!r} already owns pages")
        if len(pages) != -(-sequence_length // self.page_size):
            raise ValueError("adopted pages do not match the sequence length")
        want = np.asarray(pages, dtype=np.int32)
        self._merge_returns()
        live = self._free[self._front:]
        if np.unique(want).shape[0] != want.shape[0] or not np.isin(want, live).all():
            raise KVAllocationError("adopted pages must be distinct free pages")
        self._free = live[~np.isin(live, want)]
        self._front = 0
        self.resend_free_list = True
        self._log.clear()
        slot = self._slot_of[request_id]
        self.length[slot], self.position[slot], self.page_count[slot] = sequence_length, position_start, len(pages)
        self._states[request_id] = RequestKVState(request_id, tuple(int(p) for p in pages), sequence_length,
                                                  position_start, state.version + 1)

    # -- reservations ----------------------------------------------------------
    def slots(self, request_ids: tuple[str, ...]) -> np.ndarray:
        try:
            return np.fromiter(map(self._slot_of.__getitem__, request_ids), dtype=np.int64, count=len(request_ids))
        except KeyError as missing:
            raise KeyError(f"unknown Talker KV request {missing.args[0]!r}") from None

    def reserve(self, request_ids: tuple[str, ...], advances: tuple[int, ...],
                slots: np.ndarray | None = None) -> KVReservation:
        """``slots``: the rows' ledger slots when the caller has already looked them up."""

        rows = len(request_ids)
        if not rows or rows != len(advances):
            raise ValueError("KV reservation rows must be non-empty and aligned")
        if len(set(request_ids)) != rows:
            raise ValueError("KV reservation request rows must be unique")
        if slots is None:
            slots = self.slots(request_ids)
        if not self._inflight.keys().isdisjoint(request_ids):
            busy = next(r for r in request_ids if r in self._inflight)
            raise SlotBusyError(f"request {busy!r} KV is already in flight")
        if not set(map(type, advances)) <= {int} or min(advances) < 1:
            raise ValueError("KV sequence advances must be positive integers")
        ps = self.page_size
        available = self.free_pages
        if rows <= _SMALL_RESERVATION:
            # per-row page counts in plain integers (for a few rows numpy's per-call cost dominates)
            lo, hi, total = [], [], 0
            for length, count, a in zip(self.length[slots].tolist(), self.page_count[slots].tolist(), advances):
                lo.append(total)
                n = (length + a + ps - 1) // ps - count
                if n > 0:
                    total += n
                hi.append(total)
            end_total = total
        else:
            adv = np.asarray(advances, dtype=np.int64)
            need = (self.length[slots] + adv + ps - 1) // ps - self.page_count[slots]
            np.maximum(need, 0, out=need)
            end = np.cumsum(need)
            lo, hi, end_total = (end - need).tolist(), end.tolist(), int(end[-1])
        if end_total > available:
            k = next(r for r in range(rows) if hi[r] > available)
            raise KVAllocationError(f"Talker KV needs {hi[k] - lo[k]} pages for {request_ids[k]!r}, only "
                                    f"{available - lo[k]} remain")
        taken = self._take_front(end_total)
        serial = self._serial
        self._serial += rows
        states = self._states
        batch = _ReservedRows(self, tuple(request_ids), serial, [states[rid] for rid in request_ids], taken, lo, hi,
                              tuple(advances))
        publications = tuple(map(PendingKVPublication, [batch] * rows, range(rows)))
        self._inflight.update(zip(request_ids, publications))
        return KVReservation(publications, end_total, taken)

    def _live(self, publication: PendingKVPublication) -> None:
        """StaleKVPublicationError unless ``publication`` is its request's in-flight entry and the
        request's committed state is still the one the reservation was made against."""

        rows, i = publication._rows, publication._i
        rid = rows.request_ids[i]
        if self._inflight.get(rid) is not publication or self._states.get(rid) is not rows.priors[i]:
            raise StaleKVPublicationError(_STALE)

    def discard_all(self, publications) -> None:
        """Discard each publication in order, as ``discard()`` on each would (a stale one raises
        after the ones before it are discarded); the pages of consecutive rows of one reservation
        go back in one piece."""

        inflight, states = self._inflight, self._states
        run, lo, hi = None, 0, 0
        try:
            for publication in publications:
                rows, i = publication._rows, publication._i
                rid = rows.request_ids[i]
                if inflight.get(rid) is not publication or states.get(rid) is not rows.priors[i]:
                    raise StaleKVPublicationError(_STALE)
                del inflight[rid]
                if rows is run and rows.lo[i] == hi:
                    hi = rows.hi[i]
                    continue
                if run is not None and hi > lo:
                    self._give_back(run.taken[lo:hi])
                run, lo, hi = rows, rows.lo[i], rows.hi[i]
        finally:
            if run is not None and hi > lo:
                self._give_back(run.taken[lo:hi])

    def _settle(self, publication: PendingKVPublication, *, commit: bool) -> None:
        # the row's fields read straight from its reservation (the properties' values): this runs
        # once per row of every decode step
        rows, i = publication._rows, publication._i
        rid, prior = rows.request_ids[i], rows.priors[i]
        inflight = self._inflight
        if inflight.get(rid) is not publication or self._states.get(rid) is not prior:
            raise StaleKVPublicationError(_STALE)
        del inflight[rid]
        lo, hi = rows.lo[i], rows.hi[i]
        if not commit:
            self._give_back(rows.taken[lo:hi])
            return
        pages = publication._pages
        if pages is None:
            pages = prior.page_indices if lo == hi else prior.page_indices + tuple(rows.taken[lo:hi].tolist())
        advance = rows.advances[i]
        length, position = prior.sequence_length + advance, prior.position_start + advance
        slot = self._slot_of[rid]
        self.length[slot] = length
        self.position[slot] = position
        self.page_count[slot] = len(pages)
        self._states[rid] = RequestKVState(rid, pages, length, position, prior.version + 1)


__all__ = [
    "KVAllocationError",
    "KVPublicationProposal",
    "KVReservation",
    "PagedKVAllocator",
    "PendingKVPublication",
    "RequestKVState",
    "StaleKVPublicationError",
]
