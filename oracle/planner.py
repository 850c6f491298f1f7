"""Oracle for the ragged page-table planner (test infrastructure only).

Restates, with plain Python loops over small inputs:

- ``Allocator``: PagedKVAllocator (executor/cache.py:86-212) -- sorted free
  list, lowest free pages taken in row order (:153-162), publish/discard
  (:186-212), scratch pages claimed from the front (:103-112).
- ``metadata``: PagedTalkerKV._metadata (executor/talker_kv.py:403-483) --
  page lists, indptr, last_page_len, positions, write pages/offsets, padding
  rows (:442-452) and padding tokens (:453-457).

Pinned by tests/test_oracle_planner.py against the literal vectors of the
reference tests (tests/model_optimization/test_talker_kv_metadata.py:17-89,
tests/model_optimization/test_staging_cache_rng.py:75-136, kept as data in
tests/golden/reference_literals.json) and against an independent token-by-
token simulation.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass
class RequestState:
    pages: list[int] = field(default_factory=list)
    sequence_length: int = 0
    position_start: int = 0


class Allocator:
    """Host restatement of the reference allocator's page choice."""

    def __init__(self, total_pages: int, page_size: int) -> None:
        self.total_pages = total_pages
        self.page_size = page_size
        self.free = list(range(total_pages))
        self.states: dict[str, RequestState] = {}

    def claim_scratch(self, count: int) -> list[int]:
        pages = self.free[:count]
        del self.free[:count]
        return pages

    def add(self, rid: str) -> None:
        self.states[rid] = RequestState()

    def remove(self, rid: str) -> None:
        self.free.extend(self.states.pop(rid).pages)
        self.free.sort()

    def reserve(self, rids, advances):
        """Return (new_pages per row, proposed pages per row); raises on capacity."""

        taken: list[int] = []
        news, proposed = [], []
        for rid, adv in zip(rids, advances):
            st = self.states[rid]
            needed = -(-(st.sequence_length + adv) // self.page_size)
            missing = needed - len(st.pages)
            if missing > len(self.free):
                self.free.extend(taken)
                self.free.sort()
                raise MemoryError("not enough free pages")
            new = self.free[:missing]
            del self.free[:missing]
            taken.extend(new)
            news.append(new)
            proposed.append(st.pages + new)
        return news, proposed

    def publish(self, rid: str, proposed: list[int], advance: int) -> None:
        st = self.states[rid]
        st.pages = list(proposed)
        st.sequence_length += advance
        st.position_start += advance

    def discard(self, new_pages: list[int]) -> None:
        self.free.extend(new_pages)
        self.free.sort()


def metadata(
    rows: list[tuple[int, int, list[int]]],
    advances: list[int],
    *,
    capture_rows: int,
    token_capacity: int,
    prefill: bool,
    page_size: int,
    scratch_pages: list[int],
) -> dict[str, np.ndarray]:
    """Ragged metadata of one capture bucket.

    ``rows``: per real row (sequence_length, position_start, proposed pages),
    the pages already including the new ones (talker_kv.py:427-431).
    """

    if capture_rows > len(scratch_pages):
        raise ValueError("Talker CUDA Graph rows exceed executor-private scratch pages")
    if token_capacity > len(scratch_pages) * page_size:
        raise ValueError("Talker token capacity exceeds executor-private scratch slots")
    indptr = [0]
    indices: list[int] = []
    last: list[int] = []
    positions: list[int] = []
    wpages: list[int] = []
    woffs: list[int] = []
    qo = [0]
    for row in range(capture_rows):
        if row < len(rows):
            seq, pos0, pages = rows[row]
            adv = advances[row]
            total = seq + adv
            indices.extend(pages)
            indptr.append(len(indices))
            last.append(total % page_size or page_size)
            for off in range(adv):
                a = seq + off
                wpages.append(pages[a // page_size])
                woffs.append(a % page_size)
                positions.append(pos0 + off)
            if prefill:
                qo.append(qo[-1] + adv)
        else:
            scratch = scratch_pages[row]
            indices.append(scratch)
            indptr.append(len(indices))
            last.append(1)
            if prefill:
                qo.append(qo[-1])
            else:
                wpages.append(scratch)
                woffs.append(0)
                positions.append(0)
    sum_adv = sum(advances)
    while len(positions) < token_capacity:
        slot = len(positions) - sum_adv
        positions.append(0)
        wpages.append(scratch_pages[slot // page_size])
        woffs.append(slot % page_size)
    if len(positions) != token_capacity:
        raise ValueError("Talker KV metadata exceeds the captured token capacity")
    out = {
        "kv_indptr": np.asarray(indptr, dtype=np.int32),
        "kv_indices": np.asarray(indices, dtype=np.int32),
        "last_page_len": np.asarray(last, dtype=np.int32),
        "position_ids": np.asarray(positions, dtype=np.int64),
        "write_pages": np.asarray(wpages, dtype=np.int64),
        "write_offsets": np.asarray(woffs, dtype=np.int64),
    }
    if prefill:
        out["qo_indptr"] = np.asarray(qo, dtype=np.int32)
    return out


def synthetic_batch(
    rng: np.random.Generator,
    *,
    n_rows: int,
    prior_lengths: np.ndarray,
    advances: np.ndarray,
    total_pages: int,
    page_size: int,
    scratch_count: int,
    permute: bool = True,
):
    """Build an allocator whose requests already hold ``prior_lengths`` tokens.

    Prior pages come from a random permutation of the pool (the BASELINE
    "pages randomly permuted" condition); the remaining free list stays sorted.
    Returns (allocator, scratch_pages, request ids).
    """

    alloc = Allocator(total_pages, page_size)
    scratch = alloc.claim_scratch(scratch_count)
    pool = np.asarray(alloc.free, dtype=np.int64)
    if permute:
        pool = rng.permutation(pool)
    need = [-(-int(n) // page_size) for n in prior_lengths]
    if sum(need) > len(pool):
        raise ValueError("pool too small for the prior lengths")
    used = []
    at = 0
    rids = []
    for i in range(n_rows):
        rid = f"r{i}"
        alloc.add(rid)
        pages = [int(p) for p in pool[at : at + need[i]]]
        at += need[i]
        used.extend(pages)
        st = alloc.states[rid]
        st.pages = pages
        st.sequence_length = int(prior_lengths[i])
        st.position_start = int(prior_lengths[i])
        rids.append(rid)
    used_set = set(used)
    alloc.free = sorted(p for p in alloc.free if p not in used_set)
    return alloc, scratch, rids
