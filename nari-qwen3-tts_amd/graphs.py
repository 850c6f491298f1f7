"""hipGraph capture of fixed-shape buckets (the reference's CaptureDriver protocol).

``HipGraphCaptureDriver.capture(operation, after_warmup=None)`` runs the
operation eagerly twice, then records it into a graph sharing one memory
pool, and returns a call whose ``replay()`` launches the graph and returns
the static outputs (executor/cuda_graph.py:15-77).  PyTorch-ROCm's graph
object is a hipGraph; the HIP kernels launch on the capturing stream and
issue no memset/memcpy nodes.  ``lower_rows`` splits a logical batch over
the capture buckets as planner/catalog.py:43-71 does; ``SlotLeases`` and
``GraphPoolFence`` are the slot and shared-pool guards of
executor/cuda_graph.py:111-185.
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass
from threading import Lock

import torch

from .errors import SlotBusyError


@dataclass(slots=True)
class CapturedCall:
    graph: torch.cuda.CUDAGraph
    output: object

    def replay(self):
        self.graph.replay()
        return self.output


class HipGraphCaptureDriver:
    def __init__(self, *, device: torch.device, memory_pool=None, warmups: int = 2) -> None:
        if torch.device(device).type != "cuda" or not torch.cuda.is_available():
            raise RuntimeError("captured execution requires a GPU")
        self.device = torch.device(device)
        self.memory_pool = memory_pool or torch.cuda.graphs.graph_pool_handle()
        self.warmups = warmups

    def capture(self, operation: Callable[[], object], *, after_warmup: Callable[[], None] | None = None) -> CapturedCall:
        torch.cuda.set_device(self.device)
        torch.cuda.synchronize(self.device)
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            for _ in range(self.warmups):
                operation()
                if after_warmup is not None:
                    after_warmup()
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self.memory_pool):
            output = operation()
        torch.cuda.synchronize(self.device)
        return CapturedCall(graph, output)


class SlotLeases:
    """Exclusive use of one captured slot's static buffers (executor/cuda_graph.py:111-137): a slot is
    taken by ``reserve()`` and given back by ``release(ticket)`` with the ticket it got; taking a busy
    slot or giving back with a stale ticket raises SlotBusyError."""

    __slots__ = ("_holder", "_count")

    def __init__(self) -> None:
        self._holder: int | None = None
        self._count = 0

    @property
    def available(self) -> bool:
        return self._holder is None

    def reserve(self) -> int:
        if self._holder is not None:
            raise SlotBusyError("static CUDA Graph slot is in flight")
        self._count += 1
        self._holder = self._count
        return self._count

    def release(self, ticket: int) -> None:
        if self._holder is None or self._holder != ticket:
            raise SlotBusyError("stale or unowned static CUDA Graph slot lease")
        self._holder = None


class GraphPoolFence:
    """One submission at a time over graphs that share a memory pool (executor/cuda_graph.py:140-185):
    a second submission while one is open raises SlotBusyError instead of waiting, and each submission
    starts behind the GPU work the previous one enqueued (an event recorded at release)."""

    def __init__(self, *, device: torch.device) -> None:
        self.device = torch.device(device)
        self._lock = Lock()
        self._done: torch.cuda.Event | None = None
        self._open: int | None = None
        self._count = 0

    def reserve(self) -> int:
        if not self._lock.acquire(blocking=False):
            raise SlotBusyError("shared CUDA Graph memory pool is in flight")
        try:
            if self._done is not None:
                torch.cuda.current_stream(self.device).wait_event(self._done)
            self._count += 1
            self._open = self._count
            return self._count
        except Exception:
            self._lock.release()
            raise

    def release(self, ticket: int) -> None:
        if self._open is None or self._open != ticket:
            raise SlotBusyError("stale or unowned static CUDA Graph slot lease")
        try:
            done = torch.cuda.Event()
            done.record(torch.cuda.current_stream(self.device))
            self._done = done
            self._open = None
        finally:
            self._lock.release()


@dataclass(frozen=True, slots=True)
class RowSlice:
    start: int
    stop: int
    capture_rows: int
    padding: int

    @property
    def logical_rows(self) -> int:
        return self.stop - self.start


def lower_rows(logical_rows: int, sizes: tuple[int, ...]) -> tuple[RowSlice, ...]:
    """Split ``logical_rows`` into full largest buckets plus one padded tail bucket."""

    if isinstance(logical_rows, bool) or not isinstance(logical_rows, int) or logical_rows < 1:
        raise ValueError("logical batch size must be a positive integer")
    if not sizes:
        raise ValueError("capture batch catalog is empty")
    sizes = tuple(sorted(sizes))
    parts = []
    start = 0
    largest = sizes[-1]
    while logical_rows - start > largest:
        parts.append(RowSlice(start, start + largest, largest, 0))
        start += largest
    remaining = logical_rows - start
    rows = next(s for s in sizes if s >= remaining)
    parts.append(RowSlice(start, logical_rows, rows, rows - remaining))
    return tuple(parts)


__all__ = ["CapturedCall", "GraphPoolFence", "HipGraphCaptureDriver", "RowSlice", "SlotLeases", "lower_rows"]
