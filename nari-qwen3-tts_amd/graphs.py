"""hipGraph capture of fixed-shape buckets (the reference's CaptureDriver protocol).

``HipGraphCaptureDriver.capture(operation, after_warmup=None)`` runs the
operation eagerly twice, then records it into a graph sharing one memory
pool, and returns a call whose ``replay()`` launches the graph and returns
the static outputs (executor/cuda_graph.py:15-77).  PyTorch-ROCm's graph
object is a hipGraph; the HIP kernels launch on the capturing stream and
issue no memset/memcpy nodes.  ``lower_rows`` splits a logical batch over
the capture buckets as planner/catalog.py:43-71 does.
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass

import torch


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


__all__ = ["CapturedCall", "HipGraphCaptureDriver", "RowSlice", "lower_rows"]
