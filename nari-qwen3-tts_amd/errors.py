"""Exception types with the reference's names and meaning.

KVAllocationError / StaleKVPublicationError mirror executor/cache.py:11-16,
SlotBusyError mirrors executor/cuda_graph.py:102-103, CaptureCoverageError
planner/catalog.py:19-20.
"""

from __future__ import annotations


class KVAllocationError(RuntimeError):
    pass


class StaleKVPublicationError(RuntimeError):
    pass


class SlotBusyError(RuntimeError):
    pass


class CaptureCoverageError(RuntimeError):
    pass
