"""bfloat16 helpers for the oracle (test infrastructure only).

Round-to-nearest-even on the fp32 bit pattern, quiet NaN kept -- the rule
torch uses for ``.to(torch.bfloat16)``.
"""

from __future__ import annotations

import numpy as np


def to_bits(x: np.ndarray) -> np.ndarray:
    """fp32 values -> bf16 bit patterns (uint16), round to nearest even."""

    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def from_bits(b: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> fp32 values (exact)."""

    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_f32(x: np.ndarray) -> np.ndarray:
    """Round fp32 values to the nearest bf16 value, returned as fp32."""

    return from_bits(to_bits(x))
