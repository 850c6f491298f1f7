"""Oracle for RMSNorm, residual add + RMSNorm and SwiGLU (test infrastructure only).

Restates model/layers.py:103-115 (RMSNorm: fp32 x * rsqrt(mean(x^2) + eps)
* weight, cast back to bf16), :78-79 (residual = residual + hidden in bf16,
then the norm of the rounded sum) and :39-40 (silu(gate) * up).  Pinned by
tests/test_oracle_numerics.py against torch's own CPU ops on the same inputs.
"""

from __future__ import annotations

import numpy as np

from . import bf16


def rmsnorm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    x = x.astype(np.float32)
    var = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32)
    y = x * (np.float32(1.0) / np.sqrt(var + np.float32(eps))) * weight.astype(np.float32)
    return bf16.round_f32(y)


def add_rmsnorm(hidden: np.ndarray, residual: np.ndarray, weight: np.ndarray, eps: float):
    res = bf16.round_f32(residual.astype(np.float32) + hidden.astype(np.float32))
    return rmsnorm(res, weight, eps), res


def silu_mul(gate_up: np.ndarray) -> np.ndarray:
    g, u = np.split(gate_up.astype(np.float32), 2, axis=-1)
    with np.errstate(over="ignore"):  # exp(-g) = inf for very negative g gives silu = -0, as on the device
        return bf16.round_f32(g / (np.float32(1.0) + np.exp(-g)) * u)
