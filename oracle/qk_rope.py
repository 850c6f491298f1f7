"""Oracle for the paired q/k RMSNorm + RoPE + cache write (test infrastructure only).

Restates _paired_qk_norm_rope_paged_cache_kernel (model/kernels.py:15-91) and
the dense variant (:163-248):

    x        = head vector (fp32 from bf16)
    inv_rms  = 1 / sqrt(sum(x^2) / D + eps)                        (:61-62)
    y        = x * inv_rms * w                                     (:63-64)
    y        = bf16(y)  when round_to_input                        (:65-67, :225-227)
    inv_freq = exp(-ln(theta) * (2i / D)), angle = pos * inv_freq  (:68-70)
    out_i    = y_i cos - y_{i+D/2} sin,  out_{i+D/2} = y_{i+D/2} cos + y_i sin (:73-74)

q and k are returned rotated (bf16 values as fp32); the K cache receives the
rotated k, the V cache the unchanged v (:78-91).  Pinned by
tests/test_oracle_numerics.py: position 0 is the identity rotation, the
rotation preserves each (i, i+D/2) pair's norm, and the result matches the
reference's CPU RoPE formulation (model/components.py:213-233) written with
torch on the CPU.
"""

from __future__ import annotations

import numpy as np

from . import bf16


def norm_rope(x: np.ndarray, weight: np.ndarray, positions: np.ndarray, eps: float, theta: float,
              round_to_input: bool) -> np.ndarray:
    """x [T, H, D] (bf16 values) -> rotated bf16 values as fp32."""

    x = x.astype(np.float32)
    d = x.shape[-1]
    half = d // 2
    ss = np.sum(x * x, axis=-1, keepdims=True, dtype=np.float32)
    inv = np.float32(1.0) / np.sqrt(ss / np.float32(d) + np.float32(eps))
    y = x * inv * weight.astype(np.float32)
    if round_to_input:
        y = bf16.round_f32(y)
    i = np.arange(half, dtype=np.float32)
    inv_freq = np.exp(-np.float32(np.log(np.float32(theta))) * (i * np.float32(2.0) / np.float32(d)))
    angle = positions.astype(np.float32)[:, None] * inv_freq[None, :]
    cos = np.cos(angle)[:, None, :]
    sin = np.sin(angle)[:, None, :]
    first, second = y[..., :half], y[..., half:]
    out = np.concatenate((first * cos - second * sin, second * cos + first * sin), axis=-1)
    return bf16.round_f32(out.astype(np.float32))


def paged_write(cache: np.ndarray, k_rot: np.ndarray, v: np.ndarray, write_pages: np.ndarray,
                write_offsets: np.ndarray) -> np.ndarray:
    """Write rotated K and V of each token into a [pages, 2, ps, Hkv, D] layer."""

    out = cache.copy()
    for t in range(k_rot.shape[0]):
        out[int(write_pages[t]), 0, int(write_offsets[t])] = k_rot[t]
        out[int(write_pages[t]), 1, int(write_offsets[t])] = v[t]
    return out
