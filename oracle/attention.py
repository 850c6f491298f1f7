"""Oracle for paged GQA attention (test infrastructure only).

Restates the arithmetic of the attention calls on the hot path:

- paged decode / causal prefill over the ragged page table, as bound through
  FlashInfer in executor/talker_kv.py:140-306 (scale 1/sqrt(D), fp32 softmax,
  output cast to the query dtype, :129); causal rows are bottom-right
  aligned (BatchPrefillWithPagedKVCacheWrapper(causal=True), :218): query i
  of a row with qo_len queries and kv_len keys sees keys < kv_len-qo_len+i+1;
- the code predictor's short-cache attention (model/kernels.py:436-463) and
  its CPU reference ``_depth_attention`` (model/components.py:235-252).

All math is fp32 over bf16-valued inputs.  Pinned by
tests/test_oracle_numerics.py with closed forms (kv_len = 1 gives V, equal
keys give the mean of V) and against torch's scaled_dot_product_attention
on the CPU.
"""

from __future__ import annotations

import numpy as np


def gather_row(cache_layer: np.ndarray, pages: np.ndarray, kv_len: int):
    """K, V [kv_len, Hkv, D] of one row from a [pages, 2, ps, Hkv, D] layer."""

    ps = cache_layer.shape[2]
    k = cache_layer[pages, 0].reshape(len(pages) * ps, *cache_layer.shape[3:])[:kv_len]
    v = cache_layer[pages, 1].reshape(len(pages) * ps, *cache_layer.shape[3:])[:kv_len]
    return k, v


def attend(q: np.ndarray, k: np.ndarray, v: np.ndarray, limits: np.ndarray, scale: float) -> np.ndarray:
    """q [n, Hq, D], k/v [L, Hkv, D]; query i sees keys < limits[i]. fp32 out."""

    n, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    qf = q.astype(np.float32).reshape(n, hkv, g, d)
    kf = k.astype(np.float32)
    vf = v.astype(np.float32)
    scores = np.einsum("nhgd,lhd->nhgl", qf, kf, optimize=True) * np.float32(scale)
    keypos = np.arange(k.shape[0])
    mask = keypos[None, :] < np.asarray(limits)[:, None]
    scores = np.where(mask[:, None, None, :], scores, -np.inf)
    m = scores.max(axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    p = np.exp(scores - m)
    denom = p.sum(axis=-1, keepdims=True)
    out = np.einsum("nhgl,lhd->nhgd", p, vf, optimize=True)
    out = np.where(denom > 0, out / np.where(denom > 0, denom, 1.0), 0.0)
    return out.reshape(n, hq, d).astype(np.float32)


def paged_attention(
    q: np.ndarray,
    cache_layer: np.ndarray,
    kv_indptr: np.ndarray,
    kv_indices: np.ndarray,
    last_page_len: np.ndarray,
    qo_indptr: np.ndarray | None = None,
    scale: float | None = None,
) -> np.ndarray:
    """Mixed decode/prefill paged attention; q [tokens, Hq, D] -> fp32 out."""

    d = q.shape[-1]
    scale = float(1.0 / np.sqrt(d)) if scale is None else scale
    ps = cache_layer.shape[2]
    rows = len(kv_indptr) - 1
    qo = np.arange(rows + 1) if qo_indptr is None else np.asarray(qo_indptr)
    out = np.zeros(q.shape, dtype=np.float32)
    for r in range(rows):
        q0, q1 = int(qo[r]), int(qo[r + 1])
        if q1 <= q0:
            continue
        pages = np.asarray(kv_indices[kv_indptr[r] : kv_indptr[r + 1]])
        kv_len = (len(pages) - 1) * ps + int(last_page_len[r]) if len(pages) else 0
        k, v = gather_row(cache_layer, pages, kv_len)
        qo_len = q1 - q0
        limits = np.clip(kv_len - qo_len + np.arange(qo_len) + 1, 0, kv_len)
        out[q0:q1] = attend(q[q0:q1], k, v, limits, scale)
    return out


def short_cache_attention(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, valid_length: int) -> np.ndarray:
    """q [R, Hq, D], caches [R, S, Hkv, D]; one query per row over valid_length keys."""

    d = q.shape[-1]
    scale = float(1.0 / np.sqrt(d))
    out = np.zeros(q.shape, dtype=np.float32)
    lim = np.array([valid_length])
    for r in range(q.shape[0]):
        out[r : r + 1] = attend(q[r : r + 1], k_cache[r, :valid_length], v_cache[r, :valid_length], lim, scale)
    return out
