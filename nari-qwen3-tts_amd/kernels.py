"""The reference's attention-math kernel API, served by the HIP library.

Same names, arguments and errors as model/kernels.py of the reference:
``paired_qk_norm_rope_paged_cache_`` (:94-160), ``paired_qk_norm_rope_``
(:275-332), ``paired_qk_norm_rope_dense_cache_`` (:335-405) and
``decode_attn_nhd_short_cache`` (:466-520).  All inputs must live on the GPU;
there is no CPU path.
"""

from __future__ import annotations

import torch

from . import _lib


def _require_bf16(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t.dtype != torch.bfloat16:
            raise TypeError("HIP attention kernels take bf16 tensors")


def paired_qk_norm_rope_paged_cache_(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    query_weight: torch.Tensor,
    key_weight: torch.Tensor,
    position_ids: torch.Tensor,
    epsilon: float,
    rope_theta: float,
    layer_cache: torch.Tensor,
    write_pages: torch.Tensor,
    write_offsets: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Normalize/rotate QK in place and stage K/V into the paged cache once."""

    if query.ndim != 3 or key.ndim != 3 or value.ndim != 3:
        raise ValueError("Qwen3-TTS QKV tensors must have rank three")
    tokens, query_heads, head_dim = query.shape
    if key.shape != value.shape or key.shape[0] != tokens or key.shape[2] != head_dim:
        raise ValueError("Qwen3-TTS QKV shapes are incompatible")
    key_heads = key.shape[1]
    _lib.require_device(query, key, value, layer_cache, position_ids, write_pages, write_offsets)
    if not (query.dtype == key.dtype == value.dtype == layer_cache.dtype):
        raise TypeError("paired QKV paged staging requires one dtype")
    _require_bf16(query, query_weight, key_weight)
    if head_dim % 2 or query_weight.shape != (head_dim,) or key_weight.shape != (head_dim,):
        raise ValueError("QK norm weights must match an even head dimension")
    if position_ids.shape != (tokens,) or write_pages.shape != (tokens,) or write_offsets.shape != (tokens,):
        raise ValueError("paged QKV metadata must contain one entry per token")
    if layer_cache.ndim != 5 or layer_cache.shape[1] != 2 or layer_cache.shape[3:] != (key_heads, head_dim):
        raise ValueError("paged QKV cache has an invalid layout")
    if not all(t.stride(-1) == 1 for t in (query, key, value, layer_cache)):
        raise ValueError("QKV and paged cache must be contiguous per head")
    for t in (position_ids, write_pages, write_offsets):
        if t.dtype != torch.long:
            raise TypeError("paged QKV metadata must be int64")
    _lib.call(
        "nq_qk_norm_rope_kv_write",
        query.data_ptr(), query.stride(0), query.stride(1),
        key.data_ptr(), key.stride(0), key.stride(1),
        value.data_ptr(), value.stride(0), value.stride(1),
        query_weight.data_ptr(), key_weight.data_ptr(),
        position_ids.data_ptr(), position_ids.stride(0), tokens, query_heads, key_heads, head_dim,
        float(epsilon), float(rope_theta), 1,
        layer_cache.data_ptr(), layer_cache.stride(0), layer_cache.stride(1), layer_cache.stride(2),
        layer_cache.stride(3), write_pages.data_ptr(), write_offsets.data_ptr(), 0,
        _lib.stream(query.device),
    )
    return query, key


def _validate_qk(query, key, query_weight, key_weight, positions):
    if query.ndim != 3 or key.ndim != 3:
        raise ValueError("QK tensors must have shape [tokens, heads, head_dim]")
    tokens, query_heads, head_dim = query.shape
    if key.shape[0] != tokens or key.shape[2] != head_dim or head_dim % 2:
        raise ValueError("QK shapes are incompatible")
    _lib.require_device(query, key, positions)
    if key.device != query.device or query.dtype != key.dtype:
        raise ValueError("paired QK transform requires one dtype/device")
    _require_bf16(query, query_weight, key_weight)
    if query.stride(-1) != 1 or key.stride(-1) != 1:
        raise ValueError("QK tensors must be contiguous per head")
    if positions.shape != (tokens,) or positions.device != query.device:
        raise ValueError("positions must contain one device value per token")
    if positions.dtype != torch.long:
        raise TypeError("positions must be int64")
    if query_weight.shape != (head_dim,) or key_weight.shape != (head_dim,):
        raise ValueError("QK norm weights must match head_dim")
    return tokens, query_heads, key.shape[1], head_dim


def paired_qk_norm_rope_(query, key, query_weight, key_weight, positions, epsilon, rope_theta):
    """Apply the paired QK transform with its bf16 rounding boundary (no cache write)."""

    tokens, hq, hk, d = _validate_qk(query, key, query_weight, key_weight, positions)
    _lib.call(
        "nq_qk_norm_rope_kv_write",
        query.data_ptr(), query.stride(0), query.stride(1),
        key.data_ptr(), key.stride(0), key.stride(1),
        None, 0, 0, query_weight.data_ptr(), key_weight.data_ptr(),
        positions.data_ptr(), positions.stride(0), tokens, hq, hk, d, float(epsilon), float(rope_theta), 1,
        None, 0, 0, 0, 0, None, None, 0, _lib.stream(query.device),
    )
    return query, key


def paired_qk_norm_rope_dense_cache_(
    query, key, value, query_weight, key_weight, positions, epsilon, rope_theta, key_cache, value_cache,
    cache_position: int,
):
    """Transform one-token QK and stage K/V into the fixed code-predictor cache."""

    tokens, hq, hk, d = _validate_qk(query, key, query_weight, key_weight, positions)
    expected = (tokens, key_cache.shape[1], hk, d)
    if value.shape != (tokens, hk, d) or key_cache.shape != expected or value_cache.shape != expected:
        raise ValueError("dense CP QKV cache shape mismatch")
    if not 0 <= cache_position < key_cache.shape[1]:
        raise ValueError("dense CP cache position is invalid")
    if not (value.device == key_cache.device == value_cache.device == query.device):
        raise ValueError("dense CP QKV cache requires one device")
    if not (value.dtype == key_cache.dtype == value_cache.dtype == query.dtype):
        raise TypeError("dense CP QKV cache requires one dtype")
    if key_cache.stride() != value_cache.stride() or key_cache.stride(-1) != 1 or value.stride(-1) != 1:
        raise ValueError("dense CP K and V caches must share one layout")
    delta = value_cache.data_ptr() - key_cache.data_ptr()
    if delta % key_cache.element_size():
        raise ValueError("dense CP K and V caches are misaligned")
    c_kind = delta // key_cache.element_size()
    _lib.call(
        "nq_qk_norm_rope_kv_write",
        query.data_ptr(), query.stride(0), query.stride(1),
        key.data_ptr(), key.stride(0), key.stride(1),
        value.data_ptr(), value.stride(0), value.stride(1),
        query_weight.data_ptr(), key_weight.data_ptr(),
        positions.data_ptr(), positions.stride(0), tokens, hq, hk, d, float(epsilon), float(rope_theta), 0,
        key_cache.data_ptr(), key_cache.stride(0), c_kind, key_cache.stride(1), key_cache.stride(2),
        None, None, int(cache_position), _lib.stream(query.device),
    )
    return query, key


def qkv_partials_norm_rope_dense_cache_(
    partials, splits: int, q_out, query_weight, key_weight, positions, epsilon, rope_theta, key_cache, value_cache,
    cache_position: int,
):
    """paired_qk_norm_rope_dense_cache_ fed by the packed QKV projection's fp32 split-K planes
    [splits, tokens, (Hq + 2 Hkv) * D] (``layers.linear_partials`` leaves them at the start of its
    workspace): each value is the plane-order sum rounded to bf16, the bf16 projection output, so
    the rotated q (into ``q_out`` [tokens, Hq, D]) and the cache rows are those of the projection
    followed by paired_qk_norm_rope_dense_cache_, without the projection's reduction launch."""

    _require_bf16(q_out, query_weight, key_weight, key_cache, value_cache)
    tokens, hq, d = q_out.shape
    hk = key_cache.shape[2]
    if key_cache.shape != (tokens, key_cache.shape[1], hk, d) or value_cache.shape != key_cache.shape:
        raise ValueError("dense CP cache shape mismatch")
    if not 0 <= cache_position < key_cache.shape[1]:
        raise ValueError("dense CP cache position is invalid")
    if key_cache.stride() != value_cache.stride() or key_cache.stride(-1) != 1 or q_out.stride(-1) != 1:
        raise ValueError("dense CP K and V caches must share one layout")
    if positions.dtype != torch.long or positions.shape[0] != tokens:
        raise ValueError("positions must be int64 with one entry per token")
    if partials.numel() * partials.element_size() < splits * tokens * (hq + 2 * hk) * d * 4:
        raise ValueError("partials hold fewer planes than splits")
    delta = value_cache.data_ptr() - key_cache.data_ptr()
    if delta % key_cache.element_size():
        raise ValueError("dense CP K and V caches are misaligned")
    _lib.require_device(partials, q_out, query_weight, key_weight, positions, key_cache, value_cache)
    _lib.call(
        "nq_qkv_partials_norm_rope_kv_write", partials.data_ptr(), int(splits), tokens,
        q_out.data_ptr(), q_out.stride(0), q_out.stride(1), None, 0, 0,
        query_weight.data_ptr(), key_weight.data_ptr(), positions.data_ptr(), positions.stride(0), hq, hk, d,
        float(epsilon), float(rope_theta), 0,
        key_cache.data_ptr(), key_cache.stride(0), delta // key_cache.element_size(), key_cache.stride(1),
        key_cache.stride(2), None, None, int(cache_position), _lib.stream(q_out.device),
    )
    return q_out


def qkv_partials_rope_short_attention_(
    partials, splits: int, q_out, query_weight, key_weight, positions, epsilon, rope_theta, key_cache, value_cache,
    cache_position: int, out,
):
    """qkv_partials_norm_rope_dense_cache_ followed by decode_attn_nhd_short_cache(q_out, key_cache,
    value_cache, cache_position + 1, out=out), the pair the code predictor's decode layer runs
    (model/components.py:294-345), in one launch with the same bits: q_out receives the rotated q,
    the caches position ``cache_position``'s K and V, ``out`` [tokens, Hq, D] the attention."""

    _require_bf16(q_out, query_weight, key_weight, key_cache, value_cache, out)
    tokens, hq, d = q_out.shape
    if key_cache.ndim != 4:
        raise ValueError("dense CP cache shape mismatch")
    hk = key_cache.shape[2]
    if key_cache.shape != (tokens, key_cache.shape[1], hk, d) or value_cache.shape != key_cache.shape:
        raise ValueError("dense CP cache shape mismatch")
    if not isinstance(cache_position, int) or isinstance(cache_position, bool) or not 0 <= cache_position < min(
            key_cache.shape[1], 16):
        raise ValueError("dense CP cache position is invalid (short-cache attention covers at most 16)")
    if key_cache.stride() != value_cache.stride() or key_cache.stride(-1) != 1 or q_out.stride(-1) != 1:
        raise ValueError("dense CP K and V caches must share one layout")
    if out.shape != q_out.shape or out.stride(-1) != 1:
        raise ValueError("out must be [tokens, Hq, D] like q_out")
    if hq % hk:
        raise ValueError("short-cache attention requires compatible heads")
    if positions.dtype != torch.long or positions.shape[0] != tokens:
        raise ValueError("positions must be int64 with one entry per token")
    if partials.numel() * partials.element_size() < splits * tokens * (hq + 2 * hk) * d * 4:
        raise ValueError("partials hold fewer planes than splits")
    delta = value_cache.data_ptr() - key_cache.data_ptr()
    if delta % key_cache.element_size():
        raise ValueError("dense CP K and V caches are misaligned")
    _lib.require_device(partials, q_out, query_weight, key_weight, positions, key_cache, value_cache, out)
    _lib.call(
        "nq_cp_rope_short_attention", partials.data_ptr(), int(splits), tokens,
        query_weight.data_ptr(), key_weight.data_ptr(), positions.data_ptr(), positions.stride(0),
        float(epsilon), float(rope_theta), 0, q_out.data_ptr(), q_out.stride(0), q_out.stride(1),
        key_cache.data_ptr(), key_cache.stride(0), delta // key_cache.element_size(), key_cache.stride(1),
        key_cache.stride(2), int(cache_position), hq, hk, d, float(d) ** -0.5,
        out.data_ptr(), out.stride(0), out.stride(1), _lib.stream(q_out.device),
    )
    return out


def decode_attn_nhd_short_cache(query, key_cache, value_cache, cache_length: int, out=None):
    """Fixed 16-position code-predictor attention (one query per row)."""

    if not isinstance(cache_length, int) or isinstance(cache_length, bool) or not 1 <= cache_length <= 16:
        raise ValueError("short-cache attention requires cache_length in [1, 16]")
    squeeze = query.ndim == 4
    if squeeze:
        if query.shape[1] != 1:
            raise ValueError("short-cache attention supports one query token")
        query = query.squeeze(1)
    if query.ndim != 3 or key_cache.ndim != 4 or key_cache.shape != value_cache.shape:
        raise ValueError("short-cache QKV ranks are invalid")
    rows, hq, d = query.shape
    cache_rows, capacity, hk, cd = key_cache.shape
    if (cache_rows, cd) != (rows, d) or cache_length > capacity:
        raise ValueError("short-cache QKV shapes are incompatible")
    if hq % hk:
        raise ValueError("short-cache attention requires compatible heads")
    _lib.require_device(query, key_cache, value_cache)
    _require_bf16(query, key_cache, value_cache)
    if key_cache.stride() != value_cache.stride():
        raise ValueError("short-cache K and V caches must share one layout")
    delta = value_cache.data_ptr() - key_cache.data_ptr()
    if delta % 2:
        raise ValueError("short-cache K and V caches are misaligned")
    output = torch.empty_like(query) if out is None else out
    _lib.call(
        "nq_cp_short_attention",
        query.data_ptr(), query.stride(0), query.stride(1),
        key_cache.data_ptr(), key_cache.stride(0), delta // 2, key_cache.stride(1), key_cache.stride(2),
        rows, cache_length, hq, hk, d, float(d) ** -0.5,
        output.data_ptr(), output.stride(0), output.stride(1), _lib.stream(query.device),
    )
    return output.unsqueeze(1) if squeeze else output


def paged_attention_noalloc(query: torch.Tensor, layer_cache: torch.Tensor, metadata, *, max_pages: int,
                            sm_scale: float | None = None, parts: int = _lib.NQ_ATTN_DECODE | _lib.NQ_ATTN_PREFILL,
                            status: torch.Tensor | None = None, out: torch.Tensor) -> torch.Tensor:
    """Paged attention of ``query`` [tokens, Hq, D] over one layer ``[pages, 2, ps, Hkv, D]`` of the
    cache with ``metadata`` (a TalkerAttentionMetadata), planned and run with the library's static
    scratch (``nq_paged_attention_noalloc``): no device allocation, no workspace argument.  ``out``
    is required for the same reason.  Calls that overlap on one GPU share the scratch and race."""

    _require_bf16(query, layer_cache, out)
    if query.ndim != 3 or layer_cache.ndim != 5 or layer_cache.shape[1] != 2:
        raise ValueError("query must be [tokens, Hq, D] and the cache [pages, 2, page_size, Hkv, D]")
    tokens, hq, d = query.shape
    pages, _, page_size, hkv, d_cache = layer_cache.shape
    if d_cache != d or out.shape != query.shape or out.stride(-1) != 1 or query.stride(-1) != 1:
        raise ValueError("query, cache and out disagree on the head layout")
    rows = metadata.paged_kv_indptr.numel() - 1
    need = int(_lib.load().nq_attention_workspace_bytes(tokens, int(max_pages), page_size, hq, hkv, d))
    _lib.check(min(need, 0), "nq_attention_workspace_bytes")
    if need > _lib.NQ_NOALLOC_SCRATCH_BYTES:
        raise ValueError(f"this batch needs {need} bytes of attention scratch; the no-allocation entry point "
                         f"holds {_lib.NQ_NOALLOC_SCRATCH_BYTES} per GPU (use the workspace path)")
    for t in (metadata.paged_kv_indptr, metadata.paged_kv_last_page_len, metadata.paged_kv_indices):
        if t.dtype != torch.int32:
            raise TypeError("paged metadata must be int32")
    _lib.require_device(query, layer_cache, out, metadata.paged_kv_indptr, status)
    scale = float(d) ** -0.5 if sm_scale is None else float(sm_scale)
    _lib.call(
        "nq_paged_attention_noalloc",
        _lib.ptr(metadata.qo_indptr), metadata.paged_kv_indptr.data_ptr(),
        metadata.paged_kv_last_page_len.data_ptr(), metadata.paged_kv_indices.data_ptr(), rows,
        query.data_ptr(), query.stride(0), query.stride(1), layer_cache.data_ptr(), layer_cache.stride(0),
        layer_cache.stride(1), layer_cache.stride(2), layer_cache.stride(3), pages, page_size, hq, hkv, d, scale,
        out.data_ptr(), out.stride(0), out.stride(1), tokens, int(max_pages), int(parts), _lib.ptr(status),
        _lib.stream(query.device),
    )
    return out


__all__ = [
    "paged_attention_noalloc",
    "decode_attn_nhd_short_cache",
    "paired_qk_norm_rope_",
    "paired_qk_norm_rope_dense_cache_",
    "qkv_partials_norm_rope_dense_cache_",
    "qkv_partials_rope_short_attention_",
    "paired_qk_norm_rope_paged_cache_",
]
