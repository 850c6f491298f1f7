"""Paged talker KV with GPU-built metadata and HIP attention bindings.

Drop-in for the reference's ``PagedTalkerKV`` and its FlashInfer bindings
(executor/talker_kv.py:15-570): the same constructor, the TalkerKVBackend
methods (create_prefill/create_decode, prepare_prefill/prepare_decode,
prepare_capture/finish_capture, abort, add_request/remove_request/state) and
the TalkerAttentionContext protocol (metadata, plan, select_layer, attend,
advance_sequence_lengths).  What moves to the GPU:

- ``_metadata`` (talker_kv.py:403-483): the host keeps page ownership (the
  allocator) and stages O(rows) scalars; ``nq_plan_ragged`` writes
  qo/kv indptr, the page list, last-page lengths, positions and write slots
  straight into the binding's static buffers, reading prior pages from a
  device page table and new pages from a device copy of the sorted free list.
- ``plan`` (talker_kv.py:175-223, 259-303): ``nq_attention_plan`` splits the
  keys of every query into chunks on the GPU; there is no plan signature to
  reuse because planning is one small kernel.
- ``attend`` (talker_kv.py:104-129): ``nq_qk_norm_rope_kv_write`` then
  ``nq_paged_attention``.

Storage keeps the reference layout ``[layers, pages, 2, page_size, Hkv, D]``
(talker_kv.py:336-340), bf16.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .cache import PagedKVAllocator, PendingKVPublication, RequestKVState


@dataclass(frozen=True, slots=True)
class TalkerAttentionMetadata:
    qo_indptr: torch.Tensor | None
    paged_kv_indptr: torch.Tensor
    paged_kv_indices: torch.Tensor
    paged_kv_last_page_len: torch.Tensor
    position_ids: torch.Tensor
    write_pages: torch.Tensor
    write_offsets: torch.Tensor
    padding_pages: tuple[int, ...]
    reuse_attention_plan: bool = True


class _MetadataBuffers:
    """Static device buffers one planner launch writes into."""

    def __init__(self, *, rows: int, tokens: int, index_capacity: int, prefill: bool, device) -> None:
        i32 = dict(dtype=torch.int32, device=device)
        i64 = dict(dtype=torch.long, device=device)
        self.qo_indptr = torch.zeros(rows + 1, **i32) if prefill else None
        self.kv_indptr = torch.zeros(rows + 1, **i32)
        self.kv_indices = torch.zeros(index_capacity, **i32)
        self.last_page_len = torch.ones(rows, **i32)
        self.position_ids = torch.zeros(tokens, **i64)
        self.write_pages = torch.zeros(tokens, **i64)
        self.write_offsets = torch.zeros(tokens, **i64)
        self.status = torch.zeros(2, **i32)
        # device addresses of the planner outputs (the buffers live as long as the binding)
        self.ptrs = tuple(0 if t is None else t.data_ptr() for t in (
            self.qo_indptr, self.kv_indptr, self.kv_indices, self.last_page_len, self.position_ids, self.write_pages,
            self.write_offsets, self.status))


class _HipBindingBase:
    """One captured slot's attention context (TalkerAttentionContext)."""

    prefill = False

    def __init__(
        self,
        *,
        storage: torch.Tensor,
        capture_batch_size: int,
        token_capacity: int,
        num_qo_heads: int,
        num_kv_heads: int,
        head_dim: int,
        page_size: int,
        total_pages: int,
        device: torch.device,
        dtype: torch.dtype,
        workspace: torch.Tensor | None = None,
        **_: object,
    ) -> None:
        self.storage = storage
        self.capture_batch_size = capture_batch_size
        self.token_capacity = token_capacity
        self.num_qo_heads = num_qo_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.page_size = page_size
        self.total_pages = total_pages
        self.device = device
        self.dtype = dtype
        # Padding rows may repeat scratch pages, hence + rows (talker_kv.py:147-153).
        self.index_capacity = total_pages + capture_batch_size
        self.buffers = _MetadataBuffers(
            rows=capture_batch_size,
            tokens=token_capacity,
            index_capacity=self.index_capacity,
            prefill=self.prefill,
            device=device,
        )
        lib = _lib.load()
        nbytes = lib.nq_attention_workspace_bytes(
            token_capacity, self.index_capacity, page_size, num_qo_heads, num_kv_heads, head_dim
        )
        _lib.check(min(int(nbytes), 0), "nq_attention_workspace_bytes")
        if workspace is not None and workspace.numel() < int(nbytes):
            raise ValueError(f"the attention workspace holds {workspace.numel()} bytes; this binding needs {int(nbytes)}")
        # plan + partials; shared by the bindings of one capture slot (their graphs never run at once)
        self.workspace = workspace if workspace is not None else torch.zeros(int(nbytes), dtype=torch.uint8,
                                                                             device=device)
        self.attention_status = torch.zeros(1, dtype=torch.int32, device=device)
        self.output = torch.zeros((token_capacity, num_qo_heads, head_dim), dtype=dtype, device=device)
        self.position_ids = self.buffers.position_ids
        self.write_pages = self.buffers.write_pages
        self.write_offsets = self.buffers.write_offsets
        self.metadata: TalkerAttentionMetadata | None = None
        self._layer_index = 0
        # decode bindings take the fused bins kernel in attend_partials while the library accepts the shape
        self.fused_decode = True
        self._side: torch.cuda.Stream | None = None
        self.free_list_status: torch.Tensor | None = None
        # whether a prefill binding's attention runs a decode launch for its one-query rows (beside
        # the prefill launch, on two streams) or plans them into the prefill launch (one launch)
        self.decode_rows = not self.prefill

    # -- planning ---------------------------------------------------------
    def _stage(self, metadata: TalkerAttentionMetadata) -> None:
        """Copy metadata produced elsewhere into the static buffers."""

        b = self.buffers
        if metadata.paged_kv_indptr.data_ptr() == b.kv_indptr.data_ptr():
            return
        if metadata.position_ids.shape != b.position_ids.shape:
            raise ValueError("Talker position metadata does not match the captured token capacity")
        if metadata.paged_kv_indices.numel() > b.kv_indices.numel():
            raise ValueError("Talker page metadata exceeds its captured buffer")
        b.kv_indptr.copy_(metadata.paged_kv_indptr, non_blocking=True)
        b.kv_indices[: metadata.paged_kv_indices.numel()].copy_(metadata.paged_kv_indices, non_blocking=True)
        b.last_page_len.copy_(metadata.paged_kv_last_page_len, non_blocking=True)
        b.position_ids.copy_(metadata.position_ids, non_blocking=True)
        b.write_pages.copy_(metadata.write_pages, non_blocking=True)
        b.write_offsets.copy_(metadata.write_offsets, non_blocking=True)
        if b.qo_indptr is not None:
            b.qo_indptr.copy_(metadata.qo_indptr, non_blocking=True)

    def plan(self, metadata: TalkerAttentionMetadata) -> None:
        if self.prefill and metadata.qo_indptr is None:
            raise ValueError("Talker prefill requires packed query metadata")
        if not self.prefill and metadata.qo_indptr is not None:
            raise ValueError("Talker decode cannot contain packed query metadata")
        self._stage(metadata)
        bp = self.buffers.ptrs
        _lib.call(
            "nq_attention_plan_parts",
            bp[0] or None,
            bp[1],
            bp[3],
            bp[2],
            bp[4],
            bp[5],
            bp[6],
            self.capture_batch_size,
            self.token_capacity,
            self.index_capacity,
            self.page_size,
            self.num_qo_heads,
            self.num_kv_heads,
            self.head_dim,
            self._parts(),
            _lib.ptr(self.workspace),
            self.workspace.numel(),
            _lib.stream(self.device),
        )
        self.metadata = metadata

    def select_layer(self, index: int) -> None:
        if not 0 <= index < self.storage.shape[0]:
            raise IndexError("Talker layer index exceeds paged KV storage")
        self._layer_index = index

    # -- attention ----------------------------------------------------------
    def attend(self, attention: object, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor) -> torch.Tensor:
        tokens, hq, d = query.shape
        if tokens != self.token_capacity or hq != self.num_qo_heads or d != self.head_dim:
            raise ValueError("Talker query shape does not match the captured binding")
        if key.shape != value.shape or key.shape != (tokens, self.num_kv_heads, d):
            raise ValueError("Qwen3-TTS QKV shapes are incompatible")
        if not (query.dtype == key.dtype == value.dtype == self.storage.dtype == torch.bfloat16):
            raise TypeError("paired QKV paged staging requires bf16 q, k, v and cache")
        if any(t.stride(-1) != 1 for t in (query, key, value)):
            raise ValueError("QKV and paged cache must be contiguous per head")
        qw, kw = attention.q_norm.weight, attention.k_norm.weight
        if qw.dtype != torch.bfloat16 or kw.dtype != torch.bfloat16:
            raise TypeError("QK norm weights must be bf16")
        layer = self.storage[self._layer_index]
        b = self.buffers
        stream = _lib.stream(self.device)
        _lib.call(
            "nq_qk_norm_rope_kv_write",
            query.data_ptr(), query.stride(0), query.stride(1),
            key.data_ptr(), key.stride(0), key.stride(1),
            value.data_ptr(), value.stride(0), value.stride(1),
            qw.data_ptr(), kw.data_ptr(),
            b.position_ids.data_ptr(), 1, tokens, hq, self.num_kv_heads, d,
            float(attention.q_norm.variance_epsilon), float(attention.rope_theta), 1,
            layer.data_ptr(), layer.stride(0), layer.stride(1), layer.stride(2), layer.stride(3),
            b.write_pages.data_ptr(), b.write_offsets.data_ptr(), 0, stream,
        )
        return self.run_attention(query, self._layer_index)

    def attend_partials(self, attention: object, partials: torch.Tensor, splits: int,
                        query_out: torch.Tensor) -> torch.Tensor:
        """``attend`` fed by the packed QKV projection's fp32 split-K planes (``linear_partials``):
        q/k norm + RoPE + K/V write straight from the planes, rotated q into ``query_out``
        [tokens, Hq, D], then paged attention."""

        tokens = self.token_capacity
        if query_out.shape != (tokens, self.num_qo_heads, self.head_dim) or query_out.stride(-1) != 1:
            raise ValueError("query_out must be [tokens, Hq, D] with unit inner stride")
        qw, kw = attention.q_norm.weight, attention.k_norm.weight
        layer = self.storage[self._layer_index]
        b = self.buffers
        stream = _lib.stream(self.device)
        if not self.prefill and self.fused_decode:
            # decode rows: one fused kernel (bins of whole rows, q/k norm + RoPE + K/V write in its
            # prologue); shapes it does not take fall back to the two-kernel path below, for good
            out = self.output
            rc = _lib.load().nq_paged_decode_rope_attention(
                partials.data_ptr(), int(splits), tokens, qw.data_ptr(), kw.data_ptr(), b.position_ids.data_ptr(),
                float(attention.q_norm.variance_epsilon), float(attention.rope_theta), 1,
                layer.data_ptr(), layer.stride(0), layer.stride(1), layer.stride(2), layer.stride(3), layer.shape[0],
                b.write_pages.data_ptr(), b.write_offsets.data_ptr(), b.kv_indices.data_ptr(), self.page_size,
                self.num_qo_heads, self.num_kv_heads, self.head_dim, float(self.head_dim) ** -0.5,
                out.data_ptr(), out.stride(0), out.stride(1), self.token_capacity, self.index_capacity,
                self.workspace.data_ptr(), self.workspace.numel(), self.attention_status.data_ptr(), stream)
            if rc != _lib.NQ_ERR_UNSUPPORTED:
                _lib.check(rc, "nq_paged_decode_rope_attention")
                return out
            self.fused_decode = False
        _lib.call(
            "nq_qkv_partials_norm_rope_kv_write",
            partials.data_ptr(), int(splits), tokens, query_out.data_ptr(), query_out.stride(0), query_out.stride(1),
            None, 0, 0, qw.data_ptr(), kw.data_ptr(), b.position_ids.data_ptr(), 1, self.num_qo_heads,
            self.num_kv_heads, self.head_dim, float(attention.q_norm.variance_epsilon), float(attention.rope_theta), 1,
            layer.data_ptr(), layer.stride(0), layer.stride(1), layer.stride(2), layer.stride(3),
            b.write_pages.data_ptr(), b.write_offsets.data_ptr(), 0, stream,
        )
        return self.run_attention(query_out, self._layer_index)

    def _parts(self) -> int:
        """The attention launches this binding runs (and its plan is made for)."""

        if not self.prefill:
            return _lib.NQ_ATTN_DECODE
        return _lib.NQ_ATTN_DECODE | _lib.NQ_ATTN_PREFILL if self.decode_rows else _lib.NQ_ATTN_PREFILL

    def run_attention(self, query: torch.Tensor, layer_index: int, stream: int | None = None) -> torch.Tensor:
        """Paged attention of ``query`` over one layer with the planned metadata (no q/k transform).

        A prefill binding with ``decode_rows`` runs the prefill rows on a side stream while the
        decode rows run on the caller's stream (fork/join through events, so the pair is
        graph-capturable); without it the plan put its one-query rows into the prefill part too,
        and one launch serves the batch."""

        if not self.prefill or not self.decode_rows or stream is not None:
            return self._attention_call(query, layer_index, self._parts(),
                                        _lib.stream(self.device) if stream is None else stream)
        main = torch.cuda.current_stream(self.device)
        if self._side is None:
            self._side = torch.cuda.Stream(self.device)
            self._fork, self._join = torch.cuda.Event(), torch.cuda.Event()
        self._fork.record(main)
        self._side.wait_event(self._fork)
        # the prefill launch is issued first.  The other order helps a batch that has decode rows (its
        # bins take the CUs first: mixed layer median 124.9 against 127.2 us) but costs a batch of
        # prompt chunks alone, whose empty decode launch then goes ahead of the tiles, 6 % of a
        # prefill decision (21.09 against 19.89 ms)
        self._attention_call(query, layer_index, _lib.NQ_ATTN_PREFILL, self._side.cuda_stream)
        out = self._attention_call(query, layer_index, _lib.NQ_ATTN_DECODE | _lib.NQ_ATTN_BESIDE_PREFILL,
                                   main.cuda_stream)
        self._join.record(self._side)
        main.wait_event(self._join)
        return out

    def _attention_call(self, query: torch.Tensor, layer_index: int, parts: int, stream: int) -> torch.Tensor:
        layer = self.storage[layer_index]
        out = self.output
        _lib.call(
            "nq_paged_attention",
            query.data_ptr(), query.stride(0), query.stride(1),
            layer.data_ptr(), layer.stride(0), layer.stride(1), layer.stride(2), layer.stride(3),
            layer.shape[0], self.buffers.kv_indices.data_ptr(),
            self.page_size, self.num_qo_heads, self.num_kv_heads, self.head_dim, float(self.head_dim) ** -0.5,
            out.data_ptr(), out.stride(0), out.stride(1),
            self.token_capacity, self.index_capacity, int(parts), self.workspace.data_ptr(),
            self.workspace.numel(), self.attention_status.data_ptr(), stream,
        )
        return out

    @staticmethod
    def advance_sequence_lengths() -> None:
        # The Engine owns committed lengths; replay only proposes a publication.
        return None


class HipPrefillBinding(_HipBindingBase):
    prefill = True


class HipDecodeBinding(_HipBindingBase):
    prefill = False


class _PinnedRing:
    """Pinned host buffers for small host-to-device copies on the current stream: a buffer is
    reused only after the copy that read it has finished."""

    def __init__(self, shape: tuple[int, ...], device, depth: int = 4) -> None:
        self.host = [torch.zeros(shape, dtype=torch.int32, pin_memory=True) for _ in range(depth)]
        self.view = [h.numpy() for h in self.host]
        self.events = [torch.cuda.Event() for _ in range(depth)]
        self.used = [False] * depth
        self.next = 0

    def acquire(self) -> tuple[int, np.ndarray]:
        i = self.next
        self.next = (i + 1) % len(self.host)
        if self.used[i]:
            self.events[i].synchronize()
        return i, self.view[i]

    def send(self, i: int, dst: torch.Tensor, count: int, stream: torch.cuda.Stream | None = None) -> None:
        """Copy the first ``count`` elements (along dim -1) of buffer i to ``dst`` on the current stream
        (``stream``, when the caller already holds it)."""

        src = self.host[i]
        if count == src.shape[-1] and dst.shape == src.shape:
            dst.copy_(src, non_blocking=True)
        else:
            dst[..., :count].copy_(src[..., :count], non_blocking=True)
        self.events[i].record(stream)
        self.used[i] = True


class PagedTalkerKV:
    """Request ledger, device page table, device free list and one HIP binding per captured slot.

    The device free list is a sorted int32 array with a consumed front, double-buffered: pages
    taken by a reservation move the front (the planner kernel reads new pages from it), returned
    pages are merged in on the GPU (``nq_free_list_merge``) before the next planner launch, by
    replaying the ledger's ordered log of free-list changes.  The list is uploaded whole only at
    construction and after ``adopt_request`` (setup)."""

    def __init__(
        self,
        *,
        num_layers: int,
        num_kv_heads: int,
        num_qo_heads: int,
        head_dim: int,
        total_pages: int,
        page_size: int,
        scratch_page_count: int,
        workspace_bytes: int,
        device: torch.device,
        dtype: torch.dtype,
        binding_factory=None,
    ) -> None:
        device = torch.device(device)
        if device.type != "cuda":
            raise RuntimeError("PagedTalkerKV runs on the GPU only (HIP kernels, no CPU path)")
        if dtype != torch.bfloat16:
            raise TypeError("paged talker KV stores bf16")
        if page_size < 1 or page_size & (page_size - 1):
            raise ValueError("page_size must be a power of two")
        _lib.load()
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.num_qo_heads = num_qo_heads
        self.head_dim = head_dim
        self.total_pages = total_pages
        self.page_size = page_size
        self.workspace_bytes = workspace_bytes
        self.device = device
        self.dtype = dtype
        self.storage = torch.zeros(
            (num_layers, total_pages, 2, page_size, num_kv_heads, head_dim), dtype=dtype, device=device
        )
        self.allocator = PagedKVAllocator(total_pages=total_pages, page_size=page_size)
        self._scratch_pages = self.allocator.claim_scratch_pages(scratch_page_count)
        self._scratch_dev = torch.tensor(self._scratch_pages, dtype=torch.int32, device=device)
        self._binding_factory = binding_factory
        self._workspaces: dict[int, torch.Tensor] = {}
        self._next_capture = 0
        self._capture_requests: dict[int, tuple[str, ...]] = {}
        # device page table: row = ledger slot, up to total_pages page ids per request
        self._table = torch.zeros((self.allocator.slot_capacity, total_pages), dtype=torch.int32, device=device)
        # device free list (two buffers: a merge writes the other one), its front and length
        self._free_dev = [torch.zeros(max(total_pages, 1), dtype=torch.int32, device=device) for _ in range(2)]
        self._returned_dev = torch.zeros(max(total_pages, 1), dtype=torch.int32, device=device)
        self._free_cur = 0
        self._free_front = 0
        self._free_len = 0
        # device status word of the free-list merges (read and cleared by the step report)
        self.free_list_status = torch.zeros(1, dtype=torch.int32, device=device)
        self._pages_ring = _PinnedRing((max(total_pages, 1),), device)
        self._rows_ring: _PinnedRing | None = None
        self.allocator.resend_free_list = True

    # -- the device free list ---------------------------------------------------
    def _sync_free_list(self, current: torch.cuda.Stream | None = None) -> None:
        """Bring the device free list to the ledger's: replay its log of takes and returns (on the
        current stream, ``current`` when the caller already holds it)."""

        a = self.allocator
        if not a.resend_free_list and not a.has_log():
            return
        current = current if current is not None else torch.cuda.current_stream(self.device)
        stream = current.cuda_stream
        if a.resend_free_list:
            a.resend_free_list = False
            a.drain_log()
            free = a.free_array()
            i, buf = self._pages_ring.acquire()
            buf[: free.shape[0]] = free
            self._free_cur = 0
            self._pages_ring.send(i, self._free_dev[0], free.shape[0], current)
            self._free_front, self._free_len = 0, int(free.shape[0])
            return
        returned: list[np.ndarray] = []
        for kind, value in a.drain_log() + [("take", 0)]:
            if kind == "return":
                returned.append(value)
                continue
            if returned:  # a run of returns: one merge
                pages = returned[0] if len(returned) == 1 else np.sort(np.concatenate(returned))
                returned = []
                i, buf = self._pages_ring.acquire()
                m = int(pages.shape[0])
                buf[:m] = pages
                self._pages_ring.send(i, self._returned_dev, m, current)
                src = self._free_dev[self._free_cur]
                dst = self._free_dev[1 - self._free_cur]
                live = self._free_len - self._free_front
                _lib.call("nq_free_list_merge", src.data_ptr() + 4 * self._free_front, live,
                          self._returned_dev.data_ptr(), m, dst.data_ptr(), self.free_list_status.data_ptr(), stream)
                self._free_cur = 1 - self._free_cur
                self._free_front, self._free_len = 0, live + m
            self._free_front += value

    def device_free_list(self) -> torch.Tensor:
        """The device copy of the sorted free list (after replaying pending changes)."""

        self._sync_free_list()
        return self._free_dev[self._free_cur][self._free_front: self._free_len]

    # -- request lifecycle ----------------------------------------------------
    def add_request(self, request_id: str) -> None:
        self.allocator.add_request(request_id)
        rows = self.allocator.slot_capacity
        if rows > self._table.shape[0]:
            grown = torch.zeros((rows, self._table.shape[1]), dtype=torch.int32, device=self.device)
            grown[: self._table.shape[0]].copy_(self._table)
            self._table = grown

    def remove_request(self, request_id: str) -> None:
        self.allocator.remove_request(request_id)

    def state(self, request_id: str) -> RequestKVState:
        return self.allocator.state(request_id)

    def adopt_request(self, request_id: str, pages, sequence_length: int, position_start: int | None = None) -> None:
        """Give a live request committed KV on ``pages`` (benchmark and test setup)."""

        pages = tuple(int(p) for p in pages)
        self.allocator.adopt(
            request_id, pages, sequence_length, sequence_length if position_start is None else position_start
        )
        if pages:
            self._table[self.allocator.slot(request_id), : len(pages)].copy_(torch.tensor(pages, dtype=torch.int32))

    # -- bindings -----------------------------------------------------------
    def _binding(self, key, slot: int):
        prefill = hasattr(key, "token_capacity")
        factory = self._binding_factory or (HipPrefillBinding if prefill else HipDecodeBinding)
        arguments = dict(
            storage=self.storage,
            capture_batch_size=key.capture_batch_size,
            token_capacity=key.token_capacity if prefill else key.capture_batch_size,
            num_qo_heads=self.num_qo_heads,
            num_kv_heads=self.num_kv_heads,
            head_dim=self.head_dim,
            page_size=self.page_size,
            total_pages=self.total_pages,
            device=self.device,
            dtype=self.dtype,
        )
        if self._binding_factory is not None:
            arguments.update(slot=slot, metadata=None)
        else:
            arguments.update(workspace=self._slot_workspace(slot, key, prefill))
        binding = factory(**arguments)
        if isinstance(binding, _HipBindingBase):
            # the step report reads the free-list merge status next to the binding's own words
            binding.free_list_status = self.free_list_status
        return binding

    def _slot_workspace(self, slot: int, key, prefill: bool) -> torch.Tensor:
        """The attention workspace of capture slot ``slot``, shared by every binding of that slot
        (executor/talker_kv.py:361): at least ``workspace_bytes``, grown (for later bindings; earlier
        ones keep theirs) when a bucket needs more."""

        tokens = key.token_capacity if prefill else key.capture_batch_size
        need = int(_lib.load().nq_attention_workspace_bytes(
            tokens, self.total_pages + key.capture_batch_size, self.page_size, self.num_qo_heads, self.num_kv_heads,
            self.head_dim))
        _lib.check(min(need, 0), "nq_attention_workspace_bytes")
        ws = self._workspaces.get(slot)
        if ws is None or ws.numel() < need:
            ws = torch.zeros(max(need, int(self.workspace_bytes)), dtype=torch.uint8, device=self.device)
            self._workspaces[slot] = ws
        return ws

    def create_prefill(self, key, *, slot: int, decode_rows: bool = False):
        """The prefill binding of ``key`` in capture slot ``slot``.  ``decode_rows``: batches of this
        capture may hold many one-query (decode) rows beside the prompt chunks; their attention then
        runs as a decode launch beside the prefill launch, on two streams.  Without it (the
        reference's prefill batches, prompt chunks only) a one-query row is attended in the prefill
        launch, and the empty decode launch and the fork/join it needs are saved."""

        binding = self._binding(key, slot)
        if isinstance(binding, _HipBindingBase):
            binding.decode_rows = bool(decode_rows)
        return binding

    def create_decode(self, key, *, slot: int):
        return self._binding(key, slot)

    @staticmethod
    def _set_metadata(context: object, metadata: TalkerAttentionMetadata) -> None:
        if isinstance(context, dict):
            context["metadata"] = metadata
        else:
            context.plan(metadata)

    def _validate_scratch_capacity(self, *, capture_rows: int, token_capacity: int) -> None:
        if capture_rows > len(self._scratch_pages):
            raise ValueError("Talker CUDA Graph rows exceed executor-private scratch pages")
        if token_capacity > len(self._scratch_pages) * self.page_size:
            raise ValueError("Talker token capacity exceeds executor-private scratch slots")

    def _metadata(
        self,
        *,
        request_ids: tuple[str, ...],
        advances: tuple[int, ...],
        capture_rows: int,
        token_capacity: int,
        prefill: bool,
        context: object,
        reuse_attention_plan: bool = True,
    ) -> tuple[tuple[PendingKVPublication, ...], TalkerAttentionMetadata]:
        self._validate_scratch_capacity(capture_rows=capture_rows, token_capacity=token_capacity)
        n = len(request_ids)
        if n > capture_rows:
            raise ValueError("Talker request rows do not fit the capture")
        if sum(advances) + (0 if prefill else capture_rows - n) > token_capacity:
            raise ValueError("Talker KV metadata exceeds the captured token capacity")
        current = torch.cuda.current_stream(self.device)
        self._sync_free_list(current)
        a = self.allocator
        slots = a.slots(request_ids)
        # rows 0-4: one column per request row; row 5: the pages the reservation takes (at most
        # ceil(advance / page_size) + 1 per row), which the planner checks against the device list
        width = max(64, capture_rows + token_capacity // self.page_size + 1)
        if self._rows_ring is None or self._rows_ring.view[0].shape[1] < width:
            self._rows_ring = _PinnedRing((6, width), self.device)
            self._rows_dev = torch.zeros((6, width), dtype=torch.int32, device=self.device)
            self._rows_ptrs = tuple(self._rows_dev[k].data_ptr() for k in range(6))
        # the rows' committed numbers, read before the reservation (it does not change them)
        i, rows = self._rows_ring.acquire()
        np.take(a.length, slots, out=rows[0, :n])
        np.take(a.position, slots, out=rows[1, :n])
        np.take(a.page_count, slots, out=rows[3, :n])
        rows[4, :n] = slots
        reservation = a.reserve(request_ids, advances, slots)
        publications = reservation.publications
        try:
            rows[2, :n] = advances
            if reservation.pages_taken:
                rows[5, : reservation.pages_taken] = reservation.taken
            if isinstance(context, _HipBindingBase):
                buffers = context.buffers
            else:
                buffers = _MetadataBuffers(
                    rows=capture_rows,
                    tokens=token_capacity,
                    index_capacity=self.total_pages + capture_rows,
                    prefill=prefill,
                    device=self.device,
                )
            staged = self._rows_dev
            self._rows_ring.send(i, staged, staged.shape[1], current)  # the whole (small, contiguous) block
            free = self._free_dev[self._free_cur]
            # the planner takes this reservation's pages from the current front; the ledger logged
            # the take, and the next sync moves the device front past them
            rp, bp = self._rows_ptrs, buffers.ptrs
            _lib.call(
                "nq_plan_ragged",
                rp[0], rp[1], rp[2], rp[3], rp[4], n, capture_rows, token_capacity, self.page_size,
                int(prefill), self._table.data_ptr(), self._table.stride(0),
                free.data_ptr() + 4 * self._free_front, self._free_len - self._free_front, rp[5],
                self._scratch_dev.data_ptr(), len(self._scratch_pages),
                bp[0] or None, bp[1], bp[2], buffers.kv_indices.numel(), bp[3], bp[4], bp[5], bp[6], bp[7], 0,
                current.cuda_stream,
            )
            # the rows' committed page counts (row 3, unchanged by the reservation) and the new pages
            total_pages = int(rows[3, :n].sum()) + reservation.pages_taken + (capture_rows - n)
            metadata = TalkerAttentionMetadata(
                qo_indptr=buffers.qo_indptr,
                paged_kv_indptr=buffers.kv_indptr,
                paged_kv_indices=buffers.kv_indices[:total_pages],
                paged_kv_last_page_len=buffers.last_page_len,
                position_ids=buffers.position_ids,
                write_pages=buffers.write_pages,
                write_offsets=buffers.write_offsets,
                padding_pages=self._scratch_pages,
                reuse_attention_plan=reuse_attention_plan,
            )
            return publications, metadata
        except Exception:
            self.abort(publications)
            raise

    def prepare_prefill(self, context, key, request_ids, sequence_lengths):
        if len(request_ids) != len(sequence_lengths) or len(request_ids) > key.capture_batch_size:
            raise ValueError("Talker prefill request rows do not fit the capture")
        if sum(sequence_lengths) > key.token_capacity:
            raise ValueError("Talker prefill tokens exceed the capture")
        publications, metadata = self._metadata(
            request_ids=tuple(request_ids),
            advances=tuple(sequence_lengths),
            capture_rows=key.capture_batch_size,
            token_capacity=key.token_capacity,
            prefill=True,
            context=context,
        )
        try:
            self._set_metadata(context, metadata)
        except Exception:
            self.abort(publications)
            raise
        return publications

    def prepare_decode(self, context, key, request_ids, *, reuse_attention_plan: bool = True):
        if not request_ids or len(request_ids) > key.capture_batch_size:
            raise ValueError("Talker decode request rows do not fit the capture")
        publications, metadata = self._metadata(
            request_ids=tuple(request_ids),
            advances=(1,) * len(request_ids),
            capture_rows=key.capture_batch_size,
            token_capacity=key.capture_batch_size,
            prefill=False,
            context=context,
            reuse_attention_plan=reuse_attention_plan,
        )
        try:
            self._set_metadata(context, metadata)
        except Exception:
            self.abort(publications)
            raise
        return publications

    def prepare_capture(self, context, key):
        capture_id = self._next_capture
        self._next_capture += 1
        request_ids = tuple(f"__hip_capture_{capture_id}_{row}__" for row in range(key.capture_batch_size))
        for rid in request_ids:
            self.add_request(rid)
        self._capture_requests[id(context)] = request_ids
        if not hasattr(key, "token_capacity"):
            return self.prepare_decode(context, key, request_ids)
        base, extra = divmod(key.token_capacity, key.capture_batch_size)
        lengths = tuple(base + (1 if row < extra else 0) for row in range(key.capture_batch_size))
        return self.prepare_prefill(context, key, request_ids, lengths)

    def finish_capture(self, context, publications) -> None:
        self.abort(publications)
        for rid in self._capture_requests.pop(id(context), ()):
            self.remove_request(rid)

    @staticmethod
    def abort(publications) -> None:
        """Discard every publication (in order; the ledger returns each reservation's pages in one
        piece when its rows come together)."""

        publications = tuple(publications)
        if not publications:
            return
        ledger = publications[0]._ledger
        if all(p._rows.ledger is ledger for p in publications):
            ledger.discard_all(publications)
            return
        for publication in publications:
            publication.discard()


__all__ = [
    "HipDecodeBinding",
    "HipPrefillBinding",
    "PagedTalkerKV",
    "TalkerAttentionMetadata",
]
