"""The captured talker decode buckets of the serving path.

Follows TalkerExecutor._capture_decode / _reserve / _replay_decode (executor/talker.py:461-560,
:592-607) over the balanced profile's decode catalog (profiles/balanced.yaml:10-12, 33): every bucket
size is captured ``capture_slots`` times, each capture slot with its own static inputs, attention
binding and hipGraph; a bucket's slots are taken in rotation, each under a lease; all captures share
one graph memory pool, so a decision runs under one pool fence.  Bindings and decode steps of one
slot index share that slot's attention workspace and projection workspace (their graphs never run at
the same time), as executor/talker_kv.py:361 shares FlashInfer workspaces.

A decision's logical rows are lowered onto the buckets (planner/catalog.py:43-71: full largest
buckets, then the smallest bucket that holds the rest, padded).  Padding rows get the reference's
neutral sampling inputs (greedy, top-k 1, top-p 1, penalty 1, seed 0, offset 0; executor/talker.py:
532-552).  Each part is planned and replayed before the next is planned, so parts that land on the
same slot index never see each other's attention plan.  ``decode`` returns without waiting for the
GPU: the result's ``end_of_speech()`` reads the step reports (one copy per part) when the caller is
ready to finalize.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from .errors import CaptureCoverageError
from .graphs import GraphPoolFence, HipGraphCaptureDriver, SlotLeases, lower_rows
from .talker import TalkerDecodeStep, TalkerPrefillStep, TalkerWeights

DECODE_BUCKETS = (1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 16, 24, 32, 40, 48, 56, 64)
CAPTURE_SLOTS = 4


class DecodeKey:
    """TalkerDecodeCaptureKey's shape field (contract of TalkerKVBackend.create_decode)."""

    def __init__(self, capture_batch_size: int) -> None:
        self.capture_batch_size = capture_batch_size


@dataclass(frozen=True)
class DecodeRows:
    """One decision's logical rows, staged by the executor (device tensors, first dim = rows)."""

    request_ids: tuple[str, ...]
    step_embed: torch.Tensor  # [n, hidden] bf16
    text_ids: torch.Tensor  # [n] int64
    temperature: torch.Tensor  # [n] fp32
    top_k: torch.Tensor  # [n] int32
    top_p: torch.Tensor  # [n] fp32
    repetition_penalty: torch.Tensor  # [n] fp32
    seed: torch.Tensor  # [n] int64
    offsets: torch.Tensor  # [n] int64
    seen: torch.Tensor  # [n, vocab] bool
    suppress_eos: torch.Tensor  # [n] bool


@dataclass(frozen=True)
class DecodeResult:
    """A submitted decision.  The device outputs are valid in stream order at once; the host learns
    whether the step succeeded and which rows reached end-of-speech from ``end_of_speech()``, which
    waits for the decision's report copies (one per part) -- the host finalize of
    engine/pipeline.py:585-610 with one copy per part instead of one ``.item()`` per row.
    ``completion_fence`` (ready / wait) lets a submission window keep several decisions in flight."""

    tokens: torch.Tensor  # [n] int64
    logits: torch.Tensor  # [n, vocab] bf16
    seen: torch.Tensor  # [n, vocab] bool, with this step's token marked
    publications: tuple
    parts: tuple  # (bucket, slot) per lowered part
    reports: tuple  # (StepReport, ticket, first row, end row) per part
    completion_fence: object

    def end_of_speech(self) -> np.ndarray:
        """[n] bool; raises the mapped error (fail closed) if any part reported a bad status."""

        n = self.tokens.shape[0]
        eos = np.zeros(n, dtype=bool)
        for report, ticket, a, b in self.reports:
            eos[a:b] = report.read(ticket)[: b - a]
        return eos


@dataclass
class _Slot:
    key: object
    context: object
    step: object
    call: object
    leases: SlotLeases


class TalkerDecodeCatalog:
    def __init__(self, weights: TalkerWeights, kv, *, buckets: tuple[int, ...] = DECODE_BUCKETS,
                 capture_slots: int = CAPTURE_SLOTS, use_counter_rng: bool = True,
                 driver: HipGraphCaptureDriver | None = None) -> None:
        if not buckets or any(int(b) < 1 for b in buckets) or capture_slots < 1:
            raise ValueError("the decode catalog needs positive bucket sizes and at least one capture slot")
        self.weights = weights
        self.kv = kv
        self.buckets = tuple(sorted(set(int(b) for b in buckets)))
        self.capture_slots = capture_slots
        self.device = weights.codec_head.device
        self.driver = driver or HipGraphCaptureDriver(device=self.device)
        self.fence = GraphPoolFence(device=self.device)
        self._slots: dict[int, tuple[_Slot, ...]] = {}
        self._next: dict[int, int] = {}
        workspaces: dict[int, torch.Tensor] = {}
        # largest bucket first: each slot index's projection workspace is sized once, by it
        for rows in reversed(self.buckets):
            captured = []
            for index in range(capture_slots):
                key = DecodeKey(rows)
                context = kv.create_decode(key, slot=index)
                step = TalkerDecodeStep(weights, context, rows, use_counter_rng=use_counter_rng,
                                        workspace=workspaces.get(index))
                workspaces.setdefault(index, step.linear_workspace)
                publications = kv.prepare_capture(context, key)
                try:
                    call = self.driver.capture(step.forward)
                finally:
                    kv.finish_capture(context, publications)
                captured.append(_Slot(key, context, step, call, SlotLeases()))
            self._slots[rows] = tuple(captured)
            self._next[rows] = 0

    def lower(self, rows: int):
        return lower_rows(rows, self.buckets)

    def _take(self, bucket: int) -> tuple[int, _Slot, int]:
        index = self._next[bucket]
        self._next[bucket] = (index + 1) % self.capture_slots
        slot = self._slots[bucket][index]
        return index, slot, slot.leases.reserve()

    @staticmethod
    def _stage(step: TalkerDecodeStep, rows: DecodeRows, a: int, b: int) -> None:
        k = b - a
        for dst, src, pad in ((step.step_embed, rows.step_embed, 0), (step.text_ids, rows.text_ids, 0),
                              (step.temperature, rows.temperature, 0), (step.top_k, rows.top_k, 1),
                              (step.top_p, rows.top_p, 1), (step.penalty, rows.repetition_penalty, 1),
                              (step.seed, rows.seed, 0), (step.offsets, rows.offsets, 0), (step.seen, rows.seen, 0),
                              (step.suppress_eos, rows.suppress_eos, 0)):
            dst[:k].copy_(src[a:b])
            if k < dst.shape[0]:
                dst[k:].fill_(pad)

    def decode(self, rows: DecodeRows) -> DecodeResult:
        n = len(rows.request_ids)
        if n < 1:
            raise ValueError("a decode decision needs at least one row")
        for name in ("step_embed", "text_ids", "temperature", "top_k", "top_p", "repetition_penalty", "seed",
                     "offsets", "seen", "suppress_eos"):
            if getattr(rows, name).shape[0] != n:
                raise ValueError(f"decode rows: {name} does not have one entry per request")
        vocab = self.weights.config.vocab
        tokens = torch.empty(n, dtype=torch.long, device=self.device)
        logits = torch.empty(n, vocab, dtype=torch.bfloat16, device=self.device)
        seen = torch.empty(n, vocab, dtype=torch.bool, device=self.device)
        publications: list = []
        tickets: list = []
        parts = []
        fence = self.fence.reserve()
        try:
            for part in self.lower(n):
                a, b = part.start, part.stop
                index, slot, lease = self._take(part.capture_rows)
                try:
                    step = slot.step
                    self._stage(step, rows, a, b)
                    pubs = self.kv.prepare_decode(slot.context, slot.key, rows.request_ids[a:b])
                    try:
                        slot.call.replay()
                        tickets.append((slot, step.report.fetch(), a, b))
                    except Exception:
                        self.kv.abort(pubs)
                        raise
                    publications.extend(pubs)
                    tokens[a:b].copy_(step.tokens[: b - a])
                    logits[a:b].copy_(step.logits[: b - a])
                    seen[a:b].copy_(step.seen[: b - a])
                    parts.append((part.capture_rows, index))
                finally:
                    slot.leases.release(lease)
        except Exception:
            self.kv.abort(tuple(publications))
            raise
        finally:
            self.fence.release(fence)
        reports = tuple((slot.step.report, ticket, a, b) for slot, ticket, a, b in tickets)
        last_report, last_ticket = reports[-1][0], reports[-1][1]
        return DecodeResult(tokens, logits, seen, tuple(publications), tuple(parts), reports,
                            last_report.fence(last_ticket))


# The balanced profile's prefill catalog (profiles/balanced.yaml:4-9): token buckets for batch sizes
# 1, 2, 4, 8 and exact 10-token captures for 1..8 rows.
PREFILL_BATCH_SIZES = (1, 2, 4, 8)
PREFILL_TOKEN_BUCKETS = (32, 64, 128, 192, 384, 640)
PREFILL_EXACT_SEQUENCE_LENGTHS = (10,)
PREFILL_EXACT_BATCH_SIZES = (1, 2, 3, 4, 5, 6, 7, 8)
PREFILL_MAX_BATCH = 8


@dataclass(frozen=True)
class PrefillKey:
    """TalkerPrefillCaptureKey (contract/stage.py:39-48): rows, packed token capacity and, for an
    exact capture, the one sequence length it was built for."""

    capture_batch_size: int
    token_capacity: int
    capture_sequence_length: int | None = None

    def __post_init__(self) -> None:
        for name in ("capture_batch_size", "token_capacity"):
            value = getattr(self, name)
            if isinstance(value, bool) or not isinstance(value, int) or value < 1:
                raise ValueError(f"{name.replace('_', ' ')} must be a positive integer")
        length = self.capture_sequence_length
        if length is not None and (isinstance(length, bool) or not isinstance(length, int) or length < 1):
            raise ValueError("capture sequence length must be a positive integer")


def prefill_keys(*, batch_sizes=PREFILL_BATCH_SIZES, token_buckets=PREFILL_TOKEN_BUCKETS,
                 exact_sequence_lengths=PREFILL_EXACT_SEQUENCE_LENGTHS,
                 exact_batch_sizes=PREFILL_EXACT_BATCH_SIZES) -> frozenset:
    """Every prefill capture of a profile (CaptureCatalog.from_config, planner/catalog.py:86-97)."""

    exact = {PrefillKey(b, b * s, s) for s in exact_sequence_lengths for b in exact_batch_sizes}
    return frozenset(exact | {PrefillKey(b, t) for b in batch_sizes for t in token_buckets})


@dataclass(frozen=True)
class PrefillSlice:
    key: PrefillKey
    start: int
    stop: int
    capture_rows: int
    padding: int


def lower_prefill(sequence_lengths: tuple[int, ...], keys, max_batch_size: int = PREFILL_MAX_BATCH):
    """Pack consecutive requests into prefill captures (lower_talker_prefill, planner/catalog.py:
    262-314): a part takes requests while it has fewer than ``max_batch_size`` and their tokens fit
    the largest token capacity; it runs on the capture that covers its rows and tokens with the
    least token capacity, then the fewest rows, then exact before bucketed (a key's
    ``capture_sequence_length is None`` sorts False first), then the shorter exact length -- the
    reference's min() key (planner/catalog.py:296-303)."""

    if not isinstance(sequence_lengths, tuple) or not sequence_lengths:
        raise ValueError("Talker prefill sequence lengths must be a non-empty tuple")
    if any(isinstance(n, bool) or not isinstance(n, int) or n <= 0 for n in sequence_lengths):
        raise ValueError("Talker prefill sequence lengths must be positive integers")
    keys = tuple(keys)
    most = max(k.token_capacity for k in keys)
    order = sorted(keys, key=lambda k: (k.token_capacity, k.capture_batch_size, k.capture_sequence_length is None,
                                        k.capture_sequence_length or 0))
    parts = []
    start = 0
    count = len(sequence_lengths)
    while start < count:
        if sequence_lengths[start] > most:
            raise CaptureCoverageError("Talker prefill capture token capacity exceeded")
        stop, tokens = start, 0
        while stop < count and stop - start < max_batch_size and tokens + sequence_lengths[stop] <= most:
            tokens += sequence_lengths[stop]
            stop += 1
        rows = stop - start
        key = next((k for k in order if k.capture_batch_size >= rows and k.token_capacity >= tokens), None)
        if key is None:
            raise CaptureCoverageError(f"no Talker prefill capture covers {rows} rows and {tokens} tokens")
        parts.append(PrefillSlice(key, start, stop, key.capture_batch_size, key.capture_batch_size - rows))
        start = stop
    return tuple(parts)


@dataclass(frozen=True)
class PrefillRows:
    """One prefill decision's requests, staged by the executor: the rows' prompt tokens packed in row
    order (device tensors of sum(lengths) entries) and per-row sampling inputs (first dim = rows)."""

    request_ids: tuple[str, ...]
    lengths: tuple[int, ...]
    text_ids: torch.Tensor  # [tokens] int64
    codec_ids: torch.Tensor  # [tokens] int64
    codec_mask: torch.Tensor  # [tokens] bool
    temperature: torch.Tensor  # [n] fp32
    top_k: torch.Tensor  # [n] int32
    top_p: torch.Tensor  # [n] fp32
    repetition_penalty: torch.Tensor  # [n] fp32
    seed: torch.Tensor  # [n] int64
    offsets: torch.Tensor  # [n] int64
    seen: torch.Tensor  # [n, vocab] bool
    suppress_eos: torch.Tensor  # [n] bool


@dataclass(frozen=True)
class PrefillResult:
    """A submitted prefill decision (TalkerExecutionResult of executor/rows.py:126-130 over every
    part): tokens, last-token hidden states, logits and next seen masks of the rows, the pending
    KV publications, and the parts' step reports (``end_of_speech()`` reads them, fail closed)."""

    tokens: torch.Tensor  # [n] int64
    last_hidden: torch.Tensor  # [n, hidden] bf16
    logits: torch.Tensor  # [n, vocab] bf16
    seen: torch.Tensor  # [n, vocab] bool
    publications: tuple
    parts: tuple  # (key, slot) per lowered part
    reports: tuple
    completion_fence: object

    end_of_speech = DecodeResult.end_of_speech


class TalkerPrefillCatalog:
    """Every prefill capture key x ``capture_slots`` captured prefill steps sharing one graph pool
    (TalkerExecutor._capture_prefill, executor/talker.py:397-459); decisions are lowered with
    ``lower_prefill`` and replayed part by part like the decode catalog (slot rotation under leases,
    one pool fence).  Steps of one slot index share the slot's projection workspace."""

    def __init__(self, weights: TalkerWeights, kv, *, keys=None, capture_slots: int = CAPTURE_SLOTS,
                 max_batch_size: int = PREFILL_MAX_BATCH, driver: HipGraphCaptureDriver | None = None,
                 fence: GraphPoolFence | None = None) -> None:
        keys = prefill_keys() if keys is None else frozenset(keys)
        if not keys or capture_slots < 1:
            raise ValueError("the prefill catalog needs at least one key and one capture slot")
        self.weights = weights
        self.kv = kv
        self.keys = keys
        self.capture_slots = capture_slots
        self.max_batch_size = max_batch_size
        self.device = weights.codec_head.device
        self.driver = driver or HipGraphCaptureDriver(device=self.device)
        self.fence = fence or GraphPoolFence(device=self.device)
        self._slots: dict[PrefillKey, tuple[_Slot, ...]] = {}
        self._next: dict[PrefillKey, int] = {}
        workspaces: dict[int, torch.Tensor] = {}
        for key in sorted(keys, key=lambda k: (-k.token_capacity, -k.capture_batch_size)):
            captured = []
            for index in range(capture_slots):
                context = kv.create_prefill(key, slot=index)
                step = TalkerPrefillStep(weights, context, key.capture_batch_size, key.token_capacity,
                                         workspace=workspaces.get(index))
                workspaces.setdefault(index, step.linear_workspace)
                publications = kv.prepare_capture(context, key)
                try:
                    call = self.driver.capture(step.forward)
                finally:
                    kv.finish_capture(context, publications)
                captured.append(_Slot(key, context, step, call, SlotLeases()))
            self._slots[key] = tuple(captured)
            self._next[key] = 0

    def lower(self, lengths: tuple[int, ...]):
        return lower_prefill(tuple(lengths), self.keys, self.max_batch_size)

    def _take(self, key: PrefillKey):
        index = self._next[key]
        self._next[key] = (index + 1) % self.capture_slots
        slot = self._slots[key][index]
        return index, slot, slot.leases.reserve()

    @staticmethod
    def _stage(step: TalkerPrefillStep, rows: PrefillRows, a: int, b: int, t0: int, t1: int) -> None:
        k, t = b - a, t1 - t0
        for dst, src in ((step.text_ids, rows.text_ids), (step.codec_ids, rows.codec_ids),
                         (step.codec_mask, rows.codec_mask)):
            dst[:t].copy_(src[t0:t1])
            if t < dst.shape[0]:
                dst[t:].fill_(0)
        for dst, src, pad in ((step.temperature, rows.temperature, 0), (step.top_k, rows.top_k, 1),
                              (step.top_p, rows.top_p, 1), (step.penalty, rows.repetition_penalty, 1),
                              (step.seed, rows.seed, 0), (step.offsets, rows.offsets, 0), (step.seen, rows.seen, 0),
                              (step.suppress_eos, rows.suppress_eos, 1)):
            dst[:k].copy_(src[a:b])
            if k < dst.shape[0]:
                dst[k:].fill_(pad)

    def prefill(self, rows: PrefillRows) -> PrefillResult:
        n = len(rows.request_ids)
        if n < 1 or len(rows.lengths) != n:
            raise ValueError("Talker prefill row count does not match request IDs")
        total = sum(rows.lengths)
        for name in ("text_ids", "codec_ids", "codec_mask"):
            if getattr(rows, name).shape != (total,):
                raise ValueError("Talker prefill row tensors must have equal sequence lengths")
        for name in ("temperature", "top_k", "top_p", "repetition_penalty", "seed", "offsets", "seen",
                     "suppress_eos"):
            if getattr(rows, name).shape[0] != n:
                raise ValueError(f"prefill rows: {name} does not have one entry per request")
        c = self.weights.config
        tokens = torch.empty(n, dtype=torch.long, device=self.device)
        hidden = torch.empty(n, c.hidden, dtype=torch.bfloat16, device=self.device)
        logits = torch.empty(n, c.vocab, dtype=torch.bfloat16, device=self.device)
        seen = torch.empty(n, c.vocab, dtype=torch.bool, device=self.device)
        starts = np.concatenate([[0], np.cumsum(rows.lengths)])
        publications: list = []
        tickets: list = []
        parts = []
        fence = self.fence.reserve()
        try:
            for part in self.lower(tuple(rows.lengths)):
                a, b = part.start, part.stop
                index, slot, lease = self._take(part.key)
                try:
                    step = slot.step
                    self._stage(step, rows, a, b, int(starts[a]), int(starts[b]))
                    pubs = self.kv.prepare_prefill(slot.context, part.key, rows.request_ids[a:b], rows.lengths[a:b])
                    try:
                        slot.call.replay()
                        tickets.append((slot, step.report.fetch(), a, b))
                    except Exception:
                        self.kv.abort(pubs)
                        raise
                    publications.extend(pubs)
                    k = b - a
                    tokens[a:b].copy_(step.tokens[:k])
                    hidden[a:b].copy_(step.last_hidden[:k])
                    logits[a:b].copy_(step.logits[:k])
                    seen[a:b].copy_(step.seen[:k])
                    parts.append((part.key, index))
                finally:
                    slot.leases.release(lease)
        except Exception:
            self.kv.abort(tuple(publications))
            raise
        finally:
            self.fence.release(fence)
        reports = tuple((slot.step.report, ticket, a, b) for slot, ticket, a, b in tickets)
        return PrefillResult(tokens, hidden, logits, seen, tuple(publications), tuple(parts), reports,
                             reports[-1][0].fence(reports[-1][1]))


__all__ = ["CAPTURE_SLOTS", "DECODE_BUCKETS", "PREFILL_BATCH_SIZES", "PREFILL_EXACT_BATCH_SIZES",
           "PREFILL_EXACT_SEQUENCE_LENGTHS", "PREFILL_MAX_BATCH", "PREFILL_TOKEN_BUCKETS", "DecodeKey", "DecodeResult",
           "DecodeRows", "PrefillKey", "PrefillResult", "PrefillRows", "PrefillSlice", "TalkerDecodeCatalog",
           "TalkerPrefillCatalog", "lower_prefill", "prefill_keys"]
