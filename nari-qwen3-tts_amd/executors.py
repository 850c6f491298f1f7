"""The reference's executor interfaces over the HIP talker steps and the code-predictor frame.

``build_cuda_execution`` (executor/build.py:61-105) constructs a ``TalkerExecutor`` and a
``CodePredictorExecutor`` and hands them to ``Executor``, which captures every declared key at startup
(executor/executor.py:215-250) and replays them per decision through ``_replay_stage``
(:252-285).  The two classes here keep those interfaces, so they can be injected there unchanged:

- ``HipTalkerExecutor``: ``capture(key)`` for decode keys (``capture_batch_size``) and prefill keys
  (``capture_batch_size``, ``token_capacity``, ``capture_sequence_length``), ``replay(key, values)``
  with the reference's typed row inputs (``TalkerDecodeRowsExecutionInput`` /
  ``TalkerPrefillRowsExecutionInput``: per-row step embedding or prompt tokens and the per-row
  sampling scalars and seen mask), returning a ``TalkerExecutionResult`` (tokens, last hidden state,
  logits, next seen masks, next RNG offsets, pending KV publications) -- executor/talker.py:376-807.
  Each key is captured ``capture_slots`` times; slots rotate under leases and every replay holds the
  submission fence.  The captured operation is the whole HIP step (``TalkerDecodeStep`` /
  ``TalkerPrefillStep``): embedding, 28 layers on the library's kernels, codec head, masks and the
  fused sampler with its seen-mask update.
- ``HipCodePredictorExecutor``: ``whole_frame(values, *, capture_sampler=None)``, ``capture(key)``
  and ``replay(key, values)`` with the two captured sampler routes per key
  (executor/code_predictor.py:159-441; route rule contract/rng.py:20-29).  Both routes draw with
  the library's sampler: the fused route straight from the lm_head's split-K planes, the general
  route from the bf16 logits through ``sampling.sample_logits_cuda_graph``.

Rows are duck-typed: any objects with the reference's field names work, so the reference's own
dataclasses pass through as they are.  The result types below have the reference's field names
(plus ``step_reports`` / ``end_of_speech()`` on the talker result, the device status words of the
step, read without a per-row sync).  Draws come from each row's (seed, offset) through the
library's Philox-4x32-10 uniforms, not Triton's ``tl.rand`` stream.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from .code_predictor import CodePredictorFrame, CodePredictorWeights
from .graphs import GraphPoolFence, HipGraphCaptureDriver, SlotLeases
from .sampling import sample_logits_cuda_graph
from .talker import TalkerDecodeStep, TalkerPrefillStep, TalkerWeights

# contract/rng.py:11-13: 16 codebooks x a Philox stride of 32 per codebook
QWEN3_TTS_CODEBOOKS = 16
PHILOX_CODEBOOK_STRIDE = 32
TALKER_FRAME_OFFSET_STRIDE = QWEN3_TTS_CODEBOOKS * PHILOX_CODEBOOK_STRIDE
MAX_FUSED_RESIDUAL_TOP_K = 64


@dataclass(frozen=True, slots=True)
class TalkerResult:
    tokens: torch.Tensor
    last_hidden: torch.Tensor
    logits: torch.Tensor


@dataclass(frozen=True, slots=True)
class TalkerExecutionResult:
    result: TalkerResult
    next_seen_token_masks: torch.Tensor
    next_sampling_offsets: torch.Tensor
    kv_publications: tuple
    # (StepReport, ticket) of the replayed step: planner / attention / embedding status words and
    # per-row end-of-speech flags, copied to the host once per step
    step_reports: tuple = field(default=())

    def end_of_speech(self) -> np.ndarray:
        """[rows] bool; raises the mapped exception when the step reported a bad status."""

        rows = int(self.result.tokens.shape[0])
        eos = np.zeros(rows, dtype=bool)
        for report, ticket in self.step_reports:
            eos[:] = report.read(ticket)[:rows]
        return eos


@dataclass(frozen=True, slots=True)
class CodePredictorResult:
    frames: torch.Tensor
    codec_sum: torch.Tensor


def _is_prefill_key(key) -> bool:
    return hasattr(key, "token_capacity")


def _route_name(route) -> str:
    return str(getattr(route, "value", route))


def code_predictor_sampler_route(*, temperature: float, top_k: int) -> str:
    """The captured sampler route a row needs (contract/rng.py:20-29): "general" for a sampled row
    whose top-k lies outside 1..64, else "fused"."""

    if temperature > 0 and not 1 <= top_k <= MAX_FUSED_RESIDUAL_TOP_K:
        return "general"
    return "fused"


class _HostStaging:
    """Pinned host arrays for one slot's per-row inputs, sent with one copy per field; the arrays are
    rewritten only after the previous copies from them have completed (``wait``)."""

    def __init__(self, fields: dict[str, tuple[torch.dtype, tuple[int, ...]]]) -> None:
        self.host = {name: torch.zeros(shape, dtype=dtype, pin_memory=True) for name, (dtype, shape) in fields.items()}
        self.view = {name: t.numpy() for name, t in self.host.items()}
        self._done: torch.cuda.Event | None = None

    def wait(self) -> None:
        if self._done is not None:
            self._done.synchronize()

    def send(self, pairs) -> None:
        """(field, device tensor[, count]) pairs: copy the field (its first ``count`` entries)."""

        for name, device, *count in pairs:
            src = self.host[name]
            if count:
                device[: count[0]].copy_(src[: count[0]], non_blocking=True)
            else:
                device.copy_(src, non_blocking=True)
        self._done = torch.cuda.Event()
        self._done.record()


@dataclass
class _TalkerSlot:
    key: object
    context: object
    step: object
    call: object
    leases: SlotLeases
    staging: _HostStaging


_SAMPLING_FIELDS = {"temperature": torch.float32, "top_k": torch.int32, "top_p": torch.float32,
                    "repetition_penalty": torch.float32, "seed": torch.long, "offset": torch.long,
                    "suppress_eos": torch.bool, "text": torch.long}
_PROMPT_FIELDS = {"text_token_ids": torch.long, "codec_token_ids": torch.long, "codec_token_mask": torch.bool}
# padding-row values (executor/talker.py:532-552): greedy, top-k 1, top-p 1, penalty 1, seed 0, offset 0
_SAMPLING_PADDING = {"temperature": 0.0, "top_k": 1, "top_p": 1.0, "repetition_penalty": 1.0, "seed": 0, "offset": 0}


class HipTalkerExecutor:
    """TalkerExecutor's interface (executor/talker.py:135-807) over the HIP decode and prefill steps."""

    def __init__(self, *, weights: TalkerWeights, cache, capture_slots: int,
                 driver: HipGraphCaptureDriver | None = None, submission_fence: GraphPoolFence | None = None) -> None:
        if isinstance(capture_slots, bool) or not isinstance(capture_slots, int) or capture_slots < 1:
            raise ValueError("Talker capture slots must be a positive integer")
        self.weights = weights
        self.config = weights.config
        self.cache = cache
        self.hidden_size = int(weights.config.hidden)
        self.vocab_size = int(weights.config.vocab)
        self.device = weights.codec_head.device
        self.capture_slots = capture_slots
        self.driver = driver or HipGraphCaptureDriver(device=self.device)
        self.submission_fence = submission_fence or GraphPoolFence(device=self.device)
        self._prefill: dict[object, tuple[_TalkerSlot, ...]] = {}
        self._decode: dict[object, tuple[_TalkerSlot, ...]] = {}
        self._next_prefill: dict[object, int] = {}
        self._next_decode: dict[object, int] = {}
        # projection workspace per capture slot index, shared by every key's step of that index (all
        # graphs replay in stream order and keep nothing in it between replays)
        self._workspaces: dict[int, torch.Tensor] = {}

    # -- requests (TalkerExecutor.add_request / remove_request) ------------------
    def add_request(self, request_id: str) -> None:
        self.cache.add_request(request_id)

    def remove_request(self, request_id: str) -> None:
        self.cache.remove_request(request_id)

    @property
    def captured_cuda_graph_instances(self) -> int:
        return sum(len(slots) for slots in (*self._prefill.values(), *self._decode.values()))

    # -- capture -------------------------------------------------------------------
    def capture(self, key) -> None:
        if not hasattr(key, "capture_batch_size"):
            raise TypeError("Talker executor received the wrong capture key")
        prefill = _is_prefill_key(key)
        table, cursor = (self._prefill, self._next_prefill) if prefill else (self._decode, self._next_decode)
        if key in table:
            return
        rows = int(key.capture_batch_size)
        slots = []
        for index in range(self.capture_slots):
            context = self.cache.create_prefill(key, slot=index) if prefill else self.cache.create_decode(key, slot=index)
            workspace = self._workspaces.get(index)
            if prefill:
                step = TalkerPrefillStep(self.weights, context, rows, int(key.token_capacity), workspace=workspace)
            else:
                step = TalkerDecodeStep(self.weights, context, rows, use_counter_rng=True, workspace=workspace)
            if workspace is None or step.linear_workspace.numel() > workspace.numel():
                self._workspaces[index] = step.linear_workspace
            publications = self.cache.prepare_capture(context, key)
            try:
                call = self.driver.capture(step.forward)
            finally:
                self.cache.finish_capture(context, publications)
            fields = {name: (dtype, (rows,)) for name, dtype in _SAMPLING_FIELDS.items()}
            if prefill:
                fields.update({name: (dtype, (int(key.token_capacity),)) for name, dtype in _PROMPT_FIELDS.items()})
            staging = _HostStaging(fields)
            slots.append(_TalkerSlot(key, context, step, call, SlotLeases(), staging))
        table[key] = tuple(slots)
        cursor[key] = 0

    # -- replay --------------------------------------------------------------------
    def replay(self, key, values) -> TalkerExecutionResult:
        submission = self.submission_fence.reserve()
        try:
            if not hasattr(key, "capture_batch_size"):
                raise TypeError("Talker executor received the wrong replay key")
            if _is_prefill_key(key):
                return self._replay_prefill(key, values)
            return self._replay_decode(key, values)
        finally:
            self.submission_fence.release(submission)

    @staticmethod
    def _reserve(key, slots, cursor):
        available = slots.get(key)
        if available is None:
            raise RuntimeError("Talker CUDA Graph has not been captured")
        index = cursor[key]
        cursor[key] = (index + 1) % len(available)
        slot = available[index]
        return slot, slot.leases.reserve()

    def _validate_sampling(self, sources) -> None:
        for source in sources:
            mask = source.seen_token_mask
            if mask is not None and tuple(mask.shape) != (self.vocab_size,):
                raise ValueError("seen_token_mask must match the captured vocabulary")
            if mask is not None and mask.device != self.device:
                raise ValueError("seen_token_mask must be on the execution device")

    def _stage_sampling(self, slot: _TalkerSlot, rows) -> None:
        """Per-row sampling scalars and suppress flags through the slot's pinned arrays (padding rows
        get the neutral values), then the seen masks row by row on the device."""

        step, view = slot.step, slot.staging.view
        n = len(rows)
        slot.staging.wait()
        for name, pad in _SAMPLING_PADDING.items():
            view[name][:n] = [getattr(row.sampling, name) for row in rows]
            view[name][n:] = pad
        view["suppress_eos"][:n] = [row.suppress_eos for row in rows]
        view["suppress_eos"][n:] = True
        step.seen.zero_()
        masks = [(i, row.sampling.seen_token_mask) for i, row in enumerate(rows)
                 if row.sampling.seen_token_mask is not None]
        if masks:
            torch._foreach_copy_([step.seen[i] for i, _ in masks], [m for _, m in masks])

    def _sampling_pairs(self, step):
        return (("temperature", step.temperature), ("top_k", step.top_k), ("top_p", step.top_p),
                ("repetition_penalty", step.penalty), ("seed", step.seed), ("offset", step.offsets),
                ("suppress_eos", step.suppress_eos))

    def _result(self, slot: _TalkerSlot, rows: int, publications, hidden: torch.Tensor) -> TalkerExecutionResult:
        step = slot.step
        slot.call.replay()
        ticket = step.report.fetch()
        return TalkerExecutionResult(
            result=TalkerResult(tokens=step.tokens[:rows].clone(), last_hidden=hidden[:rows].clone(),
                                logits=step.logits[:rows].clone()),
            next_seen_token_masks=step.seen[:rows].clone(),
            next_sampling_offsets=step.offsets[:rows] + TALKER_FRAME_OFFSET_STRIDE,
            kv_publications=tuple(publications),
            step_reports=((step.report, ticket),),
        )

    def _replay_decode(self, key, values) -> TalkerExecutionResult:
        if not hasattr(values, "rows") or not hasattr(values, "request_ids") or _is_prefill_row(values):
            raise TypeError("Talker decode requires a typed Talker decode input")
        slot, lease = self._reserve(key, self._decode, self._next_decode)
        publications = ()
        try:
            rows = len(values.request_ids)
            if len(values.rows) != rows:
                raise ValueError("Talker decode row count does not match request IDs")
            if rows > key.capture_batch_size:
                raise ValueError("Talker decode rows exceed the captured shape")
            if any(row.talker_step_embed.numel() != self.hidden_size for row in values.rows):
                raise ValueError("talker_step_embed must match the captured hidden size")
            if any(row.talker_step_embed.device != self.device for row in values.rows):
                raise ValueError("Talker decode rows must be on the execution device")
            self._validate_sampling(tuple(row.sampling for row in values.rows))
            step = slot.step
            step.step_embed.zero_()
            torch.stack([row.talker_step_embed.reshape(-1) for row in values.rows], out=step.step_embed[:rows])
            self._stage_sampling(slot, values.rows)
            text = slot.staging.view["text"]
            on_host = [row.text_token_id.device.type == "cpu" for row in values.rows]
            text[:rows] = [int(row.text_token_id.reshape(())) if host else 0
                           for row, host in zip(values.rows, on_host)]
            text[rows:] = 0
            slot.staging.send((*self._sampling_pairs(step), ("text", step.text_ids)))
            on_device = [i for i, host in enumerate(on_host) if not host]
            if len(on_device) == rows:
                torch.stack([row.text_token_id.reshape(()) for row in values.rows], out=step.text_ids[:rows])
            else:
                for i in on_device:
                    step.text_ids[i].copy_(values.rows[i].text_token_id.reshape(()))
            publications = self.cache.prepare_decode(slot.context, key, tuple(values.request_ids),
                                                     reuse_attention_plan=getattr(values, "reuse_attention_plan",
                                                                                  False))
            return self._result(slot, rows, publications, step.hidden)
        except Exception:
            if publications:
                self.cache.abort(publications)
            raise
        finally:
            slot.leases.release(lease)

    def _replay_prefill(self, key, values) -> TalkerExecutionResult:
        if not hasattr(values, "rows") or not hasattr(values, "request_ids") or not _is_prefill_row(values):
            raise TypeError("Talker prefill requires a typed Talker prefill input")
        slot, lease = self._reserve(key, self._prefill, self._next_prefill)
        publications = ()
        try:
            rows = len(values.request_ids)
            if len(values.rows) != rows:
                raise ValueError("Talker prefill row count does not match request IDs")
            lengths = tuple(int(row.text_token_ids.numel()) for row in values.rows)
            if rows > key.capture_batch_size or sum(lengths) > key.token_capacity:
                raise ValueError("Talker prefill rows exceed the captured shape")
            if any(row.codec_token_ids.numel() != n or row.codec_token_mask.numel() != n
                   for row, n in zip(values.rows, lengths)):
                raise ValueError("Talker prefill row tensors must have equal sequence lengths")
            source = values.rows[0].text_token_ids.device
            if any(row.text_token_ids.device != source for row in values.rows):
                raise ValueError("Talker prefill rows must share one source device")
            if source.type != "cpu" and source != self.device:
                raise ValueError("Talker prefill rows must be on the host or execution device")
            self._validate_sampling(tuple(row.sampling for row in values.rows))
            step = slot.step
            tokens = sum(lengths)
            self._stage_sampling(slot, values.rows)
            prompt = (("text_token_ids", step.text_ids), ("codec_token_ids", step.codec_ids),
                      ("codec_token_mask", step.codec_mask))
            if source.type == "cpu":
                # host rows pack into the slot's pinned arrays and go over with the sampling scalars
                view = slot.staging.view
                for name, _ in prompt:
                    view[name][:] = 0
                    view[name][:tokens] = np.concatenate([getattr(row, name).reshape(-1).numpy()
                                                          for row in values.rows])
                slot.staging.send((*self._sampling_pairs(step), *prompt))
            else:
                slot.staging.send(self._sampling_pairs(step))
                for name, dst in prompt:
                    dst.zero_()
                    torch.cat([getattr(row, name).reshape(-1) for row in values.rows], out=dst[:tokens])
            publications = self.cache.prepare_prefill(slot.context, key, tuple(values.request_ids), lengths)
            return self._result(slot, rows, publications, step.last_hidden)
        except Exception:
            if publications:
                self.cache.abort(publications)
            raise
        finally:
            slot.leases.release(lease)


def _is_prefill_row(values) -> bool:
    rows = getattr(values, "rows", ())
    return bool(rows) and hasattr(rows[0], "text_token_ids")


@dataclass
class _FrameSlot:
    frame: CodePredictorFrame
    fused_call: object
    general_call: object
    leases: SlotLeases
    staging: _HostStaging
    default_positions: torch.Tensor


_CP_FIELDS = {"temperature": torch.float32, "top_k": torch.int32, "top_p": torch.float32, "seed": torch.long}
_CP_PADDING = {"temperature": 0.0, "top_k": 1, "top_p": 1.0, "seed": 0}


class HipCodePredictorExecutor:
    """CodePredictorExecutor's interface (executor/code_predictor.py:42-441) over the HIP frame."""

    def __init__(self, *, weights: CodePredictorWeights, max_batch_size: int,
                 driver: HipGraphCaptureDriver | None = None, submission_fence: GraphPoolFence | None = None) -> None:
        if isinstance(max_batch_size, bool) or not isinstance(max_batch_size, int) or max_batch_size < 1:
            raise ValueError("Code Predictor max_batch_size must be a positive integer")
        if max_batch_size > 128:
            raise ValueError("the HIP code-predictor frame runs at most 128 rows")
        self.weights = weights
        self.config = weights.config
        self.max_batch_size = max_batch_size
        self.hidden_size = int(weights.config.talker_hidden)
        self.num_code_groups = int(weights.config.num_code_groups)
        self.device = weights.lm_head.device
        self.driver = driver or HipGraphCaptureDriver(device=self.device)
        self.submission_fence = submission_fence or GraphPoolFence(device=self.device)
        self._slots: dict[object, _FrameSlot] = {}
        self._eager: dict[int, CodePredictorFrame] = {}

    @property
    def capture_instances_per_key(self) -> int:
        return 2

    @property
    def captured_cuda_graph_instances(self) -> int:
        return len(self._slots) * self.capture_instances_per_key

    # -- the direct frame ------------------------------------------------------------
    def whole_frame(self, values, *, capture_sampler=None) -> CodePredictorResult:
        """One frame of ``values`` (CodePredictorInput: per-row tensors) run eagerly: the fused draw
        when ``capture_sampler`` is None, else that sampler on each group's logits."""

        if values.num_code_groups != self.num_code_groups:
            raise ValueError("Code Predictor whole-frame jobs require the configured code groups: "
                             f"got {values.num_code_groups}, expected {self.num_code_groups}")
        rows = int(values.layer0_token.shape[0])
        if not 1 <= rows <= self.max_batch_size:
            raise ValueError(f"Code Predictor batch {rows} exceeds max_batch_size={self.max_batch_size}")
        if capture_sampler is None:
            for name, value in (("temperature", values.temperature), ("top_p", values.top_p)):
                if not bool(torch.all(torch.isfinite(value))):
                    raise ValueError(f"Code Predictor {name} must contain only finite values")
            if torch.any(values.temperature < 0):
                raise ValueError("Code Predictor temperature must be non-negative")
            if torch.any(values.top_k < 0):
                raise ValueError("Code Predictor top_k must be non-negative")
            if torch.any((values.top_p <= 0) | (values.top_p > 1)):
                raise ValueError("Code Predictor top_p must be in (0, 1]")
            if torch.any(values.seed < 0) or torch.any(values.offsets < 0):
                raise ValueError("Code Predictor seed and offsets must be non-negative")
        frame = self._eager.get(rows)
        if frame is None:
            frame = self._eager[rows] = CodePredictorFrame(self.weights, rows, use_counter_rng=True)
        frame.layer0_token.copy_(values.layer0_token)
        frame.past_hidden.copy_(values.past_hidden)
        frame.temperature.copy_(values.temperature)
        frame.top_k.copy_(values.top_k)
        frame.top_p.copy_(values.top_p)
        frame.seed.copy_(values.seed)
        frame.offsets.copy_(values.offsets)
        positions = values.position_ids
        if positions is None:
            frame.position_ids.copy_(torch.arange(self.num_code_groups, device=self.device).expand(rows, -1))
        else:
            frame.position_ids.copy_(positions)
        frame.sampler = capture_sampler
        try:
            frames, codec_sum = frame.forward()
        finally:
            frame.sampler = None
        return CodePredictorResult(frames=frames.clone(), codec_sum=codec_sum.clone())

    # -- captured frames ---------------------------------------------------------------
    def capture(self, key) -> None:
        if not hasattr(key, "capture_batch_size") or hasattr(key, "token_capacity"):
            raise TypeError("Code Predictor executor received the wrong capture key")
        if key in self._slots:
            return
        rows = int(key.capture_batch_size)
        if rows > self.max_batch_size:
            raise ValueError(f"Code Predictor batch {rows} exceeds max_batch_size={self.max_batch_size}")
        frame = CodePredictorFrame(self.weights, rows, use_counter_rng=True)
        frame.sampler = None
        fused = self.driver.capture(frame.forward)
        frame.sampler = sample_logits_cuda_graph
        general = self.driver.capture(frame.forward)
        frame.sampler = None
        fields = {name: (dtype, (rows,)) for name, dtype in _CP_FIELDS.items()}
        fields["offsets"] = (torch.long, (rows, self.num_code_groups - 1))
        self._slots[key] = _FrameSlot(frame, fused, general, SlotLeases(), _HostStaging(fields),
                                      frame.position_ids.clone())

    def replay(self, key, values) -> CodePredictorResult:
        submission = self.submission_fence.reserve()
        try:
            return self._replay_owned(key, values)
        finally:
            self.submission_fence.release(submission)

    def _replay_owned(self, key, values) -> CodePredictorResult:
        if not hasattr(key, "capture_batch_size") or hasattr(key, "token_capacity"):
            raise TypeError("Code Predictor executor received the wrong capture key")
        if not hasattr(values, "rows") or not hasattr(values, "sampler_route"):
            raise TypeError("Code Predictor replay requires a typed Code Predictor input")
        slot = self._slots.get(key)
        if slot is None:
            raise RuntimeError("Code Predictor CUDA Graph has not been captured")
        n = len(values.rows)
        if n > key.capture_batch_size:
            raise ValueError("Code Predictor input exceeds its captured shape")
        lease = slot.leases.reserve()
        try:
            groups = self.num_code_groups
            if any(len(row.offsets) != groups - 1 for row in values.rows):
                raise ValueError("Code Predictor row RNG offsets do not cover every residual codebook")
            route = _route_name(values.sampler_route)
            if {code_predictor_sampler_route(temperature=row.temperature, top_k=row.top_k)
                    for row in values.rows} != {route}:
                raise ValueError("Code Predictor rows must match one homogeneous sampler route")
            if any(row.past_hidden.numel() != self.hidden_size for row in values.rows):
                raise ValueError("Code Predictor row past_hidden does not match the captured hidden size")
            if any(row.layer0_token.device != self.device for row in values.rows):
                raise ValueError("Code Predictor rows must be on the execution device")
            if any(row.position_ids is not None and (row.position_ids.numel() != groups
                                                     or row.position_ids.dtype is not torch.long)
                   for row in values.rows):
                raise ValueError("Code Predictor row position IDs do not match the captured shape")
            frame = slot.frame
            frame.layer0_token.zero_()
            frame.past_hidden.zero_()
            torch.stack([row.layer0_token.reshape(()) for row in values.rows], out=frame.layer0_token[:n])
            torch.stack([row.past_hidden.reshape(-1).to(frame.past_hidden.dtype) for row in values.rows],
                        out=frame.past_hidden[:n])
            frame.position_ids.copy_(slot.default_positions)
            for i, row in enumerate(values.rows):
                if row.position_ids is not None:
                    frame.position_ids[i].copy_(row.position_ids.reshape(-1))
            staging, view = slot.staging, slot.staging.view
            staging.wait()
            for name, pad in _CP_PADDING.items():
                view[name][:n] = [getattr(row, name) for row in values.rows]
                view[name][n:] = pad
            view["offsets"][:n] = [row.offsets for row in values.rows]
            view["offsets"][n:] = 0
            staging.send((("temperature", frame.temperature), ("top_k", frame.top_k), ("top_p", frame.top_p),
                          ("seed", frame.seed), ("offsets", frame.offsets)))
            call = slot.general_call if route == "general" else slot.fused_call
            frames, codec_sum = call.replay()
            return CodePredictorResult(frames=frames[:n].clone(), codec_sum=codec_sum[:n].clone())
        finally:
            slot.leases.release(lease)


__all__ = ["CodePredictorResult", "HipCodePredictorExecutor", "HipTalkerExecutor", "TalkerExecutionResult",
           "TalkerResult", "code_predictor_sampler_route"]
