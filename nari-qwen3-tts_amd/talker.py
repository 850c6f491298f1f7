"""One talker decode step on the GPU: the unit the serving metric counts.

Follows the reference step (executor/talker.py:231-262, 341-374 and
model/components.py:29-90): decode embedding = step embed + projected text
embedding, then per layer input norm, packed QKV projection, fused
qk-norm/RoPE/paged KV write + paged attention (TalkerAttentionContext.attend),
o-proj, fused residual add + RMSNorm, SwiGLU MLP and the next fused add-norm;
the codec head; the fused sampler (logit masks, repetition penalty over the
seen mask, temperature, top-k, top-p, draw) with the seen-mask update.

The projections run on the HIP library's skinny GEMM with the following
kernel fused in (o_proj and down with the residual add-RMSNorm, gate_up with
SiLU-mul); a decode bucket holds at most 128 rows, and larger shapes are
refused (ValueError) rather than sent to another GEMM backend.  With ``fp8_gate_up`` (the default, as the reference's serving
build requires FP8 gate/up for every talker layer, executor/build.py:73 and
executor/optimizations.py:22-46) the gate/up weights are held as 128 x 128
FP8 blocks, the post-attention add-RMSNorm stores its output quantized per
128 columns, and gate/up runs as the block-scaled FP8 product
(model/layers.py:226-262).  Weights are random (N(0, 0.02), norm weights 1)
because no checkpoint is available; shapes follow the Qwen3-TTS 1.7B talker.
"""

from __future__ import annotations

from dataclasses import dataclass
from types import SimpleNamespace

import torch

from . import _lib
from .layers import (
    FP8,
    embed_add_rmsnorm,
    gather_sum_rows,
    linear,
    linear_add_rmsnorm,
    linear_add_rmsnorm_fp8,
    linear_fp8_swiglu,
    linear_fp8_workspace_bytes,
    pack_fp8_swiglu,
    linear_partials,
    linear_silu_mul,
    linear_workspace_bytes,
    prefill_embed_rmsnorm,
    quantize_fp8_weight_blocks,
    tgemm,
    tgemm_add_rmsnorm_fp8,
    tgemm_fp8_swiglu,
    tgemm_partials,
    tgemm_workspace_bytes,
)
from .errors import KVAllocationError
from .sampling import sample_with_counter, sample_with_counter_from_planes, sample_with_uniforms


@dataclass(frozen=True)
class TalkerConfig:
    num_layers: int = 28
    hidden: int = 2048
    num_qo_heads: int = 16
    num_kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 6144
    vocab: int = 3072
    text_vocab: int = 4096
    codec_vocab: int = 2048  # ids >= this are suppressed except EOS (executor/talker.py:173-183)
    eos_id: int = 2150
    rms_eps: float = 1e-6
    rope_theta: float = 1_000_000.0

    @property
    def qkv_width(self) -> int:
        return (self.num_qo_heads + 2 * self.num_kv_heads) * self.head_dim


class TalkerWeights:
    """Random-init talker parameters in bf16 on one device; with ``fp8_gate_up`` each layer also
    holds its gate/up weights as FP8 blocks (``gate_up_q``, ``gate_up_scales``), as
    GatedMLP.initialize_fp8_gate_up_weight prepares them (model/layers.py:226-239)."""

    def __init__(self, config: TalkerConfig, device: torch.device, seed: int = 0, std: float = 0.02,
                 fp8_gate_up: bool = True) -> None:
        self.config = config
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        c = config
        bf = dict(dtype=torch.bfloat16, device=device)

        def randn(*shape):
            return (torch.randn(*shape, generator=g, device=device, dtype=torch.float32) * std).to(torch.bfloat16)

        self.layers = []
        for _ in range(c.num_layers):
            self.layers.append(
                SimpleNamespace(
                    input_norm=torch.ones(c.hidden, **bf),
                    qkv=randn(c.qkv_width, c.hidden),
                    o=randn(c.hidden, c.num_qo_heads * c.head_dim),
                    post_norm=torch.ones(c.hidden, **bf),
                    gate_up=randn(2 * c.intermediate, c.hidden),
                    down=randn(c.hidden, c.intermediate),
                    attention=SimpleNamespace(
                        q_norm=SimpleNamespace(weight=torch.ones(c.head_dim, **bf), variance_epsilon=c.rms_eps),
                        k_norm=SimpleNamespace(weight=torch.ones(c.head_dim, **bf), variance_epsilon=c.rms_eps),
                        rope_theta=c.rope_theta,
                    ),
                )
            )
        self.final_norm = torch.ones(c.hidden, **bf)
        self.codec_head = randn(c.vocab, c.hidden)
        self.text_embedding = randn(c.text_vocab, c.hidden)
        # codec token embeddings (Qwen3TTSTalkerInnerModel.codec_embedding, model/components.py:71)
        self.codec_embedding = randn(c.vocab, c.hidden)
        self._derive(fp8_gate_up)

    def _derive(self, fp8_gate_up: bool) -> None:
        self.fp8_gate_up = fp8_gate_up
        for layer in self.layers:
            layer.gate_up_q, layer.gate_up_scales = (
                quantize_fp8_weight_blocks(layer.gate_up) if fp8_gate_up else (None, None))
            # the same codes with gate/up rows interleaved for the fused SwiGLU kernel
            layer.gate_up_packed = pack_fp8_swiglu(layer.gate_up_q) if fp8_gate_up else None

    @classmethod
    def from_reference_model(cls, model, config, *, fp8_gate_up: bool = True) -> "TalkerWeights":
        """The parameters of a loaded reference talker: ``model`` a ``Qwen3TTSTalkerModel``
        (model/components.py:93-130; its projected text-embedding cache initialised, as
        ``initialize_projected_text_embedding_cache`` does at load) and ``config`` the reference's
        ``Qwen3TTSConfig`` (model/config.py:66-118).  Every tensor is the model's own, as contiguous
        bf16 on the model's device: per layer the input / post-attention norms, the packed QKV and
        o projections, the q/k norms and the packed [gate; up] and down projections; the final norm,
        the codec head, the projected text embedding and the codec embedding.  The FP8 gate/up blocks
        are made from the bf16 weights as GatedMLP.initialize_fp8_gate_up_weight makes them
        (model/layers.py:226-239)."""

        t = config.talker
        c = TalkerConfig(num_layers=int(t.num_hidden_layers), hidden=int(t.hidden_size),
                         num_qo_heads=int(t.num_attention_heads), num_kv_heads=int(t.num_key_value_heads),
                         head_dim=int(t.head_dim), intermediate=int(t.intermediate_size), vocab=int(t.vocab_size),
                         text_vocab=int(t.text_vocab_size), codec_vocab=int(t.code_predictor.vocab_size),
                         eos_id=int(t.codec_eos_token_id), rms_eps=float(t.rms_norm_eps),
                         rope_theta=float(t.rope_theta))
        inner = model.model
        if len(inner.layers) != c.num_layers:
            raise ValueError(f"the model has {len(inner.layers)} layers, the config {c.num_layers}")

        def bf(x, shape):
            x = x.detach()
            if tuple(x.shape) != tuple(shape):
                raise ValueError(f"reference weight of shape {tuple(x.shape)} where {tuple(shape)} was expected")
            return x.to(torch.bfloat16).contiguous()

        self = cls.__new__(cls)
        self.config = c
        self.layers = []
        for L in inner.layers:
            a, mlp = L.self_attn, L.mlp
            self.layers.append(SimpleNamespace(
                input_norm=bf(L.input_layernorm.weight, (c.hidden,)),
                qkv=bf(a.qkv_proj.weight, (c.qkv_width, c.hidden)),
                o=bf(a.o_proj.weight, (c.hidden, c.num_qo_heads * c.head_dim)),
                post_norm=bf(L.post_attention_layernorm.weight, (c.hidden,)),
                gate_up=bf(mlp.gate_up_proj.weight, (2 * c.intermediate, c.hidden)),
                down=bf(mlp.down_proj.weight, (c.hidden, c.intermediate)),
                attention=SimpleNamespace(
                    q_norm=SimpleNamespace(weight=bf(a.q_norm.weight, (c.head_dim,)),
                                           variance_epsilon=float(a.q_norm.variance_epsilon)),
                    k_norm=SimpleNamespace(weight=bf(a.k_norm.weight, (c.head_dim,)),
                                           variance_epsilon=float(a.k_norm.variance_epsilon)),
                    rope_theta=float(a.rope_theta),
                ),
            ))
        self.final_norm = bf(inner.norm.weight, (c.hidden,))
        self.codec_head = bf(model.codec_head.weight, (c.vocab, c.hidden))
        self.text_embedding = bf(model.get_projected_text_embedding_cache(), (c.text_vocab, c.hidden))
        self.codec_embedding = bf(inner.codec_embedding.weight, (c.vocab, c.hidden))
        self._derive(fp8_gate_up)
        return self

    def weight_bytes(self) -> int:
        """Bytes of weights one decode step reads (FP8 codes + scales for gate/up when enabled)."""

        total = 2 * (self.final_norm.numel() + self.codec_head.numel())
        for layer in self.layers:
            total += 2 * sum(t.numel() for t in (layer.input_norm, layer.qkv, layer.o, layer.post_norm, layer.down))
            total += 2 * (layer.attention.q_norm.weight.numel() + layer.attention.k_norm.weight.numel())
            if self.fp8_gate_up:
                total += layer.gate_up_q.numel() + 4 * layer.gate_up_scales.numel()
            else:
                total += 2 * layer.gate_up.numel()
        return total


def check_step_report(head) -> None:
    """Fail closed on a decode step's report (the status words of ``nq_step_report``): map each
    non-zero word to the reference's exception type (KVAllocationError for the planner running out
    of pages, ValueError for inputs outside their tables, RuntimeError otherwise)."""

    plan, merge, attention, embed, bad_tokens = (int(x) for x in head[:5])
    if plan == _lib.NQ_ERR_CAPACITY:
        raise KVAllocationError("the GPU planner ran out of free Talker KV pages")
    if plan == _lib.NQ_ERR_STATE:
        raise RuntimeError("the GPU planner took other pages than the host ledger reserved (the device free "
                           "list diverged from the ledger)")
    if plan != _lib.NQ_OK:
        raise RuntimeError(f"GPU planner status {plan} ({_lib.status_string(plan)})")
    if merge != _lib.NQ_OK:
        raise RuntimeError("a returned KV page was already on the device free list")
    if attention != _lib.NQ_OK:
        raise ValueError("paged attention met a page id outside the KV pool or an invalid K/V write slot")
    if embed != _lib.NQ_OK:
        raise ValueError("a text token id lies outside the embedding table")
    if bad_tokens:
        raise RuntimeError(f"{bad_tokens} sampled token ids lie outside the vocabulary")


class StepReport:
    """The device report of a decode step and pinned host copies of it: ``fetch`` queues one
    device-to-host copy on the current stream and returns its ticket, ``read`` waits for it, fails
    closed on the status words and returns the per-row end-of-speech flags.

    The host copies form a ring of ``depth`` buffers; a ticket is the copy's serial number, and a
    ticket whose buffer has since been reused by a later fetch is refused (RuntimeError) instead of
    returning another step's words."""

    def __init__(self, rows: int, device, depth: int = 4) -> None:
        head = _lib.NQ_REPORT_HEAD
        self.rows = rows
        self.device = torch.zeros(head + rows, dtype=torch.int32, device=device)
        self._host = [torch.zeros(head + rows, dtype=torch.int32, pin_memory=True) for _ in range(depth)]
        self._events: list[torch.cuda.Event | None] = [None] * depth
        self._holder = [-1] * depth  # serial of the copy each buffer holds
        self._serial = 0

    def fetch(self) -> int:
        ticket = self._serial
        self._serial += 1
        i = ticket % len(self._host)
        if self._events[i] is not None:
            self._events[i].synchronize()
        self._host[i].copy_(self.device, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self._events[i] = ev
        self._holder[i] = ticket
        return ticket

    def _slot(self, ticket: int) -> int:
        i = ticket % len(self._host)
        if ticket < 0 or self._holder[i] != ticket:
            raise RuntimeError(f"step report {ticket} was overwritten by a later step (only the last "
                               f"{len(self._host)} reports are kept)")
        return i

    def read(self, ticket: int):
        i = self._slot(ticket)
        self._events[i].synchronize()
        words = self._host[i].numpy()
        check_step_report(words[: _lib.NQ_REPORT_HEAD])
        return words[_lib.NQ_REPORT_HEAD:].astype(bool)

    def fence(self, ticket: int) -> "ReportFence":
        return ReportFence(self._events[self._slot(ticket)])


class ReportFence:
    """Completion fence of one report copy: ``ready()`` without blocking, ``wait()`` blocking -- the
    interface the reference's SubmissionWindow polls before a host finalize
    (executor/submission.py:126-228)."""

    __slots__ = ("_event",)

    def __init__(self, event) -> None:
        self._event = event

    def ready(self) -> bool:
        return bool(self._event.query())

    def wait(self) -> None:
        self._event.synchronize()


class TalkerDecodeStep:
    """Static buffers and the forward of one decode bucket (``rows`` physical rows)."""

    def __init__(self, weights: TalkerWeights, context, rows: int, *, use_counter_rng: bool = False,
                 workspace: torch.Tensor | None = None) -> None:
        c = weights.config
        self.w = weights
        self.context = context
        self.rows = rows
        dev = weights.codec_head.device
        self.device = dev
        bf = dict(dtype=torch.bfloat16, device=dev)
        self.step_embed = torch.zeros(rows, c.hidden, **bf)
        self.text_ids = torch.zeros(rows, dtype=torch.long, device=dev)
        self.temperature = torch.zeros(rows, dtype=torch.float32, device=dev)
        self.top_k = torch.ones(rows, dtype=torch.int32, device=dev)
        self.top_p = torch.ones(rows, dtype=torch.float32, device=dev)
        self.penalty = torch.ones(rows, dtype=torch.float32, device=dev)
        self.seen = torch.zeros(rows, c.vocab, dtype=torch.bool, device=dev)
        self.suppress_eos = torch.zeros(rows, dtype=torch.bool, device=dev)
        self.uniforms = torch.zeros(rows, dtype=torch.float32, device=dev)
        self.seed = torch.zeros(rows, dtype=torch.long, device=dev)
        self.offsets = torch.zeros(rows, dtype=torch.long, device=dev)
        self.use_counter_rng = use_counter_rng
        # work buffers
        self.residual = torch.zeros(rows, c.hidden, **bf)
        self.hidden = torch.zeros(rows, c.hidden, **bf)
        self.qkv = torch.zeros(rows, c.qkv_width, **bf)
        self.act = torch.zeros(rows, c.intermediate, **bf)
        self.logits = torch.zeros(rows, c.vocab, **bf)
        self.tokens = torch.zeros(rows, dtype=torch.long, device=dev)
        q_w = c.num_qo_heads * c.head_dim
        projections = (
            (c.qkv_width, c.hidden, _lib.NQ_EPI_PARTIALS),
            (c.hidden, q_w, _lib.NQ_EPI_ADD_RMSNORM),
            (2 * c.intermediate, c.hidden, _lib.NQ_EPI_SILU_MUL),
            (c.hidden, c.intermediate, _lib.NQ_EPI_ADD_RMSNORM),
            (c.vocab, c.hidden, _lib.NQ_EPI_PARTIALS),  # the codec head's planes feed the sampler
        )
        declined = [(n, k) for n, k, _ in projections if _lib.load().nq_linear_splits(rows, n, k) <= 0]
        if declined:
            raise ValueError(f"the decode projections take buckets of at most 128 rows; {rows} rows x "
                             f"{declined[0]} is a prefill-sized shape (TalkerPrefillStep runs those)")
        self.fp8 = weights.fp8_gate_up
        need = max(16, max(linear_workspace_bytes(rows, n, k, e) for n, k, e in projections))
        if self.fp8:
            # activation codes / scales of the gate/up input
            self.act_q = torch.zeros(rows, c.hidden, dtype=FP8, device=dev)
            self.act_scales = torch.zeros(rows, c.hidden // 128, dtype=torch.float32, device=dev)
            need = max(need, linear_fp8_workspace_bytes(rows, 2 * c.intermediate, c.hidden, _lib.NQ_EPI_SILU_MUL))
        # split-K planes of the projections; may be shared by steps whose graphs never run at once
        if workspace is not None and workspace.numel() >= need:
            self.linear_workspace = workspace
        else:
            self.linear_workspace = torch.empty(need, dtype=torch.uint8, device=dev)
        # optional [layers + 1, rows, hidden] bf16 record of the residual stream: the step input, then
        # the residual after each layer (device-to-device copies, for layer-by-layer checks)
        self.trace: torch.Tensor | None = None
        # fail-closed report: planner / free-list / attention / embedding status and per-row EOS flags
        self.embed_status = torch.zeros(1, dtype=torch.int32, device=dev)
        self.report = StepReport(rows, dev)

    def forward(self) -> torch.Tensor:
        c = self.w.config
        ctx = self.context
        n = self.rows
        # materialize_decode (executor/talker.py:256-262) and the first input norm, one launch
        embed_add_rmsnorm(self.text_ids, self.w.text_embedding, self.step_embed, self.w.layers[0].input_norm,
                          c.rms_eps, self.residual, self.hidden, status=self.embed_status)
        trace = self.trace
        if trace is not None:
            trace[0].copy_(self.residual)
        q_w = c.num_qo_heads * c.head_dim
        ws = self.linear_workspace
        for index, layer in enumerate(self.w.layers):
            ctx.select_layer(index)
            nxt = self.w.final_norm if index + 1 == len(self.w.layers) else self.w.layers[index + 1].input_norm
            # the split-K planes of the QKV projection feed the q/k norm + RoPE + KV write directly
            splits = linear_partials(self.hidden, layer.qkv, ws)
            q = self.qkv[:, :q_w].view(n, c.num_qo_heads, c.head_dim)
            attended = ctx.attend_partials(layer.attention, ws, splits, q).view(n, q_w)
            if self.fp8:
                # post-attention add-RMSNorm quantized per 128 columns, block-scaled FP8 gate/up + SwiGLU
                linear_add_rmsnorm_fp8(attended, layer.o, self.residual, layer.post_norm, c.rms_eps,
                                       self.act_q, self.act_scales, ws)
                linear_fp8_swiglu(self.act_q, self.act_scales, layer.gate_up_packed, layer.gate_up_scales,
                                  self.act, weight_q=layer.gate_up_q, workspace=ws)
            else:
                linear_add_rmsnorm(attended, layer.o, self.residual, layer.post_norm, c.rms_eps, self.hidden, ws)
                linear_silu_mul(self.hidden, layer.gate_up, out=self.act, workspace=ws)
            linear_add_rmsnorm(self.act, layer.down, self.residual, nxt, c.rms_eps, self.hidden, ws)
            if trace is not None:
                trace[index + 1].copy_(self.residual)
        ctx.advance_sequence_lengths()
        self._sample()
        self._report()
        return self.tokens

    def _report(self) -> None:
        ctx, c = self.context, self.w.config
        buffers = getattr(ctx, "buffers", None)
        _lib.call("nq_step_report", _lib.ptr(None if buffers is None else buffers.status),
                  _lib.ptr(getattr(ctx, "free_list_status", None)), _lib.ptr(getattr(ctx, "attention_status", None)),
                  self.embed_status.data_ptr(), self.tokens.data_ptr(), self.rows, c.eos_id, c.vocab,
                  self.report.device.data_ptr(), _lib.stream(self.device))

    def _sample(self) -> None:
        c = self.w.config
        n = self.rows
        ws = self.linear_workspace
        options = dict(repetition_penalty=self.penalty, seen_token_mask=self.seen, mask_from=c.codec_vocab,
                       eos_id=c.eos_id, suppress_eos=self.suppress_eos, update_seen=True, out=self.tokens)
        if self.use_counter_rng:
            # codec head as split-K planes, summed, rounded and drawn from in the sampling launch
            # (the same logits and tokens as the projection followed by the sampler)
            splits = linear_partials(self.hidden, self.w.codec_head, ws)
            planes = ws[: splits * n * c.vocab * 4].view(torch.float32).view(splits, n, c.vocab)
            sample_with_counter_from_planes(planes, self.temperature, self.top_k, self.top_p, self.seed, self.offsets,
                                            logits_out=self.logits, **options)
            return
        # caller-supplied uniforms
        linear(self.hidden, self.w.codec_head, out=self.logits, workspace=ws)
        sample_with_uniforms(self.logits, self.temperature, self.top_k, self.top_p, self.uniforms, **options)


class TalkerPrefillStep:
    """Static buffers and the forward of one prefill bucket: ``tokens`` packed prompt tokens of at
    most ``rows`` requests (TalkerPrefillCaptureKey: token_capacity, capture_batch_size).

    Follows the reference's captured prefill operation (executor/talker.py:397-459 with
    materialize_prefill :246-254 and forward_logits :231-244): input embedding = text embedding
    plus, where the codec mask is set, the codec embedding; the layer stack over every packed token
    (causal prefill attention over the paged KV, writing each token's K/V); the final-norm hidden
    state of each request's last token (``last`` indices); the codec head, the logit masks and the
    sampler on those rows.  From TILED_FROM tokens the projections are the tiled MFMA GEMMs over
    every token (``tgemm``: QKV as split-K planes feeding the q/k norm + RoPE + K/V write, o_proj
    and down through the add-RMSNorm that reduces their planes; FP8 gate/up + SwiGLU as
    ``tgemm_fp8_swiglu``); smaller buckets run the decode step's skinny GEMM with its fused
    epilogues in pieces of at most CHUNK rows."""

    CHUNK = 128
    TILED_FROM = 128

    def __init__(self, weights: TalkerWeights, context, rows: int, tokens: int, *,
                 workspace: torch.Tensor | None = None) -> None:
        if rows < 1 or tokens < rows:
            raise ValueError("a prefill bucket needs at least one row and one token per row")
        c = weights.config
        self.w = weights
        self.context = context
        self.rows = rows
        self.tokens_capacity = tokens
        dev = weights.codec_head.device
        self.device = dev
        bf = dict(dtype=torch.bfloat16, device=dev)
        # static inputs (the reference's _PrefillSlot text / codec / mask / last / suppress / sampling)
        self.text_ids = torch.zeros(tokens, dtype=torch.long, device=dev)
        self.codec_ids = torch.zeros(tokens, dtype=torch.long, device=dev)
        self.codec_mask = torch.zeros(tokens, dtype=torch.bool, device=dev)
        self.last = torch.zeros(rows, dtype=torch.long, device=dev)
        self.derive_last = True  # False: ``last`` is staged by the caller
        self.suppress_eos = torch.ones(rows, dtype=torch.bool, device=dev)
        self.temperature = torch.zeros(rows, dtype=torch.float32, device=dev)
        self.top_k = torch.ones(rows, dtype=torch.int32, device=dev)
        self.top_p = torch.ones(rows, dtype=torch.float32, device=dev)
        self.penalty = torch.ones(rows, dtype=torch.float32, device=dev)
        self.seed = torch.zeros(rows, dtype=torch.long, device=dev)
        self.offsets = torch.zeros(rows, dtype=torch.long, device=dev)
        self.seen = torch.zeros(rows, c.vocab, dtype=torch.bool, device=dev)
        # work buffers
        q_w = c.num_qo_heads * c.head_dim
        self.residual = torch.zeros(tokens, c.hidden, **bf)
        self.hidden = torch.zeros(tokens, c.hidden, **bf)
        self.qkv = torch.zeros(tokens, c.qkv_width, **bf)
        self.act = torch.zeros(tokens, c.intermediate, **bf)
        self.last_hidden = torch.zeros(rows, c.hidden, **bf)
        self.logits = torch.zeros(rows, c.vocab, **bf)
        self.tokens = torch.zeros(rows, dtype=torch.long, device=dev)
        self.fp8 = weights.fp8_gate_up
        # the tiled prefill GEMMs from TILED_FROM tokens; below, the decode GEMM in one piece
        self.tiled = tokens >= self.TILED_FROM
        piece = min(tokens, self.CHUNK)
        projections = (
            (c.qkv_width, c.hidden, _lib.NQ_EPI_NONE),
            (c.hidden, q_w, _lib.NQ_EPI_ADD_RMSNORM),
            (2 * c.intermediate, c.hidden, _lib.NQ_EPI_SILU_MUL),
            (c.hidden, c.intermediate, _lib.NQ_EPI_ADD_RMSNORM),
        )
        need = max(16, max(linear_workspace_bytes(piece, n, k, e) for n, k, e in projections),
                   linear_workspace_bytes(rows, c.vocab, c.hidden, _lib.NQ_EPI_NONE))
        if self.tiled:
            need = max(need, tgemm_workspace_bytes(tokens, c.qkv_width, c.hidden, _lib.NQ_EPI_PARTIALS),
                       tgemm_workspace_bytes(tokens, c.hidden, q_w, _lib.NQ_EPI_ADD_RMSNORM),
                       tgemm_workspace_bytes(tokens, c.hidden, c.intermediate, _lib.NQ_EPI_ADD_RMSNORM))
        if self.fp8:
            self.act_q = torch.zeros(tokens, c.hidden, dtype=FP8, device=dev)
            self.act_scales = torch.zeros(tokens, c.hidden // 128, dtype=torch.float32, device=dev)
            need = max(need, linear_fp8_workspace_bytes(piece, 2 * c.intermediate, c.hidden, _lib.NQ_EPI_SILU_MUL))
        if workspace is not None and workspace.numel() >= need:
            self.linear_workspace = workspace
        else:
            self.linear_workspace = torch.empty(need, dtype=torch.uint8, device=dev)
        self.embed_status = torch.zeros(1, dtype=torch.int32, device=dev)
        self.report = StepReport(rows, dev)
        # optional [layers + 1, tokens, hidden] record of the residual stream (as the decode step's)
        self.trace: torch.Tensor | None = None
        # the last-token gather is gather_sum_rows with no summed groups
        self._no_ids = torch.zeros((0, rows), dtype=torch.long, device=dev)
        self._no_tables = torch.zeros((0, 1, c.hidden), **bf)

    def _pieces(self):
        t = self.tokens_capacity
        return [(r0, min(t, r0 + self.CHUNK)) for r0 in range(0, t, self.CHUNK)]

    def forward(self) -> torch.Tensor:
        c = self.w.config
        ctx = self.context
        t = self.tokens_capacity
        ws = self.linear_workspace
        q_w = c.num_qo_heads * c.head_dim
        kv_w = c.num_kv_heads * c.head_dim
        pieces = self._pieces()
        # materialize_prefill and the first input norm, one launch
        prefill_embed_rmsnorm(self.text_ids, self.w.text_embedding, self.codec_ids, self.w.codec_embedding,
                              self.codec_mask, self.w.layers[0].input_norm, c.rms_eps, self.residual, self.hidden,
                              status=self.embed_status)
        trace = self.trace
        if trace is not None:
            trace[0].copy_(self.residual)
        for index, layer in enumerate(self.w.layers):
            ctx.select_layer(index)
            nxt = self.w.final_norm if index + 1 == len(self.w.layers) else self.w.layers[index + 1].input_norm
            if self.tiled:
                # the tiled GEMMs over every token: QKV as split-K planes feeding the q/k norm + RoPE +
                # K/V write, o_proj and down with the add-RMSNorm reducing their planes
                splits = tgemm_partials(self.hidden, layer.qkv, ws)
                q = self.qkv[:, :q_w].view(t, c.num_qo_heads, c.head_dim)
                attended = ctx.attend_partials(layer.attention, ws, splits, q).view(t, q_w)
                if self.fp8:
                    tgemm_add_rmsnorm_fp8(attended, layer.o, self.residual, layer.post_norm, c.rms_eps, self.act_q,
                                          self.act_scales, ws)
                    tgemm_fp8_swiglu(self.act_q, self.act_scales, layer.gate_up_packed, layer.gate_up_scales, self.act)
                else:
                    tgemm(attended, layer.o, self.hidden, _lib.NQ_EPI_ADD_RMSNORM, self.residual, layer.post_norm,
                          c.rms_eps, ws)
                    tgemm(self.hidden, layer.gate_up, self.act, _lib.NQ_EPI_SILU_MUL)
                tgemm(self.act, layer.down, self.hidden, _lib.NQ_EPI_ADD_RMSNORM, self.residual, nxt, c.rms_eps, ws)
                if trace is not None:
                    trace[index + 1].copy_(self.residual)
                continue
            for a, b in pieces:
                linear(self.hidden[a:b], layer.qkv, out=self.qkv[a:b], workspace=ws)
            q = self.qkv[:, :q_w].view(t, c.num_qo_heads, c.head_dim)
            k = self.qkv[:, q_w : q_w + kv_w].view(t, c.num_kv_heads, c.head_dim)
            v = self.qkv[:, q_w + kv_w :].view(t, c.num_kv_heads, c.head_dim)
            attended = ctx.attend(layer.attention, q, k, v).view(t, q_w)
            for a, b in pieces:
                if self.fp8:
                    linear_add_rmsnorm_fp8(attended[a:b], layer.o, self.residual[a:b], layer.post_norm, c.rms_eps,
                                           self.act_q[a:b], self.act_scales[a:b], ws)
                    linear_fp8_swiglu(self.act_q[a:b], self.act_scales[a:b], layer.gate_up_packed,
                                      layer.gate_up_scales, self.act[a:b], weight_q=layer.gate_up_q, workspace=ws)
                else:
                    linear_add_rmsnorm(attended[a:b], layer.o, self.residual[a:b], layer.post_norm, c.rms_eps,
                                       self.hidden[a:b], ws)
                    linear_silu_mul(self.hidden[a:b], layer.gate_up, out=self.act[a:b], workspace=ws)
                linear_add_rmsnorm(self.act[a:b], layer.down, self.residual[a:b], nxt, c.rms_eps, self.hidden[a:b],
                                   ws)
            if trace is not None:
                trace[index + 1].copy_(self.residual)
        ctx.advance_sequence_lengths()
        # forward_logits: the final-norm hidden state of each request's last token.  With the planner's
        # qo_indptr on the device, last = qo_indptr[1:] - 1: the reference's host cumsum - 1 for every
        # real row (padding rows, which hold no tokens, repeat the previous row's index), without a copy
        qo = getattr(getattr(ctx, "buffers", None), "qo_indptr", None)
        if qo is not None and self.derive_last:
            torch.sub(qo[1 : self.rows + 1], 1, out=self.last)
        gather_sum_rows(self.last, self.hidden, self._no_ids, self._no_tables, self.last_hidden,
                        status=self.embed_status)
        linear(self.last_hidden, self.w.codec_head, out=self.logits, workspace=ws)
        sample_with_counter(self.logits, self.temperature, self.top_k, self.top_p, self.seed, self.offsets,
                            repetition_penalty=self.penalty, seen_token_mask=self.seen, mask_from=c.codec_vocab,
                            eos_id=c.eos_id, suppress_eos=self.suppress_eos, update_seen=True, out=self.tokens)
        TalkerDecodeStep._report(self)
        return self.tokens


__all__ = ["ReportFence", "StepReport", "TalkerConfig", "TalkerDecodeStep", "TalkerPrefillStep", "TalkerWeights",
           "check_step_report"]
