"""Code-predictor frame loop on the GPU: one hipGraph-capturable pass that turns
each row's layer-0 codec token and talker hidden state into the 16-code frame.

Mirrors ``CodePredictorExecutor.whole_frame`` (executor/code_predictor.py:
159-235) and ``Qwen3TTSCodePredictor.forward_depth_unrolled`` on its fused
branch (model/components.py:254-356):

- pass 0 runs the small->MTP projection of ``past_hidden`` through the layers
  at cache position 0 (only the K/V it writes matter);
- codec_sum starts as the layer-0 embedding of the layer-0 token, the first
  input is the projected layer-0 embedding of that token;
- for group g = 1..15: the layers at cache position g with the final norm,
  logits = hidden @ lm_head[g-1]^T, one sampled token per row, codec_sum +=
  codec_embedding[g-1][token], next input = projected codec embedding.

Each layer is: RMSNorm (first layer; later ones come out of the previous
epilogue), packed QKV projection, then one launch for the q/k RMSNorm + RoPE
with the K/V write into the dense 16-slot cache (no bf16 rounding before the
rotation, model/kernels.py:335-405) and the short-cache attention over the
valid positions, o_proj with the residual add + post-attention RMSNorm fused,
gate_up with the SwiGLU fused (one kernel over interleaved gate/up rows), down
with the residual add + next RMSNorm fused.  The residual
adds are the reference's plain bf16 ``residual + projection`` followed by the
norm (components.py:331-346), which is what the fused epilogue computes.

Sampling takes uniforms ([15, rows], one per row and group); with
``use_counter_rng`` they are derived on the device from (seed, offsets[:, g-1])
by Philox-4x32-10 like the reference's counter-addressed draws.  Rows with
temperature 0 take the argmax (the reference maps them to top-1,
executor/code_predictor.py:149-162, which selects the same token).
"""

from __future__ import annotations

from dataclasses import dataclass
from types import SimpleNamespace

import torch
import torch.nn.functional as F

from . import _lib
from .kernels import qkv_partials_rope_short_attention_
from .layers import (
    embed_add_rmsnorm,
    gather_sum_rows,
    linear,
    linear_add_rmsnorm,
    linear_partials,
    linear_swiglu,
    linear_workspace_bytes,
    pack_swiglu,
    rmsnorm,
)
from .sampling import sample_with_counter_from_planes, sample_with_uniforms


@dataclass(frozen=True)
class CodePredictorConfig:
    num_layers: int = 5
    hidden: int = 1024
    num_qo_heads: int = 16
    num_kv_heads: int = 8
    head_dim: int = 64
    intermediate: int = 3072
    vocab: int = 2048
    talker_hidden: int = 2048
    talker_vocab: int = 3072
    num_code_groups: int = 16
    rms_eps: float = 1e-6
    rope_theta: float = 1_000_000.0

    @property
    def qkv_width(self) -> int:
        return (self.num_qo_heads + 2 * self.num_kv_heads) * self.head_dim


class CodePredictorWeights:
    """Random-init code-predictor parameters (bf16) plus the tables the executor derives once:
    ``projected_layer0`` = projection(layer-0 embedding) and ``projected_residual[g]`` =
    projection(codec_embedding[g]) for g < 14 (executor/code_predictor.py:72-88)."""

    def __init__(self, config: CodePredictorConfig, device: torch.device, seed: int = 0, std: float = 0.02) -> None:
        self.config = c = config
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        bf = dict(dtype=torch.bfloat16, device=device)

        def randn(*shape, scale=std):
            return (torch.randn(*shape, generator=g, device=device) * scale).to(torch.bfloat16)

        self.layers = [
            SimpleNamespace(
                input_norm=torch.ones(c.hidden, **bf),
                qkv=randn(c.qkv_width, c.hidden),
                o=randn(c.hidden, c.num_qo_heads * c.head_dim),
                post_norm=torch.ones(c.hidden, **bf),
                gate_up=randn(2 * c.intermediate, c.hidden),
                down=randn(c.hidden, c.intermediate),
                q_norm=torch.ones(c.head_dim, **bf),
                k_norm=torch.ones(c.head_dim, **bf),
            )
            for _ in range(c.num_layers)
        ]
        self.final_norm = torch.ones(c.hidden, **bf)
        groups = c.num_code_groups - 1
        self.lm_head = randn(groups, c.vocab, c.hidden)
        self.proj_w = randn(c.hidden, c.talker_hidden)
        self.proj_b = randn(c.hidden)
        self.layer0_embedding = randn(c.talker_vocab, c.talker_hidden, scale=1.0)
        self.codec_embedding = randn(groups, c.vocab, c.talker_hidden, scale=1.0)
        self._derive()

    def _derive(self) -> None:
        for L in self.layers:  # gate/up rows interleaved for the fused SwiGLU kernel
            L.gate_up_packed = pack_swiglu(L.gate_up)
        groups = self.config.num_code_groups - 1
        # derived once, as the executor does (executor/code_predictor.py:72-88: torch GEMM with bias,
        # not on the per-frame path)
        self.projected_layer0 = F.linear(self.layer0_embedding, self.proj_w, self.proj_b).contiguous()
        self.projected_residual = torch.stack(
            [F.linear(self.codec_embedding[i], self.proj_w, self.proj_b) for i in range(groups - 1)]
        ).contiguous()

    @classmethod
    def from_reference_model(cls, model, layer0_embedding, config) -> "CodePredictorWeights":
        """The parameters of a loaded reference code predictor: ``model`` a ``Qwen3TTSCodePredictor``
        (model/components.py:132-200), ``layer0_embedding`` the talker's codec embedding the executor
        is given (executor/build.py:74-76) and ``config`` the reference's ``Qwen3TTSConfig``
        (model/config.py:66-118).  Every tensor is the model's own, as contiguous bf16 on its device:
        per layer the norms, the packed QKV and o projections, the q/k norms and the packed [gate; up]
        and down projections; the final norm, the 15 heads, the small-to-MTP projection with its bias
        and the codec embeddings; the projected embedding tables are derived as the executor derives
        them."""

        t = config.talker
        p = t.code_predictor
        c = CodePredictorConfig(num_layers=int(p.num_hidden_layers), hidden=int(p.hidden_size),
                                num_qo_heads=int(p.num_attention_heads), num_kv_heads=int(p.num_key_value_heads),
                                head_dim=int(p.head_dim), intermediate=int(p.intermediate_size),
                                vocab=int(p.vocab_size), talker_hidden=int(t.hidden_size),
                                talker_vocab=int(t.vocab_size), num_code_groups=int(t.num_code_groups),
                                rms_eps=float(p.rms_norm_eps), rope_theta=float(p.rope_theta))
        inner = model.model
        groups = c.num_code_groups - 1
        if len(inner.layers) != c.num_layers or len(model.lm_head) != groups or len(inner.codec_embedding) != groups:
            raise ValueError("the code predictor's layer, head or embedding count does not match the config")

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
                q_norm=bf(a.q_norm.weight, (c.head_dim,)),
                k_norm=bf(a.k_norm.weight, (c.head_dim,)),
            ))
        self.final_norm = bf(inner.norm.weight, (c.hidden,))
        self.lm_head = torch.stack([bf(h.weight, (c.vocab, c.hidden)) for h in model.lm_head]).contiguous()
        proj = model.small_to_mtp_projection
        self.proj_w = bf(proj.weight, (c.hidden, c.talker_hidden))
        self.proj_b = bf(proj.bias, (c.hidden,))
        self.layer0_embedding = bf(layer0_embedding.weight, (c.talker_vocab, c.talker_hidden))
        self.codec_embedding = torch.stack(
            [bf(e.weight, (c.vocab, c.talker_hidden)) for e in inner.codec_embedding]).contiguous()
        self._derive()
        return self

    def weight_bytes_per_pass(self) -> int:
        c = self.config
        per_layer = c.qkv_width * c.hidden + c.hidden * c.num_qo_heads * c.head_dim + 3 * c.intermediate * c.hidden
        return 2 * per_layer * c.num_layers


class CodePredictorFrame:
    """Static buffers for ``rows`` physical rows and the whole-frame forward."""

    def __init__(self, weights: CodePredictorWeights, rows: int, *, use_counter_rng: bool = False) -> None:
        c = weights.config
        if not 1 <= rows <= 128:
            raise ValueError("the code-predictor frame runs 1..128 rows")
        self.w = weights
        self.rows = rows
        self.use_counter_rng = use_counter_rng
        dev = weights.lm_head.device
        bf = dict(dtype=torch.bfloat16, device=dev)
        groups = c.num_code_groups
        # inputs
        self.layer0_token = torch.zeros(rows, dtype=torch.long, device=dev)
        self.past_hidden = torch.zeros(rows, c.talker_hidden, **bf)
        self.temperature = torch.zeros(rows, dtype=torch.float32, device=dev)
        self.top_k = torch.ones(rows, dtype=torch.int32, device=dev)
        self.top_p = torch.ones(rows, dtype=torch.float32, device=dev)
        self.seed = torch.zeros(rows, dtype=torch.long, device=dev)
        self.offsets = torch.zeros(rows, groups - 1, dtype=torch.long, device=dev)
        self.uniforms = torch.zeros(groups - 1, rows, dtype=torch.float32, device=dev)
        self.position_ids = torch.arange(groups, dtype=torch.long, device=dev).unsqueeze(0).repeat(rows, 1)
        # outputs
        self.frames = torch.zeros(rows, groups, dtype=torch.long, device=dev)
        self.tokens = torch.zeros(groups - 1, rows, dtype=torch.long, device=dev)
        self.codec_sum = torch.zeros(rows, c.talker_hidden, **bf)
        self.logits = torch.zeros(groups - 1, rows, c.vocab, **bf)
        # state and work buffers
        self.kv_cache = torch.zeros(c.num_layers, rows, 2, groups, c.num_kv_heads, c.head_dim, **bf)
        self.h = torch.zeros(rows, c.hidden, **bf)  # residual stream
        self.x = torch.zeros(rows, c.hidden, **bf)  # normalised stream
        self.att = torch.zeros(rows, c.num_qo_heads, c.head_dim, **bf)
        self.q = torch.zeros(rows, c.num_qo_heads, c.head_dim, **bf)  # rotated queries
        self.act = torch.zeros(rows, c.intermediate, **bf)
        shapes = (
            (c.hidden, c.talker_hidden, _lib.NQ_EPI_NONE),
            (c.qkv_width, c.hidden, _lib.NQ_EPI_PARTIALS),  # planes feed the q/k norm + RoPE
            (c.hidden, c.num_qo_heads * c.head_dim, _lib.NQ_EPI_ADD_RMSNORM),
            (2 * c.intermediate, c.hidden, _lib.NQ_EPI_SILU_MUL),
            (c.hidden, c.intermediate, _lib.NQ_EPI_ADD_RMSNORM),
            (c.vocab, c.hidden, _lib.NQ_EPI_PARTIALS),  # planes feed the sampler
        )
        need = max(linear_workspace_bytes(rows, n, k, e) for n, k, e in shapes)
        self.workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
        # optional [groups, layers + 2, rows, hidden] bf16 record of each pass: the residual stream
        # at the pass start and after every layer, then the normalised hidden state the head reads
        # (device-to-device copies, for layer-by-layer checks)
        self.trace: torch.Tensor | None = None
        # None: the fused draw from the lm_head's split-K planes (counter RNG) or from ``uniforms``;
        # otherwise a sampler with the reference's signature (logits, temperature, top_k, top_p, seed,
        # offset) -> tokens, called on each group's bf16 logits (read when the forward is recorded)
        self.sampler = None

    def _layers(self, cache_pos: int, normed: bool = False) -> None:
        """The 5 layers at cache position ``cache_pos``; ``normed``: self.x already holds the first
        input norm of self.h."""
        c, ws = self.w.config, self.workspace
        n = self.rows
        q_w = c.num_qo_heads * c.head_dim
        positions = self.position_ids[:, cache_pos]
        layers = self.w.layers
        if not normed:
            rmsnorm(self.h, layers[0].input_norm, c.rms_eps, out=self.x)
        trace = None if self.trace is None else self.trace[cache_pos]
        if trace is not None:
            trace[0].copy_(self.h)
        for index, L in enumerate(layers):
            cache = self.kv_cache[index]
            # the QKV projection's split-K planes go straight into the q/k norm + RoPE + K/V write and
            # the short-cache attention, one launch (the same bits as the bf16 projection followed by
            # paired_qk_norm_rope_dense_cache_ and decode_attn_nhd_short_cache)
            splits = linear_partials(self.x, L.qkv, ws)
            qkv_partials_rope_short_attention_(ws, splits, self.q, L.q_norm, L.k_norm, positions, c.rms_eps,
                                               c.rope_theta, cache[:, 0], cache[:, 1], cache_pos, self.att)
            linear_add_rmsnorm(self.att.view(n, q_w), L.o, self.h, L.post_norm, c.rms_eps, self.x, ws)
            linear_swiglu(self.x, L.gate_up_packed, self.act, weight=L.gate_up, workspace=ws)
            nxt = self.w.final_norm if index + 1 == len(layers) else layers[index + 1].input_norm
            linear_add_rmsnorm(self.act, L.down, self.h, nxt, c.rms_eps, self.x, ws)
            if trace is not None:
                trace[index + 1].copy_(self.h)
        if trace is not None:
            trace[len(layers) + 1].copy_(self.x)

    def forward(self) -> tuple[torch.Tensor, torch.Tensor]:
        c, w, ws = self.w.config, self.w, self.workspace
        groups = c.num_code_groups
        # pass 0: the talker hidden state fills cache position 0
        linear(self.past_hidden, w.proj_w, out=self.h, workspace=ws, bias=w.proj_b)
        self._layers(0)
        self.frames[:, 0].copy_(self.layer0_token)
        # the next input (a projected embedding row) and the first input norm in one launch
        first_norm = w.layers[0].input_norm
        embed_add_rmsnorm(self.layer0_token, w.projected_layer0, None, first_norm, c.rms_eps, self.h, self.x)
        for group in range(1, groups):
            self._layers(group, normed=True)
            logits = self.logits[group - 1]
            token = self.tokens[group - 1]
            if self.sampler is not None:
                linear(self.x, w.lm_head[group - 1], out=logits, workspace=ws)
                token.copy_(self.sampler(logits, self.temperature, self.top_k, self.top_p, self.seed,
                                         self.offsets[:, group - 1]))
            elif self.use_counter_rng:
                # the head's split-K planes summed, rounded and drawn from in the sampling launch
                splits = linear_partials(self.x, w.lm_head[group - 1], ws)
                planes = ws[: splits * self.rows * c.vocab * 4].view(torch.float32).view(splits, self.rows, c.vocab)
                sample_with_counter_from_planes(planes, self.temperature, self.top_k, self.top_p, self.seed,
                                                self.offsets[:, group - 1], logits_out=logits, out=token)
            else:
                linear(self.x, w.lm_head[group - 1], out=logits, workspace=ws)
                sample_with_uniforms(logits, self.temperature, self.top_k, self.top_p, self.uniforms[group - 1],
                                     out=token)
            if group < groups - 1:
                embed_add_rmsnorm(token, w.projected_residual[group - 1], None, first_norm, c.rms_eps, self.h,
                                  self.x)
        # codec_sum: the layer-0 embedding plus each group's codec embedding, added in group order
        gather_sum_rows(self.layer0_token, w.layer0_embedding, self.tokens, w.codec_embedding, self.codec_sum)
        self.frames[:, 1:].copy_(self.tokens.t())
        return self.frames, self.codec_sum


__all__ = ["CodePredictorConfig", "CodePredictorFrame", "CodePredictorWeights"]
