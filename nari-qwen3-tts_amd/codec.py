"""Incremental codec-decoder step on the GPU for a batch of streams.

``IncrementalCodecDecoder`` is the ``incremental_decoder`` CodecExecutor injects
(executor/codec.py:69-118): ``decoder(codes [B, Q, F], states, *, position_ids=None,
context_lengths=None) -> wav [B, 1, F * samples_per_frame]`` over the reference's
per-row ``IncrementalCodecState`` objects, whose mapping tensors it reads and
replaces and whose frame position and context length it advances
(model/incremental_codec.py:383-466), with ``samples_per_frame`` and
``retained_context`` attributes.  The state is staged into device slot arrays
for the step and written back as new tensors, so the call can be captured into
a hipGraph the way executor/codec.py:444-467 captures it.  ``decode_ragged`` is
the same step over ragged chunks of streams whose state stays in the decoder's
own slots (no staging).

The upstream decoder (qwen-tts 0.1.1) is not available, so the module tree is
a random-init causal decoder of the same structure, sized by ``CodecConfig``:
16-codebook embedding sum (dim 512), causal pre-conv, an 8-layer transformer
with a 26-frame sliding window (25 retained frames), per-head q/k RMSNorm,
RoPE by frame position and layer scales, two transconv(x2) + ConvNeXt
upsample stages, a causal conv, four decoder blocks (SnakeBeta, causal
transconv x5/x5/x4/x5, three dilated residual units), SnakeBeta and the final
causal conv: 2000 samples per 12 Hz frame, 24 kHz fp32 PCM, clamped.

State lives in device slot arrays (one slot per stream): conv histories,
transconv overlaps, retained K/V, frame position and valid context count.
The stateful operators are HIP kernels (``nq_codec_*``); the transformer and
ConvNeXt projections and the wide convolutions (im2col) run on the library's
fp32 GEMM with its fused epilogues (``nq_sgemm``), and the norms on
``nq_row_norm``.  Its products follow torch's float32 matmul precision by name:
"high" by default, the reference's serving policy
(model/checkpoint.py:46-49: ``torch.set_float32_matmul_precision("high")``),
computed as bf16x3 split products with fp32 sums; "highest" keeps full fp32
products.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from types import SimpleNamespace

import numpy as np
import torch

from . import _lib


@dataclass(frozen=True)
class CodecConfig:
    num_quantizers: int = 16
    codebook_size: int = 2048
    dim: int = 512
    layers: int = 8
    heads: int = 8
    head_dim: int = 64
    mlp: int = 1536
    window: int = 26
    theta: float = 10000.0
    eps: float = 1e-6
    up_strides: tuple[int, ...] = (2, 2)
    convnext_mlp: int = 1024
    dec_channels: tuple[int, ...] = (128, 64, 32, 16, 8)
    dec_strides: tuple[int, ...] = (5, 5, 4, 5)
    dilations: tuple[int, ...] = (1, 3, 9)

    @property
    def samples_per_frame(self) -> int:
        return int(np.prod(self.up_strides) * np.prod(self.dec_strides))

    @property
    def retained_context(self) -> int:
        return self.window - 1

    def as_dict(self) -> dict:
        return dict(num_quantizers=self.num_quantizers, dim=self.dim, layers=self.layers, heads=self.heads,
                    head_dim=self.head_dim, window=self.window, theta=self.theta, eps=self.eps,
                    up_strides=tuple(self.up_strides), dec_channels=tuple(self.dec_channels),
                    dec_strides=tuple(self.dec_strides), dilations=tuple(self.dilations))


class CodecWeights:
    """Random-init fp32 parameters; ``host()`` gives the numpy dict the oracle reads."""

    def __init__(self, config: CodecConfig, device: torch.device, seed: int = 0) -> None:
        self.config = c = config
        g = torch.Generator(device="cpu")
        g.manual_seed(seed)

        def rnd(*shape, fan_in=None, scale=None):
            s = scale if scale is not None else 1.0 / math.sqrt(fan_in)
            return (torch.randn(*shape, generator=g) * s).to(device)

        def ones(n):
            return torch.ones(n, device=device)

        d = c.dim
        self.codebooks = rnd(c.num_quantizers, c.codebook_size, d, scale=0.25)
        self.pre_conv_w, self.pre_conv_b = rnd(d, d, 3, fan_in=3 * d), rnd(d, scale=0.01)
        self.in_w, self.in_b = rnd(d, d, fan_in=d), rnd(d, scale=0.01)
        hd = c.heads * c.head_dim
        self.tf = [
            SimpleNamespace(
                ln1=ones(d), wqkv=rnd(3 * hd, d, fan_in=d), qn=ones(c.head_dim), kn=ones(c.head_dim),
                wo=rnd(d, hd, fan_in=hd), ls1=torch.full((d,), 0.1, device=device), ln2=ones(d),
                w1=rnd(c.mlp, d, fan_in=d), w2=rnd(d, c.mlp, fan_in=c.mlp), ls2=torch.full((d,), 0.1, device=device),
            )
            for _ in range(c.layers)
        ]
        self.out_norm = ones(d)
        self.out_w, self.out_b = rnd(d, d, fan_in=d), rnd(d, scale=0.01)
        self.up = []
        for s in c.up_strides:
            self.up.append(SimpleNamespace(
                tc_w=rnd(d, d, 2 * s, fan_in=2 * d), tc_b=rnd(d, scale=0.01),
                dw_w=rnd(d, 1, 7, fan_in=7), dw_b=rnd(d, scale=0.01), ln_w=ones(d), ln_b=torch.zeros(d, device=device),
                pw1_w=rnd(c.convnext_mlp, d, fan_in=d), pw1_b=rnd(c.convnext_mlp, scale=0.01),
                pw2_w=rnd(d, c.convnext_mlp, fan_in=c.convnext_mlp), pw2_b=rnd(d, scale=0.01),
                gamma=torch.full((d,), 0.1, device=device),
            ))
        ch = c.dec_channels
        self.dec0_w, self.dec0_b = rnd(ch[0], d, 7, fan_in=7 * d), rnd(ch[0], scale=0.01)
        self.blocks = []
        for i, s in enumerate(c.dec_strides):
            cin, cout = ch[i], ch[i + 1]
            self.blocks.append(SimpleNamespace(
                alpha=rnd(cin, scale=0.1), beta=rnd(cin, scale=0.1),
                tc_w=rnd(cin, cout, 2 * s, fan_in=2 * cin), tc_b=rnd(cout, scale=0.01),
                res=[SimpleNamespace(
                    a1=rnd(cout, scale=0.1), b1=rnd(cout, scale=0.1), c1_w=rnd(cout, cout, 7, fan_in=7 * cout),
                    c1_b=rnd(cout, scale=0.01), a2=rnd(cout, scale=0.1), b2=rnd(cout, scale=0.1),
                    c2_w=rnd(cout, cout, 1, fan_in=cout) * 0.5, c2_b=rnd(cout, scale=0.01),
                ) for _ in c.dilations],
            ))
        self.final_alpha, self.final_beta = rnd(ch[-1], scale=0.1), rnd(ch[-1], scale=0.1)
        self.final_w, self.final_b = rnd(1, ch[-1], 7, fan_in=7 * ch[-1]), rnd(1, scale=0.01)

    def host(self) -> dict:
        def h(t):
            return t.detach().float().cpu().numpy()

        def ns(n):
            return {k: ([ns(x) for x in v] if isinstance(v, list) else h(v)) for k, v in vars(n).items()}

        return dict(
            codebooks=h(self.codebooks), pre_conv_w=h(self.pre_conv_w), pre_conv_b=h(self.pre_conv_b),
            in_w=h(self.in_w), in_b=h(self.in_b), out_norm=h(self.out_norm), out_w=h(self.out_w), out_b=h(self.out_b),
            tf=[ns(L) | {"wq": h(L.wqkv[: self.config.heads * self.config.head_dim]),
                         "wk": h(L.wqkv[self.config.heads * self.config.head_dim: 2 * self.config.heads * self.config.head_dim]),
                         "wv": h(L.wqkv[2 * self.config.heads * self.config.head_dim:])} for L in self.tf],
            up=[ns(U) for U in self.up], dec0_w=h(self.dec0_w), dec0_b=h(self.dec0_b),
            blocks=[ns(B) for B in self.blocks], final_alpha=h(self.final_alpha), final_beta=h(self.final_beta),
            final_w=h(self.final_w), final_b=h(self.final_b),
        )


@dataclass
class CodecStreamState:
    """One stream's handle on its state slot (the device arrays hold the values)."""

    slot: int
    frame_position: int = 0
    transformer_context_length: int = 0
    _pool: object = field(default=None, repr=False)


def _history_shapes(c: CodecConfig) -> dict[str, tuple[int, int]]:
    """Causal convolutions with history: name -> (input channels, history length)."""

    shapes = {"pre_conv": (c.dim, 2)}
    for u in range(len(c.up_strides)):
        shapes[f"up{u}.dw"] = (c.dim, 6)
    shapes["dec0"] = (c.dim, 6)
    for i in range(len(c.dec_strides)):
        for j, dil in enumerate(c.dilations):
            shapes[f"dec{i + 1}.res{j}.a"] = (c.dec_channels[i + 1], 6 * dil)
    shapes["final"] = (c.dec_channels[-1], 6)
    return shapes


def _overlap_shapes(c: CodecConfig) -> dict[str, tuple[int, int]]:
    """Causal transposed convolutions: name -> (output channels, stride = overlap length)."""

    shapes = {f"up{u}.tc": (c.dim, s) for u, s in enumerate(c.up_strides)}
    for i, s in enumerate(c.dec_strides):
        shapes[f"dec{i + 1}.tc"] = (c.dec_channels[i + 1], s)
    return shapes


class _StatePool:
    """Per-slot decoder state, channels last: histories [slots, pad, C], overlaps [slots, stride, C],
    retained K/V [layers, slots, retained, heads, head_dim], frame position and valid context."""

    def __init__(self, config: CodecConfig, slots: int, device: torch.device) -> None:
        c = config
        z = dict(dtype=torch.float32, device=device)
        self.slots = slots
        self.hist = {name: torch.zeros(slots, pad, cin, **z) for name, (cin, pad) in _history_shapes(c).items()}
        self.overlap = {name: torch.zeros(slots, s, cout, **z) for name, (cout, s) in _overlap_shapes(c).items()}
        r = c.retained_context
        self.k = torch.zeros(c.layers, slots, r, c.heads, c.head_dim, **z)
        self.v = torch.zeros_like(self.k)
        self.frame_pos = torch.zeros(slots, dtype=torch.long, device=device)
        self.ctx = torch.zeros(slots, dtype=torch.int32, device=device)
        self.free = list(range(slots))

    def reset(self, slot: int) -> None:
        for t in list(self.hist.values()) + list(self.overlap.values()):
            t[slot].zero_()
        self.k[:, slot].zero_()
        self.v[:, slot].zero_()
        self.frame_pos[slot] = 0
        self.ctx[slot] = 0


class IncrementalCodecDecoder:
    """``decoder(codes, states) -> (wav, pcm16)`` over ragged chunks of many streams."""

    MATMUL_PRECISIONS = {"highest": _lib.NQ_MATMUL_HIGHEST, "high": _lib.NQ_MATMUL_HIGH}

    def __init__(self, weights: CodecWeights, max_streams: int = 64, *, matmul_precision: str = "high") -> None:
        if matmul_precision not in self.MATMUL_PRECISIONS:
            raise ValueError(f"matmul_precision must be one of {sorted(self.MATMUL_PRECISIONS)}")
        self.matmul_precision = matmul_precision
        self._precision = self.MATMUL_PRECISIONS[matmul_precision]
        self.w = weights
        self.config = weights.config
        self.device = weights.codebooks.device
        self.samples_per_frame = self.config.samples_per_frame
        self.retained_context = self.config.retained_context
        self.pool = _StatePool(self.config, max_streams, self.device)
        self.status = torch.zeros(1, dtype=torch.int32, device=self.device)
        # pinned host staging for decode_ragged's offsets, slots and codes: a copy from pageable memory
        # makes the host wait for the stream, so every call would wait for the previous step's kernels.
        # A ring of buffers, each reused only after its last copy's event has completed.
        self._stage_ring = [[None, None] for _ in range(4)]
        self._stage_next = 0
        self._cache: dict = {}
        self._staging_pools: dict[int, _StatePool] = {}
        self._shape_cache: dict = {}
        self._pool = self.pool

    def new_state(self) -> CodecStreamState:
        if not self.pool.free:
            raise RuntimeError("no free codec state slot")
        slot = self.pool.free.pop(0)
        self.pool.reset(slot)
        return CodecStreamState(slot=slot, _pool=self.pool)

    def release(self, state: CodecStreamState) -> None:
        self.pool.free.append(state.slot)

    # -- helpers ------------------------------------------------------------
    # Wide convolutions (Cin * K >= 256 or Cin >= 64) run as one fp32 GEMM over a
    # gathered operand; narrow ones run the direct HIP kernel.
    GEMM_MIN_CIN_K = 256

    def _derived(self, key, make):
        got = self._cache.get(key)
        if got is None:
            got = make()
            self._cache[key] = got
        return got

    def _conv(self, x, u, name, w, b, *, dilation=1, groups=1, act=None, residual=None):
        c_in = x.shape[1]
        c_out, _, k = w.shape
        hist = self._pool.hist.get(name) if name else None
        a_ptr = _lib.ptr(act[0]) if act else None
        b_ptr = _lib.ptr(act[1]) if act else None
        if groups == 1 and (c_in * k >= self.GEMM_MIN_CIN_K or c_in >= 64) and c_in % 4 == 0:
            cols = torch.empty(x.shape[0], k * c_in, dtype=torch.float32, device=self.device)
            _lib.call("nq_codec_im2col", x.data_ptr(), x.stride(0), x.shape[0], self._off.data_ptr(), self._B, u,
                      self._slots.data_ptr(), _lib.ptr(hist), c_in, k, dilation, 0, a_ptr, b_ptr, cols.data_ptr(),
                      cols.stride(0), self._stream)
            # weights as [c_out, k * c_in] (column tap * c_in + ci of the gathered rows)
            w_nk = self._derived(("conv", id(w)), lambda: w.permute(0, 2, 1).reshape(c_out, k * c_in).contiguous())
            out = self._sgemm(cols, w_nk, bias=b, res=residual)
            if k > 1:
                _lib.call("nq_codec_history_update", x.data_ptr(), x.stride(0), self._off.data_ptr(), self._B, u,
                          self._slots.data_ptr(), hist.data_ptr(), c_in, (k - 1) * dilation, a_ptr, b_ptr,
                          self._stream)
            return out
        out = torch.empty(x.shape[0], c_out, dtype=torch.float32, device=self.device)
        _lib.call("nq_codec_causal_conv", x.data_ptr(), x.stride(0), x.shape[0], self._off.data_ptr(), self._B, u,
                  self._slots.data_ptr(), _lib.ptr(hist), w.data_ptr(), _lib.ptr(b), c_in, c_out, k,
                  dilation, groups, a_ptr, b_ptr, _lib.ptr(residual), residual.stride(0) if residual is not None else 0,
                  out.data_ptr(), out.stride(0), self._stream)
        return out

    def _res_unit(self, x, u, name, R, dilation):
        """x + conv1x1(snake2(conv(snake1(x)) + b1)) + b2: narrow units (8, 16 or 32 channels) in one
        launch whose intermediate never reaches memory; wider ones as the two convolutions."""

        c = x.shape[1]
        if c not in (8, 16, 32) or c * R.c1_w.shape[2] >= self.GEMM_MIN_CIN_K:
            y = self._conv(x, u, name, R.c1_w, R.c1_b, dilation=dilation, act=(R.a1, R.b1))
            return self._conv(y, u, None, R.c2_w, R.c2_b, act=(R.a2, R.b2), residual=x)
        out = torch.empty_like(x)
        _lib.call("nq_codec_residual_unit", x.data_ptr(), x.stride(0), x.shape[0], self._off.data_ptr(), self._B, u,
                  self._slots.data_ptr(), self._pool.hist[name].data_ptr(), c, R.c1_w.shape[2], dilation,
                  R.c1_w.data_ptr(), _lib.ptr(R.c1_b), R.a1.data_ptr(), R.b1.data_ptr(), R.c2_w.data_ptr(),
                  _lib.ptr(R.c2_b), R.a2.data_ptr(), R.b2.data_ptr(), out.data_ptr(), out.stride(0), self._precision,
                  self._stream)
        return out

    def _transconv(self, x, u_in, s, name, w, b, act=None):
        c_in, c_out = w.shape[0], w.shape[1]
        a_ptr = _lib.ptr(act[0]) if act else None
        b_ptr = _lib.ptr(act[1]) if act else None
        overlap = self._pool.overlap[name]
        if c_in >= 64 and c_in % 4 == 0:
            cols = torch.empty(x.shape[0], 2 * c_in, dtype=torch.float32, device=self.device)
            _lib.call("nq_codec_im2col", x.data_ptr(), x.stride(0), x.shape[0], self._off.data_ptr(), self._B, u_in,
                      self._slots.data_ptr(), None, c_in, 2, 1, 1, a_ptr, b_ptr, cols.data_ptr(), cols.stride(0),
                      self._stream)
            # weights as [s * c_out, 2 * c_in]: output column j * c_out + co, input column tap * c_in + ci
            w_nk = self._derived(("tc", id(w)), lambda: w.view(c_in, c_out, 2, s).permute(3, 1, 2, 0)
                                 .reshape(s * c_out, 2 * c_in).contiguous())
            b_s = self._derived(("tcb", id(b)), lambda: b.repeat(s).contiguous())
            out = self._sgemm(cols, w_nk, bias=b_s).view(x.shape[0] * s, c_out)
            # new overlap: each stream's last fresh frame (activated: the first half of its
            # gathered row) through the kernel's second half
            last = torch.empty(self._B, dtype=torch.int32, device=self.device)
            _lib.call("nq_codec_last_rows", self._off.data_ptr(), self._B, u_in, last.data_ptr(), self._stream)
            new_ov = self._sgemm(cols[:, :c_in], w_nk[:, c_in:], x_rows=last)
            _lib.call("nq_codec_transconv_overlap", self._off.data_ptr(), self._B, u_in, s, self._slots.data_ptr(),
                      overlap.data_ptr(), new_ov.data_ptr(), c_out, out.data_ptr(), out.stride(0), self._stream)
            return out
        out = torch.empty(x.shape[0] * s, c_out, dtype=torch.float32, device=self.device)
        _lib.call("nq_codec_causal_transconv", x.data_ptr(), x.stride(0), x.shape[0], self._off.data_ptr(), self._B,
                  u_in, s, self._slots.data_ptr(), overlap.data_ptr(), w.data_ptr(), _lib.ptr(b),
                  c_in, c_out, a_ptr, b_ptr, out.data_ptr(), out.stride(0), self._stream)
        return out

    def _sgemm(self, x, w, *, bias=None, act=0, res=None, scale=None, x_rows=None, out=None):
        """out = res + scale * act(x[x_rows] @ w.T + bias) on the fp32 MFMA GEMM at the decoder's matmul
        precision (fp32 row-major x and w [N, K] with unit inner strides; the optional pieces are left
        out when None)."""

        rows = x.shape[0] if x_rows is None else x_rows.shape[0]
        n, k = w.shape
        if out is None:
            out = torch.empty(rows, n, dtype=torch.float32, device=self.device)
        _lib.call("nq_sgemm", x.data_ptr(), x.stride(0), _lib.ptr(x_rows), w.data_ptr(), w.stride(0), rows, n, k,
                  _lib.ptr(bias), int(act), _lib.ptr(res), res.stride(0) if res is not None else 0, _lib.ptr(scale),
                  out.data_ptr(), out.stride(0), self._precision, self._stream)
        return out

    def _norm(self, x, w, eps, b=None):
        """RMSNorm (b None) or LayerNorm of fp32 rows, one launch."""

        out = torch.empty_like(x)
        _lib.call("nq_row_norm", x.data_ptr(), x.stride(0), x.shape[0], x.shape[1], w.data_ptr(), _lib.ptr(b),
                  float(eps), out.data_ptr(), out.stride(0), self._stream)
        return out

    # -- the reference's call: state objects in, waveform out ---------------------------------
    def reference_keys(self) -> tuple[dict[str, str], dict[str, str]]:
        """Our state names -> the reference's state-mapping keys (model/incremental_codec.py:383-466):
        conv histories and transconv overlaps named after the upstream module path."""

        c = self.config
        hist = {"pre_conv": "pre_conv", "dec0": "decoder.0", "final": f"decoder.{len(c.dec_strides) + 2}"}
        over = {}
        for u in range(len(c.up_strides)):
            hist[f"up{u}.dw"] = f"upsample.{u}.convnext.dwconv"
            over[f"up{u}.tc"] = f"upsample.{u}.transconv"
        for i in range(len(c.dec_strides)):
            over[f"dec{i + 1}.tc"] = f"decoder.{i + 1}.transconv"
            for j in range(len(c.dilations)):
                hist[f"dec{i + 1}.res{j}.a"] = f"decoder.{i + 1}.residual.{j}.conv1"
        return hist, over

    def _staging(self, rows: int) -> "_StatePool":
        pool = self._staging_pools.get(rows)
        if pool is None:
            pool = _StatePool(self.config, rows, self.device)
            self._staging_pools[rows] = pool
        return pool

    def _shape_tensors(self, rows: int, frames: int):
        """Device offsets / slot ids of an equal-chunk batch (made once per shape, so a captured call
        issues no host-to-device copy)."""

        key = (rows, frames)
        got = self._shape_cache.get(key)
        if got is None:
            off = torch.arange(rows + 1, dtype=torch.int32, device=self.device) * frames
            slots = torch.arange(rows, dtype=torch.int32, device=self.device)
            got = (off, np.arange(rows + 1, dtype=np.int64) * frames, slots)
            self._shape_cache[key] = got
        return got

    def _stage_in(self, states, pool: "_StatePool", rows: int, frames: int, position_ids, context_lengths) -> None:
        c = self.config
        dev = self.device
        hist_keys, over_keys = self.reference_keys()

        def gather(mapping: str, key, shape, dst_rows):
            values = [getattr(st, mapping).get(key) for st in states]
            for v in values:
                if v is not None and tuple(v.shape) != shape:
                    raise ValueError(f"invalid incremental state {key!r}: expected {shape}, got {tuple(v.shape)}")
            if all(v is None for v in values):
                dst_rows.zero_()
                return
            zero = None
            rows_in = []
            for v in values:
                if v is None:
                    zero = torch.zeros(shape, dtype=torch.float32, device=dev) if zero is None else zero
                    v = zero
                rows_in.append(v.to(device=dev, dtype=torch.float32))
            dst_rows.copy_(torch.stack(rows_in).transpose(1, 2))

        for name, (cin, pad) in _history_shapes(c).items():
            gather("conv_histories", hist_keys[name], (cin, pad), pool.hist[name][:rows])
        for name, (cout, stride) in _overlap_shapes(c).items():
            gather("transconv_overlaps", over_keys[name], (cout, stride), pool.overlap[name][:rows])
        r = c.retained_context
        for li in range(c.layers):
            gather("transformer_keys", li, (c.heads, r, c.head_dim), pool.k[li, :rows])
            gather("transformer_values", li, (c.heads, r, c.head_dim), pool.v[li, :rows])
        if position_ids is None:
            pool.frame_pos[:rows].copy_(torch.tensor([st.frame_position for st in states], dtype=torch.long))
        else:
            if tuple(position_ids.shape) != (rows, frames):
                raise ValueError(f"incremental position_ids must have shape {(rows, frames)}, got "
                                 f"{tuple(position_ids.shape)}")
            pool.frame_pos[:rows].copy_(position_ids[:, 0])
        if context_lengths is None:
            pool.ctx[:rows].copy_(torch.tensor([st.transformer_context_length for st in states], dtype=torch.int32))
        else:
            if tuple(context_lengths.shape) != (rows,):
                raise ValueError(f"incremental context_lengths must have shape {(rows,)}, got "
                                 f"{tuple(context_lengths.shape)}")
            pool.ctx[:rows].copy_(context_lengths)

    def _stage_out(self, states, pool: "_StatePool", rows: int, frames: int) -> None:
        c = self.config
        hist_keys, over_keys = self.reference_keys()
        for name in _history_shapes(c):
            new = pool.hist[name][:rows].transpose(1, 2).contiguous()
            for st, row in zip(states, new.unbind(0)):
                st.conv_histories[hist_keys[name]] = row
        for name in _overlap_shapes(c):
            new = pool.overlap[name][:rows].transpose(1, 2).contiguous()
            for st, row in zip(states, new.unbind(0)):
                st.transconv_overlaps[over_keys[name]] = row
        for li in range(c.layers):
            keys = pool.k[li, :rows].transpose(1, 2).contiguous()
            values = pool.v[li, :rows].transpose(1, 2).contiguous()
            for st, k, v in zip(states, keys.unbind(0), values.unbind(0)):
                st.transformer_keys[li] = k
                st.transformer_values[li] = v
        r = c.retained_context
        for st in states:
            st.frame_position += frames
            st.transformer_context_length = min(r, st.transformer_context_length + frames)

    def __call__(self, codes: torch.Tensor, states, *, position_ids: torch.Tensor | None = None,
                 context_lengths: torch.Tensor | None = None) -> torch.Tensor:
        """The reference's ``incremental_decoder`` call (model/incremental_codec.py:383-466, as
        CodecExecutor calls it at executor/codec.py:311-314 and 432-441): ``codes`` [B, Q, F]
        (equal fresh frames per row), one reference ``IncrementalCodecState`` per row (its mapping
        tensors are read, then replaced by new ones, and its frame position and context length
        advanced), optional device ``position_ids`` [B, F] (consecutive per row) and
        ``context_lengths`` [B].  Returns the clamped waveform [B, 1, F * samples_per_frame].

        Graph-capturable after one eager call of the same shape (the shape's device constants and
        staging buffers are made then) when position_ids and context_lengths are given."""

        c = self.config
        if not isinstance(codes, torch.Tensor) or codes.ndim != 3:
            raise ValueError(f"expected codec codes with rank 3, got shape {tuple(getattr(codes, 'shape', ()))}")
        rows, q, frames = (int(x) for x in codes.shape)
        if rows != len(states):
            raise ValueError(f"state count {len(states)} does not match batch {rows}")
        if q != c.num_quantizers:
            raise ValueError(f"expected {c.num_quantizers} codebooks, got {q}")
        if frames == 0:
            return torch.empty((rows, 1, 0), dtype=torch.float32, device=self.device)
        pool = self._staging(rows)
        self._stage_in(states, pool, rows, frames, position_ids, context_lengths)
        off_dev, off_host, slots = self._shape_tensors(rows, frames)
        packed = codes.to(device=self.device).permute(0, 2, 1).reshape(rows * frames, q).to(torch.int32).contiguous()
        wav, _ = self._run(packed, rows, off_dev, off_host, slots, pool)
        self._stage_out(states, pool, rows, frames)
        return wav.view(rows, 1, frames * c.samples_per_frame)

    def raise_on_status(self) -> None:
        """Fail closed at a point where the caller synchronizes anyway: a codec id outside the
        codebooks raises ValueError (the kernel used row 0 for it)."""

        code = int(self.status.item())
        if code != 0:
            self.status.zero_()
            raise ValueError("codec id outside the codebook range")

    # -- ragged chunks over the decoder's own state slots --------------------------------------
    def decode_ragged(self, codes, states: list[CodecStreamState]):
        """codes: [B, Q, F] or a list of [Q, F_b] tensors, one per stream (ragged); ``states`` are
        slots of this decoder (``new_state``).  Returns (wav list of [F_b * samples_per_frame] fp32,
        pcm16 list) per stream."""

        c = self.config
        chunks = list(codes) if not isinstance(codes, torch.Tensor) else [codes[i] for i in range(codes.shape[0])]
        if len(chunks) != len(states):
            raise ValueError(f"state count {len(states)} does not match batch {len(chunks)}")
        for ch in chunks:
            if ch.ndim != 2 or ch.shape[0] != c.num_quantizers:
                raise ValueError(f"expected [{c.num_quantizers}, frames] codes per stream")
        frames = [int(ch.shape[1]) for ch in chunks]
        B = len(chunks)
        off = np.zeros(B + 1, dtype=np.int64)
        off[1:] = np.cumsum(frames)
        if off[-1] == 0:
            return [torch.empty(0, device=self.device) for _ in chunks], [
                torch.empty(0, dtype=torch.int16, device=self.device) for _ in chunks]
        off_dev, slots, packed = self._stage_inputs(off, [st.slot for st in states], chunks)
        wav, pcm = self._run(packed, B, off_dev, off, slots, self.pool)
        r = c.retained_context
        for st, f in zip(states, frames):
            st.frame_position += f
            st.transformer_context_length = min(r, st.transformer_context_length + f)
        bounds = off * c.samples_per_frame
        return ([wav[bounds[i]: bounds[i + 1]] for i in range(B)], [pcm[bounds[i]: bounds[i + 1]] for i in range(B)])

    def _stage_inputs(self, off: np.ndarray, slots: list, chunks: list):
        """The packed codes [frames, Q], offsets [B + 1] and slots [B] (int32) copied to the device in one
        asynchronous copy from a pinned ring buffer."""
        B, total, q = len(slots), int(off[-1]), self.config.num_quantizers
        need = 2 * B + 1 + total * q
        entry = self._stage_ring[self._stage_next]
        self._stage_next = (self._stage_next + 1) % len(self._stage_ring)
        buf, done = entry
        if buf is None or buf.numel() < need:
            buf = torch.empty(max(need, 1 << 16), dtype=torch.int32, pin_memory=True)
        elif done is not None:
            done.synchronize()
        host = buf.numpy()
        nc = total * q  # the codes first, so that their copy keeps the allocation's alignment
        codes = host[:nc].reshape(total, q)
        host[nc:nc + B + 1] = off
        host[nc + B + 1:need] = slots
        row = 0
        for ch in chunks:
            f = int(ch.shape[1])
            codes[row:row + f] = ch.t().numpy() if ch.device.type == "cpu" else ch.t().cpu().numpy()
            row += f
        dev_buf = buf[:need].to(self.device, non_blocking=True)
        done = torch.cuda.Event()
        done.record()
        entry[0], entry[1] = buf, done
        return dev_buf[nc:nc + B + 1], dev_buf[nc + B + 1:need], dev_buf[:nc].view(total, q)

    # -- the step -------------------------------------------------------------
    def _run(self, packed: torch.Tensor, B: int, off_dev: torch.Tensor, off_host: np.ndarray, slots: torch.Tensor,
             pool: "_StatePool"):
        """One step over B streams whose fresh frames are the rows of ``packed`` [T, Q] (stream b owns
        rows off[b] .. off[b+1]), with state in ``pool`` slots ``slots``.  Returns (wav, pcm16), each
        [T * samples_per_frame]."""

        c, w = self.config, self.w
        dev = self.device
        T = int(off_host[-1])
        spf = c.samples_per_frame
        self._B = B
        self._off = off_dev
        self._slots = slots
        self._pool = pool
        self._stream = _lib.stream(dev)

        x = torch.empty(T, c.dim, dtype=torch.float32, device=dev)
        _lib.call("nq_codec_embed_sum", packed.data_ptr(), T, c.num_quantizers, w.codebooks.data_ptr(),
                  c.codebook_size, c.dim, x.data_ptr(), self.status.data_ptr(), self._stream)
        x = self._conv(x, 1, "pre_conv", w.pre_conv_w, w.pre_conv_b)

        # transformer (model/incremental_codec.py:193-381)
        hd = c.heads * c.head_dim
        r = c.retained_context
        h = self._sgemm(x, w.in_w, bias=w.in_b)
        att = torch.empty(T, hd, dtype=torch.float32, device=dev)
        for li, L in enumerate(w.tf):
            y = self._norm(h, L.ln1, c.eps)
            qkv = self._sgemm(y, L.wqkv)
            q, k, v = qkv[:, :hd], qkv[:, hd: 2 * hd], qkv[:, 2 * hd:]
            _lib.call("nq_codec_window_attention", q.data_ptr(), k.data_ptr(), v.data_ptr(), qkv.stride(0), T, c.heads,
                      c.head_dim, L.qn.data_ptr(), L.kn.data_ptr(), float(c.eps), float(c.theta), self._off.data_ptr(),
                      B, self._slots.data_ptr(), pool.frame_pos.data_ptr(), pool.ctx.data_ptr(), pool.k[li].data_ptr(),
                      pool.v[li].data_ptr(), pool.k.stride(1), r, c.window, att.data_ptr(), att.stride(0), self._stream)
            self._sgemm(att, L.wo, scale=L.ls1, res=h, out=h)
            y = self._norm(h, L.ln2, c.eps)
            self._sgemm(self._sgemm(y, L.w1, act=1), L.w2, scale=L.ls2, res=h, out=h)
        _lib.call("nq_codec_advance", self._off.data_ptr(), B, self._slots.data_ptr(), pool.frame_pos.data_ptr(),
                  pool.ctx.data_ptr(), r, self._stream)
        x = self._sgemm(self._norm(h, w.out_norm, c.eps), w.out_w, bias=w.out_b)

        # upsample: causal transconv + ConvNeXt
        u = 1
        for ui, (s, U) in enumerate(zip(c.up_strides, w.up)):
            x = self._transconv(x, u, s, f"up{ui}.tc", U.tc_w, U.tc_b)
            u *= s
            y = self._conv(x, u, f"up{ui}.dw", U.dw_w, U.dw_b, groups=c.dim)
            y = self._norm(y, U.ln_w, 1e-6, U.ln_b)
            self._sgemm(self._sgemm(y, U.pw1_w, bias=U.pw1_b, act=1), U.pw2_w, bias=U.pw2_b, scale=U.gamma, res=x,
                        out=x)
        # decoder blocks
        x = self._conv(x, u, "dec0", w.dec0_w, w.dec0_b)
        for bi, (s, Bk) in enumerate(zip(c.dec_strides, w.blocks)):
            x = self._transconv(x, u, s, f"dec{bi + 1}.tc", Bk.tc_w, Bk.tc_b, act=(Bk.alpha, Bk.beta))
            u *= s
            for j, (dil, R) in enumerate(zip(c.dilations, Bk.res)):
                x = self._res_unit(x, u, f"dec{bi + 1}.res{j}.a", R, dil)
        y = self._conv(x, u, "final", w.final_w, w.final_b, act=(w.final_alpha, w.final_beta))
        n = T * spf
        wav = torch.empty(n, dtype=torch.float32, device=dev)
        pcm = torch.empty(n, dtype=torch.int16, device=dev)
        _lib.call("nq_codec_pcm16", y.data_ptr(), n, wav.data_ptr(), pcm.data_ptr(), self._stream)
        return wav, pcm




__all__ = ["CodecConfig", "CodecStreamState", "CodecWeights", "IncrementalCodecDecoder"]
