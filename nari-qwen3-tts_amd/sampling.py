"""Graph-safe samplers backed by the fused HIP sampler.

``sample_with_uniforms`` is the north-star entry: caller-supplied uniforms,
token ids bit-exact against the oracle.  The three reference entry points
keep their signatures (executor/sampling.py:156-198, 201-239, 305-336): the
same fused kernel draws each row's uniform from its (seed, offset) counter
with Philox-4x32-10 (``sample_with_counter``, identical to
``uniforms_from_counter`` then ``sample_with_uniforms``), so a request's draw
depends only on its own counter (row-local, batch- and permutation-invariant
like model/sampling.py:192-195).
"""

from __future__ import annotations

import torch

from . import _lib


def uniforms_from_counter(seed: torch.Tensor, offset: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    if seed.dtype != torch.long or offset.dtype != torch.long:
        raise TypeError("seed and offset must use torch.int64")
    if seed.ndim != 1 or offset.ndim != 1 or seed.shape != offset.shape:
        raise ValueError("seed and offset must be row vectors of one length")
    _lib.require_device(seed, offset)
    rows = seed.shape[0]
    out = torch.empty(rows, dtype=torch.float32, device=seed.device) if out is None else out
    _lib.call(
        "nq_uniforms_from_counter",
        seed.data_ptr(), seed.stride(0), offset.data_ptr(), offset.stride(0), rows, out.data_ptr(),
        _lib.stream(seed.device),
    )
    return out


def _sample(
    logits: torch.Tensor,
    temperature: torch.Tensor,
    top_k: torch.Tensor,
    top_p: torch.Tensor,
    uniforms: torch.Tensor | None,
    seed: torch.Tensor | None,
    offset: torch.Tensor | None,
    *,
    repetition_penalty: torch.Tensor | None = None,
    seen_token_mask: torch.Tensor | None = None,
    mask_from: int | None = None,
    eos_id: int = -1,
    suppress_eos: torch.Tensor | None = None,
    update_seen: bool = False,
    out: torch.Tensor | None = None,
    planes: torch.Tensor | None = None,
    logits_out: torch.Tensor | None = None,
) -> torch.Tensor:
    if planes is not None:
        # fp32 split-K planes [S, rows, vocab] of the projection that makes the logits
        if planes.dtype != torch.float32 or planes.ndim != 3 or not planes.is_contiguous():
            raise TypeError("planes must be a contiguous float32 [splits, rows, vocabulary] tensor")
        logits = planes[0]
        if logits_out is not None and (logits_out.dtype != torch.bfloat16 or logits_out.shape != logits.shape
                                       or logits_out.stride(1) != 1):
            raise ValueError("logits_out must be a bf16 [rows, vocabulary] tensor with contiguous rows")
    if logits.ndim != 2 or logits.shape[0] < 1:
        raise ValueError("logits must have shape (rows, vocabulary)")
    rows, vocab = logits.shape
    if logits.dtype == torch.float32:
        code = _lib.NQ_F32
    elif logits.dtype == torch.bfloat16:
        code = _lib.NQ_BF16
    else:
        raise TypeError("logits must be float32 or bfloat16")
    if logits.stride(1) != 1:
        raise ValueError("logits rows must be contiguous")
    vectors = [("temperature", temperature, torch.float32), ("top_k", top_k, torch.int32), ("top_p", top_p, torch.float32)]
    if uniforms is not None:
        vectors.append(("uniforms", uniforms, torch.float32))
    for name, t, dtype in vectors:
        if t.dtype != dtype:
            raise TypeError(f"{name} must use {dtype}, got {t.dtype}")
        if t.shape != (rows,) or (rows > 1 and t.stride(0) != 1):
            raise ValueError(f"{name} must be a contiguous row vector with {rows} entries")
    if uniforms is None:
        if seed.dtype != torch.long or offset.dtype != torch.long:
            raise TypeError("seed and offset must use torch.int64")
        if seed.shape != (rows,) or offset.shape != (rows,):
            raise ValueError(f"seed and offset must be row vectors with {rows} entries")
    if repetition_penalty is not None:
        if repetition_penalty.dtype != torch.float32:
            raise TypeError("repetition_penalty must use torch.float32")
        if repetition_penalty.shape != (rows,):
            raise ValueError(f"repetition_penalty must be a row vector with {rows} entries")
    if seen_token_mask is not None:
        if seen_token_mask.dtype != torch.bool:
            raise TypeError("seen_token_mask must use torch.bool")
        if seen_token_mask.shape != logits.shape or seen_token_mask.stride(1) != 1:
            raise ValueError("seen_token_mask must match the logits shape")
    if update_seen and seen_token_mask is None:
        raise ValueError("update_seen needs a seen_token_mask")
    if suppress_eos is not None and (suppress_eos.dtype != torch.bool or suppress_eos.shape != (rows,)):
        raise ValueError("suppress_eos must be a bool row vector")
    _lib.require_device(logits, temperature, top_k, top_p, uniforms, seed, offset, repetition_penalty, seen_token_mask,
                        suppress_eos, logits_out)
    tokens = torch.empty(rows, dtype=torch.long, device=logits.device) if out is None else out
    head = (logits.data_ptr(), code, logits.stride(0), rows, vocab, temperature.data_ptr(), top_k.data_ptr(),
            top_p.data_ptr(), _lib.ptr(repetition_penalty), _lib.ptr(seen_token_mask),
            0 if seen_token_mask is None else seen_token_mask.stride(0))
    tail = (vocab if mask_from is None else int(mask_from), int(eos_id), _lib.ptr(suppress_eos), int(update_seen),
            tokens.data_ptr(), _lib.stream(logits.device))
    if planes is not None:
        if uniforms is not None:
            raise ValueError("the split-K plane source draws its uniforms from (seed, offset)")
        _lib.call("nq_sample_counter_planes", planes.data_ptr(), planes.shape[0], logits.stride(0), rows, vocab,
                  *head[5:], seed.data_ptr(), seed.stride(0), offset.data_ptr(), offset.stride(0), *tail[:4],
                  _lib.ptr(logits_out), 0 if logits_out is None else logits_out.stride(0), *tail[4:])
    elif uniforms is not None:
        _lib.call("nq_sample", *head, uniforms.data_ptr(), *tail)
    else:
        _lib.call("nq_sample_counter", *head, seed.data_ptr(), seed.stride(0), offset.data_ptr(), offset.stride(0), *tail)
    return tokens


def sample_with_uniforms(logits, temperature, top_k, top_p, uniforms, **kwargs) -> torch.Tensor:
    """One token per row: masks, penalty, temperature, top-k, top-p, inverse-CDF draw with the
    caller's uniforms."""

    return _sample(logits, temperature, top_k, top_p, uniforms, None, None, **kwargs)


def sample_with_counter(logits, temperature, top_k, top_p, seed, offset, **kwargs) -> torch.Tensor:
    """As sample_with_uniforms with row r's uniform drawn in the same launch from its (seed, offset)
    counter exactly as uniforms_from_counter computes it (same tokens, one launch)."""

    return _sample(logits, temperature, top_k, top_p, None, seed, offset, **kwargs)


def sample_with_counter_from_planes(planes, temperature, top_k, top_p, seed, offset, *, logits_out=None,
                                    **kwargs) -> torch.Tensor:
    """sample_with_counter over the logits held as a projection's fp32 split-K planes [S, rows, vocab]
    (``layers.linear_partials``): each logit is the planes' sum in plane order rounded to bf16, the
    value ``layers.linear`` stores, so the tokens are those of linear + sample_with_counter, in one
    launch; the bf16 logits also go to ``logits_out`` when given."""

    return _sample(None, temperature, top_k, top_p, None, seed, offset, planes=planes, logits_out=logits_out,
                   **kwargs)


def sample_talker_cuda_graph(
    logits: torch.Tensor,
    temperature: torch.Tensor,
    top_k: torch.Tensor,
    top_p: torch.Tensor,
    seed: torch.Tensor,
    offset: torch.Tensor,
    repetition_penalty: torch.Tensor,
    seen_token_mask: torch.Tensor,
) -> torch.Tensor:
    """Talker draw with penalty over seen ids; the caller updates ``seen``."""

    return sample_with_counter(
        logits, temperature, top_k, top_p, seed, offset, repetition_penalty=repetition_penalty,
        seen_token_mask=seen_token_mask,
    )


def sample_logits_cuda_graph(logits, temperature, top_k, top_p, seed, offset) -> torch.Tensor:
    """General-route draw (any top_k, no penalty)."""

    return sample_with_counter(logits, temperature, top_k, top_p, seed, offset)


def sample_code_predictor_cuda_graph(logits, temperature, top_k, top_p, seed, offset) -> torch.Tensor:
    """Fused code-predictor draw; ``offset`` may be a strided column of [rows, 15]."""

    return sample_with_counter(logits, temperature, top_k, top_p, seed, offset)


__all__ = [
    "sample_code_predictor_cuda_graph",
    "sample_logits_cuda_graph",
    "sample_talker_cuda_graph",
    "sample_with_counter",
    "sample_with_counter_from_planes",
    "sample_with_uniforms",
    "uniforms_from_counter",
]
