"""Norm and SwiGLU entry points with the reference's call shapes.

``qwen3_tts_add_rmsnorm`` / ``qwen3_tts_rmsnorm`` / ``qwen3_tts_silu_and_mul``
mirror model/layers.py:28-100: the fused add-norm updates both inputs in
place (residual <- residual + hidden, hidden <- rmsnorm(residual)).
"""

from __future__ import annotations

import torch

from . import _lib


def _check(t: torch.Tensor, name: str) -> None:
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bf16")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    _lib.require_device(t)


def qwen3_tts_add_rmsnorm(hidden: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    _check(hidden, "hidden_states")
    _check(residual, "residual")
    _check(weight, "norm weight")
    if hidden.shape != residual.shape or hidden.data_ptr() == residual.data_ptr():
        raise ValueError("fused add-RMSNorm needs distinct tensors of one shape")
    width = hidden.shape[-1]
    if weight.shape != (width,):
        raise ValueError("norm weight must match the hidden width")
    _lib.call(
        "nq_add_rmsnorm", hidden.data_ptr(), residual.data_ptr(), weight.data_ptr(), hidden.numel() // width, width,
        float(eps), _lib.stream(hidden.device),
    )
    return hidden, residual


def qwen3_tts_rmsnorm(hidden: torch.Tensor, weight: torch.Tensor, eps: float, out: torch.Tensor | None = None):
    _check(hidden, "hidden_states")
    _check(weight, "norm weight")
    width = hidden.shape[-1]
    if weight.shape != (width,):
        raise ValueError("norm weight must match the hidden width")
    out = torch.empty_like(hidden) if out is None else out
    _lib.call(
        "nq_rmsnorm", hidden.data_ptr(), weight.data_ptr(), out.data_ptr(), hidden.numel() // width, width,
        float(eps), _lib.stream(hidden.device),
    )
    return out


def qwen3_tts_silu_and_mul(gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    _check(gate_up, "gate_up")
    width = gate_up.shape[-1] // 2
    if gate_up.shape[-1] != 2 * width:
        raise ValueError("gate_up must have an even last dimension")
    rows = gate_up.numel() // gate_up.shape[-1]
    out = torch.empty((*gate_up.shape[:-1], width), dtype=gate_up.dtype, device=gate_up.device) if out is None else out
    _lib.call("nq_silu_mul", gate_up.data_ptr(), out.data_ptr(), rows, width, _lib.stream(gate_up.device))
    return out


__all__ = ["qwen3_tts_add_rmsnorm", "qwen3_tts_rmsnorm", "qwen3_tts_silu_and_mul"]
