"""Norm, SwiGLU and projection entry points with the reference's call shapes.

``qwen3_tts_add_rmsnorm`` / ``qwen3_tts_rmsnorm`` / ``qwen3_tts_silu_and_mul``
mirror model/layers.py:28-100: the fused add-norm updates both inputs in
place (residual <- residual + hidden, hidden <- rmsnorm(residual)).
``linear`` is the bias-free nn.Linear of model/layers.py:195-270 for decode
row counts (<= 128), computed by the skinny HIP GEMM.
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


def linear_workspace_bytes(rows: int, out_features: int, in_features: int, epilogue: int = _lib.NQ_EPI_NONE) -> int:
    """fp32 split-K scratch the projection needs (0 when none); raises for shapes it does not cover."""

    n = int(_lib.load().nq_linear_workspace_bytes(int(rows), int(out_features), int(in_features), int(epilogue)))
    if n < 0:
        raise TypeError(f"no HIP projection for rows={rows}, out={out_features}, in={in_features}")
    return n


def _linear(x, weight, epilogue, out, out_width, residual=None, norm_weight=None, eps=0.0, workspace=None,
            bias=None):
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("linear needs bf16 activations and weights")
    if x.dim() != 2 or weight.dim() != 2 or x.stride(1) != 1 or weight.stride(1) != 1:
        raise ValueError("linear needs 2-D tensors with unit inner stride")
    rows, k = x.shape
    n = weight.shape[0]
    if weight.shape[1] != k:
        raise ValueError("weight in_features must match x")
    _lib.require_device(x, weight)
    need = linear_workspace_bytes(rows, n, k, epilogue)
    out = torch.empty((rows, out_width), dtype=x.dtype, device=x.device) if out is None else out
    if out.shape != (rows, out_width) or out.stride(1) != 1 or out.dtype != torch.bfloat16:
        raise ValueError(f"out must be bf16 [{rows}, {out_width}] with unit inner stride")
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    _lib.call(
        "nq_linear", x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0), rows, n, k, int(epilogue),
        _lib.ptr(bias), out.data_ptr(), out.stride(0), _lib.ptr(residual), _lib.ptr(norm_weight), float(eps),
        _lib.ptr(workspace) if need else None, workspace.numel() * workspace.element_size() if need else 0,
        _lib.stream(x.device),
    )
    return out


def linear(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor | None = None,
           workspace: torch.Tensor | None = None, bias: torch.Tensor | None = None) -> torch.Tensor:
    """out = x @ weight.T (+ bias) for bf16 x [rows, in] (row stride free) and weight [out, in]."""

    if bias is not None:
        _check(bias, "bias")
        if bias.shape != (weight.shape[0],):
            raise ValueError("bias must match out_features")
    return _linear(x, weight, _lib.NQ_EPI_NONE, out, weight.shape[0], workspace=workspace, bias=bias)


def linear_add_rmsnorm(x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor, norm_weight: torch.Tensor,
                       eps: float, out: torch.Tensor, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """The projection followed by the fused add-RMSNorm: residual += x @ weight.T (bf16);
    out = rmsnorm(residual) * norm_weight."""

    for t, name in ((residual, "residual"), (norm_weight, "norm weight")):
        _check(t, name)
    if residual.shape != (x.shape[0], weight.shape[0]) or norm_weight.shape != (weight.shape[0],):
        raise ValueError("residual / norm weight must match the projection output")
    return _linear(x, weight, _lib.NQ_EPI_ADD_RMSNORM, out, weight.shape[0], residual, norm_weight, eps, workspace)


def linear_partials(x: torch.Tensor, weight: torch.Tensor, workspace: torch.Tensor) -> int:
    """Run the projection but leave its fp32 split-K planes [S, rows, out] at the start of
    ``workspace`` for a consumer that sums them; returns S."""

    rows, k = x.shape
    n = weight.shape[0]
    splits = int(_lib.load().nq_linear_splits(rows, n, k))
    if splits < 1:
        raise TypeError(f"no HIP projection for rows={rows}, out={n}, in={k}")
    need = linear_workspace_bytes(rows, n, k, _lib.NQ_EPI_PARTIALS)
    if workspace.numel() * workspace.element_size() < need:
        raise ValueError("workspace too small for the projection partials")
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16 or x.stride(1) != 1 or weight.stride(1) != 1:
        raise TypeError("linear needs bf16 tensors with unit inner stride")
    _lib.require_device(x, weight, workspace)
    _lib.call("nq_linear", x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0), rows, n, k,
              _lib.NQ_EPI_PARTIALS, None, None, 0, None, None, 0.0, workspace.data_ptr(),
              workspace.numel() * workspace.element_size(), _lib.stream(x.device))
    return splits


def linear_silu_mul(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor | None = None,
                    workspace: torch.Tensor | None = None) -> torch.Tensor:
    """SwiGLU input: y = x @ weight.T with weight [2 * I, in] (gate rows, then up rows);
    out = silu(y[:, :I]) * y[:, I:]."""

    if weight.shape[0] % 2:
        raise ValueError("gate_up weight needs an even number of rows")
    return _linear(x, weight, _lib.NQ_EPI_SILU_MUL, out, weight.shape[0] // 2, workspace=workspace)


__all__ = [
    "linear",
    "linear_add_rmsnorm",
    "linear_partials",
    "linear_silu_mul",
    "linear_workspace_bytes",
    "qwen3_tts_add_rmsnorm",
    "qwen3_tts_rmsnorm",
    "qwen3_tts_silu_and_mul",
]
