"""Norm, SwiGLU and projection entry points with the reference's call shapes.

``qwen3_tts_add_rmsnorm`` / ``qwen3_tts_rmsnorm`` / ``qwen3_tts_silu_and_mul``
keep the signatures of model/layers.py:28-100 (the RMSNorm module, the
``use_cuda_kernel`` keyword and the reference's own torch math for inputs it
does not send to a kernel); the fused add-norm updates both inputs in place
(residual <- residual + hidden, hidden <- rmsnorm(residual)).  The
(weight, eps) forms ``add_rmsnorm`` / ``rmsnorm`` / ``silu_mul`` are what the
step code calls.
``linear`` is the bias-free nn.Linear of model/layers.py:195-270 for decode
row counts (<= 128), computed by the skinny HIP GEMM.

FP8 gate/up (model/layers.py:10-25, 195-262): ``quantize_fp8_weight_blocks``
keeps the reference's name, block layout and errors; the activations are
quantized per row and 128 columns by the add-RMSNorm that produces them
(``add_rmsnorm_fp8`` / ``linear_add_rmsnorm_fp8``) or by
``quantize_fp8_rows``, and ``linear_fp8`` runs the block-scaled product.
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


def _check_out(out: torch.Tensor, like: torch.Tensor, shape, name: str = "out") -> None:
    if out.dtype != like.dtype or out.device != like.device:
        raise TypeError(f"{name} must match the input's dtype and device")
    if tuple(out.shape) != tuple(shape) or not out.is_contiguous():
        raise ValueError(f"{name} must be a contiguous tensor of shape {tuple(shape)}")


def add_rmsnorm(hidden: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    """In place: residual <- bf16(residual + hidden), hidden <- rmsnorm(residual) * weight."""

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


def rmsnorm(hidden: torch.Tensor, weight: torch.Tensor, eps: float, out: torch.Tensor | None = None):
    """out = rmsnorm(hidden) * weight (bf16 in and out, fp32 statistics)."""

    _check(hidden, "hidden_states")
    _check(weight, "norm weight")
    width = hidden.shape[-1]
    if weight.shape != (width,):
        raise ValueError("norm weight must match the hidden width")
    if out is None:
        out = torch.empty_like(hidden)
    else:
        _check_out(out, hidden, hidden.shape)
    _lib.call(
        "nq_rmsnorm", hidden.data_ptr(), weight.data_ptr(), out.data_ptr(), hidden.numel() // width, width,
        float(eps), _lib.stream(hidden.device),
    )
    return out


def silu_mul(gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """out = silu(gate) * up over the two halves of the last dimension (bf16)."""

    _check(gate_up, "gate_up")
    width = gate_up.shape[-1] // 2
    if gate_up.shape[-1] != 2 * width:
        raise ValueError("gate_up must have an even last dimension")
    rows = gate_up.numel() // gate_up.shape[-1]
    shape = (*gate_up.shape[:-1], width)
    if out is None:
        out = torch.empty(shape, dtype=gate_up.dtype, device=gate_up.device)
    else:
        _check_out(out, gate_up, shape)
    _lib.call("nq_silu_mul", gate_up.data_ptr(), out.data_ptr(), rows, width, _lib.stream(gate_up.device))
    return out


def _kernel_input(t: torch.Tensor, use_cuda_kernel: bool) -> bool:
    """The reference's dispatch guard (model/layers.py:34,63-71,89): a kernel takes CUDA-device
    half-precision inputs; everything else runs the reference's own torch math.  Here the kernel
    is bf16 only, so an fp16 device tensor that the reference would send to its kernel is refused
    instead of being computed some other way."""

    if not (use_cuda_kernel and t.is_cuda and t.dtype in (torch.float16, torch.bfloat16)):
        return False
    if t.dtype != torch.bfloat16:
        raise TypeError("the HIP norm / SwiGLU kernels take bf16 device tensors (fp16 is not built)")
    return True


def _norm_weight(norm) -> torch.Tensor:
    weight = norm.weight
    if weight.dtype != torch.bfloat16:
        raise TypeError("RMSNorm weight must be bf16 for the HIP kernel")
    return weight.detach()


def qwen3_tts_silu_and_mul(gate_up: torch.Tensor, *, use_cuda_kernel: bool = True) -> torch.Tensor:
    """Drop-in for model/layers.py:28-39: SwiGLU of the two halves of ``gate_up``'s last dimension.

    bf16 device tensors run ``nq_silu_mul``; other inputs take the reference's torch math, as the
    reference does for them."""

    if _kernel_input(gate_up, use_cuda_kernel):
        return silu_mul(gate_up if gate_up.is_contiguous() else gate_up.contiguous())
    gate, up = gate_up.chunk(2, dim=-1)
    return torch.nn.functional.silu(gate) * up


def qwen3_tts_add_rmsnorm(hidden_states: torch.Tensor, residual: torch.Tensor, norm, *,
                          use_cuda_kernel: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    """Drop-in for model/layers.py:42-78: residual add + the following RMSNorm (``norm`` is the
    reference's RMSNorm module: ``weight`` and ``variance_epsilon`` are read from it).

    Device inputs that the reference hands to its fused kernel (half precision, contiguous, same
    shape, distinct storage) run ``nq_add_rmsnorm`` in place on both tensors and are returned;
    the others take the reference's own torch math and return new tensors."""

    if (
        _kernel_input(hidden_states, use_cuda_kernel)
        and hidden_states.is_contiguous()
        and residual.is_contiguous()
        and hidden_states.shape == residual.shape
        and hidden_states.data_ptr() != residual.data_ptr()
    ):
        add_rmsnorm(hidden_states, residual, _norm_weight(norm), float(norm.variance_epsilon))
        return hidden_states, residual
    residual = residual + hidden_states
    return norm(residual), residual


def qwen3_tts_rmsnorm(hidden_states: torch.Tensor, norm, *, use_cuda_kernel: bool = True) -> torch.Tensor:
    """Drop-in for model/layers.py:81-100: one RMSNorm (``norm.weight``, ``norm.variance_epsilon``)."""

    if _kernel_input(hidden_states, use_cuda_kernel):
        x = hidden_states if hidden_states.is_contiguous() else hidden_states.contiguous()
        return rmsnorm(x, _norm_weight(norm), float(norm.variance_epsilon))
    return norm(hidden_states)


def embed_add_rmsnorm(ids: torch.Tensor, table: torch.Tensor, addend: torch.Tensor | None, weight: torch.Tensor,
                      eps: float, residual: torch.Tensor, out: torch.Tensor,
                      status: torch.Tensor | None = None) -> torch.Tensor:
    """residual = bf16(addend + table[ids]) (the gathered row itself when ``addend`` is None);
    out = rmsnorm(residual) * weight, one launch (the talker step's input embedding and first input
    norm; the code predictor's next input and first input norm).  ``status`` (int32 [1], optional)
    receives NQ_ERR_INVALID_ARGUMENT for an id outside the table."""

    for t, name in ((table, "embedding table"), (addend, "addend"), (weight, "norm weight"), (residual, "residual"),
                    (out, "out")):
        if t is not None and (t.dtype != torch.bfloat16 or t.stride(-1) != 1):
            raise TypeError(f"{name} must be bf16 with unit inner stride")
    if ids.dtype != torch.long or ids.ndim != 1:
        raise TypeError("ids must be an int64 vector")
    if ids.stride(0) != 1:
        raise ValueError("ids must be a unit-stride vector")
    rows, width = residual.shape
    if ids.shape != (rows,) or table.shape[1] != width or weight.shape != (width,):
        raise ValueError("ids / table / norm weight do not match the residual")
    if addend is not None and addend.shape != (rows, width):
        raise ValueError("addend must match the residual")
    if out.shape != (rows, width) or not residual.is_contiguous() or not out.is_contiguous():
        raise ValueError("residual and out must be contiguous [rows, width]")
    _lib.require_device(ids, table, addend, weight, residual, out, status)
    _lib.call("nq_embed_add_rmsnorm", ids.data_ptr(), table.data_ptr(), table.stride(0), table.shape[0],
              _lib.ptr(addend), 0 if addend is None else addend.stride(0), weight.data_ptr(), rows, width, float(eps),
              residual.data_ptr(), out.data_ptr(), _lib.ptr(status), _lib.stream(residual.device))
    return out


def prefill_embed_rmsnorm(text_ids: torch.Tensor, text_table: torch.Tensor, codec_ids: torch.Tensor,
                          codec_table: torch.Tensor, mask: torch.Tensor, weight: torch.Tensor, eps: float,
                          residual: torch.Tensor, out: torch.Tensor, status: torch.Tensor | None = None) -> torch.Tensor:
    """Prefill input embedding (executor/talker.py:246-254) and the first input norm in one launch:
    residual = where(mask, text_table[text_ids] + codec_table[codec_ids], text_table[text_ids]) (bf16),
    out = rmsnorm(residual) * weight."""

    for t, name in ((text_table, "text table"), (codec_table, "codec table"), (weight, "norm weight"),
                    (residual, "residual"), (out, "out")):
        if t.dtype != torch.bfloat16 or t.stride(-1) != 1:
            raise TypeError(f"{name} must be bf16 with unit inner stride")
    for ids, name in ((text_ids, "text_ids"), (codec_ids, "codec_ids")):
        if ids.dtype != torch.long or ids.ndim != 1 or ids.stride(0) != 1:
            raise TypeError(f"{name} must be a unit-stride int64 vector")
    if mask.dtype != torch.bool or mask.ndim != 1 or mask.stride(0) != 1:
        raise TypeError("mask must be a unit-stride bool vector")
    rows, width = residual.shape
    if text_ids.shape != (rows,) or codec_ids.shape != (rows,) or mask.shape != (rows,):
        raise ValueError("ids / mask must have one entry per row")
    if text_table.shape[1] != width or codec_table.shape[1] != width or weight.shape != (width,):
        raise ValueError("tables / norm weight do not match the residual width")
    if out.shape != (rows, width) or not residual.is_contiguous() or not out.is_contiguous():
        raise ValueError("residual and out must be contiguous [rows, width]")
    _lib.require_device(text_ids, text_table, codec_ids, codec_table, mask, weight, residual, out, status)
    _lib.call("nq_prefill_embed_rmsnorm", text_ids.data_ptr(), text_table.data_ptr(), text_table.stride(0),
              text_table.shape[0], codec_ids.data_ptr(), codec_table.data_ptr(), codec_table.stride(0),
              codec_table.shape[0], mask.data_ptr(), weight.data_ptr(), rows, width, float(eps), residual.data_ptr(),
              out.data_ptr(), _lib.ptr(status), _lib.stream(residual.device))
    return out


def linear_rows(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor, workspace: torch.Tensor | None = None,
                chunk: int = 128) -> torch.Tensor:
    """out = x @ weight.T for any number of rows: the decode-sized projection over row pieces of at
    most ``chunk`` rows (each piece streams the weights again; the prefill buckets' projections)."""

    rows = x.shape[0]
    for r0 in range(0, rows, chunk):
        r1 = min(rows, r0 + chunk)
        linear(x[r0:r1], weight, out=out[r0:r1], workspace=workspace)
    return out


def tgemm_workspace_bytes(rows: int, out_features: int, in_features: int,
                          epilogue: int = _lib.NQ_EPI_NONE) -> int:
    """fp32 split-K planes the tiled prefill GEMM needs (0 when none); raises for shapes it does not cover."""

    n = int(_lib.load().nq_tgemm_workspace_bytes(int(rows), int(out_features), int(in_features), int(epilogue)))
    if n < 0:
        raise TypeError(f"no tiled projection for rows={rows}, out={out_features}, in={in_features}")
    return n


def _tgemm_args(x, weight):
    for t, name in ((x, "x"), (weight, "weight")):
        if t.dtype != torch.bfloat16 or t.dim() != 2 or t.stride(1) != 1:
            raise TypeError(f"{name} must be a bf16 matrix with unit inner stride")
    if weight.shape[1] != x.shape[1]:
        raise ValueError("weight in_features must match x")
    _lib.require_device(x, weight)
    return x.shape[0], weight.shape[0], x.shape[1]


def _workspace(ws, need, device):
    if need and (ws is None or ws.numel() * ws.element_size() < need):
        raise ValueError(f"the tiled projection needs a workspace of {need} bytes")
    return (ws.data_ptr(), ws.numel() * ws.element_size()) if need else (None, 0)


def tgemm(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor, epilogue: int = _lib.NQ_EPI_NONE,
          residual: torch.Tensor | None = None, norm_weight: torch.Tensor | None = None, eps: float = 0.0,
          workspace: torch.Tensor | None = None) -> torch.Tensor:
    """The tiled prefill GEMM for any number of rows, with the epilogues of ``linear``: out = x @ weight.T
    (NQ_EPI_NONE), silu(bf16(gate)) * bf16(up) on [gate; up] weights (NQ_EPI_SILU_MUL), or
    residual += x @ weight.T, out = rmsnorm(residual) * norm_weight (NQ_EPI_ADD_RMSNORM)."""

    rows, n, k = _tgemm_args(x, weight)
    width = n // 2 if epilogue == _lib.NQ_EPI_SILU_MUL else n
    if out.dtype != torch.bfloat16 or out.shape != (rows, width) or out.stride(1) != 1:
        raise ValueError(f"out must be bf16 [{rows}, {width}] with unit inner stride")
    if epilogue == _lib.NQ_EPI_ADD_RMSNORM:
        for t, name in ((residual, "residual"), (norm_weight, "norm weight")):
            _check(t, name)
        if residual.shape != (rows, n) or norm_weight.shape != (n,) or not residual.is_contiguous():
            raise ValueError("residual / norm weight must match the projection output")
    ws, ws_bytes = _workspace(workspace, tgemm_workspace_bytes(rows, n, k, epilogue), x.device)
    _lib.call("nq_tgemm", x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0), rows, n, k, int(epilogue),
              out.data_ptr(), out.stride(0), _lib.ptr(residual), _lib.ptr(norm_weight), float(eps), ws, ws_bytes,
              _lib.stream(x.device))
    return out


def tgemm_partials(x: torch.Tensor, weight: torch.Tensor, workspace: torch.Tensor) -> int:
    """The tiled GEMM leaving its fp32 split-K planes [S, rows, out] at the start of ``workspace``
    (the layout ``linear_partials`` leaves); returns S."""

    rows, n, k = _tgemm_args(x, weight)
    ws, ws_bytes = _workspace(workspace, tgemm_workspace_bytes(rows, n, k, _lib.NQ_EPI_PARTIALS), x.device)
    _lib.call("nq_tgemm", x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0), rows, n, k,
              _lib.NQ_EPI_PARTIALS, None, 0, None, None, 0.0, ws, ws_bytes, _lib.stream(x.device))
    return int(_lib.load().nq_tgemm_splits(rows, n, k))


def tgemm_add_rmsnorm_fp8(x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor, norm_weight: torch.Tensor,
                          eps: float, q: torch.Tensor, scales: torch.Tensor, workspace: torch.Tensor):
    """The tiled GEMM followed by the add-RMSNorm with the normalised rows stored as FP8 codes and
    per-128-column scales (linear_add_rmsnorm_fp8 for any number of rows)."""

    rows, n, k = _tgemm_args(x, weight)
    for t, name in ((residual, "residual"), (norm_weight, "norm weight")):
        _check(t, name)
    if residual.shape != (rows, n) or norm_weight.shape != (n,):
        raise ValueError("residual / norm weight must match the projection output")
    q, scales = _fp8_out(rows, n, x.device, q, scales)
    ws, ws_bytes = _workspace(workspace, tgemm_workspace_bytes(rows, n, k, _lib.NQ_EPI_ADD_RMSNORM), x.device)
    _lib.call("nq_tgemm_add_rmsnorm_fp8", x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0), rows, n,
              k, residual.data_ptr(), norm_weight.data_ptr(), float(eps), q.data_ptr(), q.stride(0),
              scales.data_ptr(), scales.stride(0), ws, ws_bytes, _lib.stream(x.device))
    return q, scales


def tgemm_fp8_swiglu(q: torch.Tensor, scales: torch.Tensor, packed: torch.Tensor, weight_scales: torch.Tensor,
                     out: torch.Tensor) -> torch.Tensor:
    """The tiled prefill form of linear_fp8_swiglu (same codes, scales and interleaved weights) for any
    number of rows."""

    rows, k = q.shape
    inter = packed.shape[0] // 2
    if q.dtype != FP8 or packed.dtype != FP8 or packed.shape[1] != k:
        raise TypeError("FP8 codes expected")
    if scales.shape != (rows, k // 128) or weight_scales.shape != (2 * inter // 128, k // 128):
        raise ValueError("FP8 scales do not match")
    if out.shape != (rows, inter) or out.dtype != torch.bfloat16 or out.stride(1) != 1:
        raise ValueError(f"out must be bf16 [{rows}, {inter}] with unit inner stride")
    _lib.require_device(q, scales, packed, weight_scales, out)
    _lib.call("nq_tgemm_fp8_swiglu", q.data_ptr(), q.stride(0), scales.data_ptr(), scales.stride(0), rows,
              packed.data_ptr(), packed.stride(0), weight_scales.data_ptr(), weight_scales.stride(0), inter, k,
              out.data_ptr(), out.stride(0), _lib.stream(q.device))
    return out


def gather_sum_rows(first_ids: torch.Tensor, first_table: torch.Tensor, ids: torch.Tensor, tables: torch.Tensor,
                    out: torch.Tensor, status: torch.Tensor | None = None) -> torch.Tensor:
    """out[r] = first_table[first_ids[r]] + sum over g of tables[g][ids[g, r]], added in group order
    with each partial sum rounded to bf16 (the code predictor's codec_sum in one launch).
    ``ids`` int64 [G, rows] (any strides); ``tables`` bf16 [>= G, V, width]."""

    if first_ids.dtype != torch.long or ids.dtype != torch.long or first_ids.ndim != 1 or ids.ndim != 2:
        raise TypeError("ids must be int64: first_ids [rows], ids [groups, rows]")
    if first_ids.stride(0) != 1:
        raise ValueError("first_ids must be a unit-stride vector")
    for t, name in ((first_table, "first table"), (tables, "tables"), (out, "out")):
        if t.dtype != torch.bfloat16 or t.stride(-1) != 1:
            raise TypeError(f"{name} must be bf16 with unit inner stride")
    groups, rows = ids.shape
    width = out.shape[1]
    if first_ids.shape != (rows,) or out.shape[0] != rows or first_table.shape[1] != width or tables.ndim != 3 \
            or tables.shape[0] < groups or tables.shape[2] != width:
        raise ValueError("ids / tables / out shapes do not match")
    _lib.require_device(first_ids, first_table, ids, tables, out, status)
    _lib.call("nq_gather_sum_rows", first_ids.data_ptr(), first_table.data_ptr(), first_table.stride(0),
              first_table.shape[0], ids.data_ptr(), ids.stride(0), ids.stride(1), tables.data_ptr(), tables.stride(0),
              tables.stride(1), tables.shape[1], groups, rows, width, out.data_ptr(), out.stride(0), _lib.ptr(status),
              _lib.stream(out.device))
    return out


def linear_workspace_bytes(rows: int, out_features: int, in_features: int, epilogue: int = _lib.NQ_EPI_NONE) -> int:
    """fp32 split-K scratch the projection needs (0 when none); raises for shapes it does not cover."""

    n = int(_lib.load().nq_linear_workspace_bytes(int(rows), int(out_features), int(in_features), int(epilogue)))
    if n < 0:
        raise TypeError(f"no HIP projection for rows={rows}, out={out_features}, in={in_features}")
    return n


def _weight_arg(weight, k: int) -> tuple[int, int, int]:
    """(pointer, row stride, out_features) of a projection weight."""

    if weight.dtype != torch.bfloat16 or weight.dim() != 2 or weight.stride(1) != 1:
        raise TypeError("linear needs a bf16 2-D weight with unit inner stride")
    if weight.shape[1] != k:
        raise ValueError("weight in_features must match x")
    return weight.data_ptr(), weight.stride(0), weight.shape[0]


def _linear(x, weight, epilogue, out, out_width, residual=None, norm_weight=None, eps=0.0, workspace=None,
            bias=None):
    if x.dtype != torch.bfloat16:
        raise TypeError("linear needs bf16 activations and weights")
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("linear needs 2-D tensors with unit inner stride")
    rows, k = x.shape
    w_ptr, w_s0, n = _weight_arg(weight, k)
    _lib.require_device(x, weight)
    need = linear_workspace_bytes(rows, n, k, epilogue)
    out = torch.empty((rows, out_width), dtype=x.dtype, device=x.device) if out is None else out
    if out.shape != (rows, out_width) or out.stride(1) != 1 or out.dtype != torch.bfloat16:
        raise ValueError(f"out must be bf16 [{rows}, {out_width}] with unit inner stride")
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    _lib.call(
        "nq_linear", x.data_ptr(), x.stride(0), w_ptr, w_s0, rows, n, k, int(epilogue),
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
    if x.dtype != torch.bfloat16 or x.stride(1) != 1:
        raise TypeError("linear needs bf16 tensors with unit inner stride")
    w_ptr, w_s0, n = _weight_arg(weight, k)
    splits = int(_lib.load().nq_linear_splits(rows, n, k))
    if splits < 1:
        raise TypeError(f"no HIP projection for rows={rows}, out={n}, in={k}")
    need = linear_workspace_bytes(rows, n, k, _lib.NQ_EPI_PARTIALS)
    if workspace.numel() * workspace.element_size() < need:
        raise ValueError("workspace too small for the projection partials")
    _lib.require_device(x, workspace)
    _lib.call("nq_linear", x.data_ptr(), x.stride(0), w_ptr, w_s0, rows, n, k,
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


FP8 = torch.float8_e4m3fn


def quantize_fp8_weight_blocks(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize a row-major bf16 gate/up matrix into 128 x 128 FP8 blocks (model/layers.py:10-25):
    returns (e4m3fn codes with the weight's shape, fp32 power-of-two scales [rows/128, cols/128])."""

    if weight.ndim != 2 or not weight.is_contiguous():
        raise ValueError("FP8 block quantization requires a contiguous matrix")
    rows, columns = weight.shape
    if rows % 128 or columns % 128:
        raise ValueError(
            f"FP8 block quantization requires dimensions divisible by 128, got {tuple(weight.shape)}"
        )
    _check(weight, "weight")
    q = torch.empty((rows, columns), dtype=FP8, device=weight.device)
    scales = torch.empty((rows // 128, columns // 128), dtype=torch.float32, device=weight.device)
    _lib.call("nq_quantize_fp8_blocks", weight.data_ptr(), weight.stride(0), rows, columns, q.data_ptr(),
              q.stride(0), scales.data_ptr(), scales.stride(0), _lib.stream(weight.device))
    return q, scales


def _fp8_out(rows: int, width: int, device, q: torch.Tensor | None, scales: torch.Tensor | None):
    q = torch.empty((rows, width), dtype=FP8, device=device) if q is None else q
    scales = torch.empty((rows, width // 128), dtype=torch.float32, device=device) if scales is None else scales
    if q.dtype != FP8 or q.shape != (rows, width) or q.stride(1) != 1:
        raise ValueError(f"FP8 codes must be float8_e4m3fn [{rows}, {width}] with unit inner stride")
    if scales.dtype != torch.float32 or scales.shape != (rows, width // 128) or scales.stride(1) != 1:
        raise ValueError(f"FP8 scales must be fp32 [{rows}, {width // 128}]")
    _lib.require_device(q, scales)
    return q, scales


def quantize_fp8_rows(x: torch.Tensor, q: torch.Tensor | None = None, scales: torch.Tensor | None = None):
    """bf16 [rows, K] -> (e4m3fn codes, fp32 scales [rows, K/128]): scale = max|x| / 448 per 128 columns."""

    if x.dtype != torch.bfloat16 or x.dim() != 2 or x.stride(1) != 1:
        raise TypeError("row quantization needs bf16 [rows, K] with unit inner stride")
    rows, k = x.shape
    if k % 128:
        raise ValueError("row quantization needs a multiple of 128 columns")
    _lib.require_device(x)
    q, scales = _fp8_out(rows, k, x.device, q, scales)
    _lib.call("nq_quantize_fp8_rows", x.data_ptr(), x.stride(0), rows, k, q.data_ptr(), q.stride(0),
              scales.data_ptr(), scales.stride(0), _lib.stream(x.device))
    return q, scales


def add_rmsnorm_fp8(hidden: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float,
                    q: torch.Tensor | None = None, scales: torch.Tensor | None = None):
    """residual += hidden; the rmsnorm of residual is returned quantized as (codes, scales)."""

    _check(hidden, "hidden_states")
    _check(residual, "residual")
    _check(weight, "norm weight")
    if hidden.shape != residual.shape or hidden.dim() != 2:
        raise ValueError("fused add-RMSNorm needs 2-D tensors of one shape")
    rows, width = hidden.shape
    if weight.shape != (width,):
        raise ValueError("norm weight must match the hidden width")
    q, scales = _fp8_out(rows, width, hidden.device, q, scales)
    _lib.call("nq_add_rmsnorm_fp8", hidden.data_ptr(), residual.data_ptr(), weight.data_ptr(), rows, width,
              float(eps), q.data_ptr(), q.stride(0), scales.data_ptr(), scales.stride(0), _lib.stream(hidden.device))
    return q, scales


def linear_add_rmsnorm_fp8(x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor, norm_weight: torch.Tensor,
                           eps: float, q: torch.Tensor, scales: torch.Tensor, workspace: torch.Tensor | None = None):
    """linear_add_rmsnorm with the normalised output stored quantized in (q, scales)."""

    for t, name in ((residual, "residual"), (norm_weight, "norm weight")):
        _check(t, name)
    if x.dtype != torch.bfloat16 or x.stride(1) != 1:
        raise TypeError("linear needs bf16 tensors with unit inner stride")
    rows, k = x.shape
    w_ptr, w_s0, n = _weight_arg(weight, k)
    if residual.shape != (rows, n) or norm_weight.shape != (n,):
        raise ValueError("residual / norm weight must match the projection output")
    q, scales = _fp8_out(rows, n, x.device, q, scales)
    need = linear_workspace_bytes(rows, n, k, _lib.NQ_EPI_ADD_RMSNORM)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    _lib.require_device(x, workspace)
    _lib.call("nq_linear_add_rmsnorm_fp8", x.data_ptr(), x.stride(0), w_ptr, w_s0, rows, n,
              k, residual.data_ptr(), norm_weight.data_ptr(), float(eps), q.data_ptr(), q.stride(0),
              scales.data_ptr(), scales.stride(0), workspace.data_ptr(), workspace.numel() * workspace.element_size(),
              _lib.stream(x.device))
    return q, scales


def linear_fp8_workspace_bytes(rows: int, out_features: int, in_features: int,
                               epilogue: int = _lib.NQ_EPI_NONE) -> int:
    """fp32 split-K scratch of the FP8 projection for up to 128 rows (0 when none)."""

    n = int(_lib.load().nq_linear_fp8_workspace_bytes(int(min(rows, 128)), int(out_features), int(in_features),
                                                      int(epilogue)))
    if n < 0:
        raise TypeError(f"no FP8 projection for rows={rows}, out={out_features}, in={in_features}")
    return n


def linear_fp8(q: torch.Tensor, scales: torch.Tensor, weight_q: torch.Tensor, weight_scales: torch.Tensor,
               epilogue: int = _lib.NQ_EPI_NONE, out: torch.Tensor | None = None,
               workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Block-scaled FP8 projection y = dequant(q) @ dequant(weight_q).T in fp32, bf16 out
    (NQ_EPI_NONE) or silu(y[:, :N/2]) * y[:, N/2:] (NQ_EPI_SILU_MUL).  Rows beyond 128 run in
    128-row pieces."""

    if q.dtype != FP8 or weight_q.dtype != FP8:
        raise TypeError("FP8 projection needs float8_e4m3fn codes")
    if epilogue not in (_lib.NQ_EPI_NONE, _lib.NQ_EPI_SILU_MUL):
        raise ValueError("FP8 projection epilogue must be NONE or SILU_MUL")
    rows, k = q.shape
    n = weight_q.shape[0]
    if weight_q.shape[1] != k or scales.shape != (rows, k // 128) or weight_scales.shape != (n // 128, k // 128):
        raise ValueError("FP8 codes and scales do not match")
    for t in (scales, weight_scales):
        if t.dtype != torch.float32 or t.stride(1) != 1:
            raise TypeError("FP8 scales must be fp32 with unit inner stride")
    _lib.require_device(q, scales, weight_q, weight_scales)
    width = n // 2 if epilogue == _lib.NQ_EPI_SILU_MUL else n
    out = torch.empty((rows, width), dtype=torch.bfloat16, device=q.device) if out is None else out
    if out.shape != (rows, width) or out.stride(1) != 1 or out.dtype != torch.bfloat16:
        raise ValueError(f"out must be bf16 [{rows}, {width}] with unit inner stride")
    need = linear_fp8_workspace_bytes(rows, n, k, epilogue)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    for r0 in range(0, rows, 128):
        m = min(128, rows - r0)
        _lib.call("nq_linear_fp8", q[r0:].data_ptr(), q.stride(0), scales[r0:].data_ptr(), scales.stride(0),
                  weight_q.data_ptr(), weight_q.stride(0), weight_scales.data_ptr(), weight_scales.stride(0), m, n, k,
                  int(epilogue), out[r0:].data_ptr(), out.stride(0), _lib.ptr(workspace) if need else None,
                  workspace.numel() * workspace.element_size() if need else 0, _lib.stream(q.device))
    return out


def pack_fp8_swiglu(weight_q: torch.Tensor) -> torch.Tensor:
    """Interleave the rows of FP8 [gate; up] codes [2I, K] for linear_fp8_swiglu (the block
    scales stay those of the original layout)."""

    if weight_q.dtype != FP8 or weight_q.dim() != 2 or weight_q.shape[0] % 16 or weight_q.stride(1) != 1:
        raise ValueError("FP8 gate/up codes [2I, K] with I % 8 == 0 expected")
    _lib.require_device(weight_q)
    packed = torch.empty_like(weight_q)
    _lib.call("nq_fp8_pack_swiglu", weight_q.data_ptr(), weight_q.stride(0), weight_q.shape[0] // 2,
              weight_q.shape[1], packed.data_ptr(), packed.stride(0), _lib.stream(weight_q.device))
    return packed


def pack_swiglu(weight: torch.Tensor) -> torch.Tensor:
    """Interleave the rows of a bf16 [gate; up] matrix [2I, K] for linear_swiglu (the row permutation
    of pack_fp8_swiglu, applied to the bf16 rows as bytes)."""

    if weight.dtype != torch.bfloat16 or weight.dim() != 2 or weight.shape[0] % 16 or weight.stride(1) != 1:
        raise ValueError("bf16 gate/up rows [2I, K] with I % 8 == 0 expected")
    _lib.require_device(weight)
    packed = torch.empty_like(weight)
    _lib.call("nq_fp8_pack_swiglu", weight.data_ptr(), weight.stride(0) * 2, weight.shape[0] // 2,
              weight.shape[1] * 2, packed.data_ptr(), packed.stride(0) * 2, _lib.stream(weight.device))
    return packed


def linear_swiglu(x: torch.Tensor, packed: torch.Tensor, out: torch.Tensor, weight: torch.Tensor | None = None,
                  workspace: torch.Tensor | None = None) -> torch.Tensor:
    """silu(gate) * up of the bf16 gate/up projection in one kernel where the shape allows it (K = 1024;
    the bits of linear_silu_mul at 128 rows, where both sum K in the same four slices); else
    linear_silu_mul on the unpacked ``weight``."""

    rows, k = x.shape
    inter = packed.shape[0] // 2
    if out.shape != (rows, inter) or out.dtype != torch.bfloat16 or out.stride(1) != 1:
        raise ValueError(f"out must be bf16 [{rows}, {inter}] with unit inner stride")
    if x.dtype != torch.bfloat16 or packed.dtype != torch.bfloat16 or packed.shape[1] != k or x.stride(1) != 1:
        raise TypeError("bf16 activations and packed bf16 gate/up rows expected")
    _lib.require_device(x, packed, out)
    rc = _lib.load().nq_linear_swiglu(x.data_ptr(), x.stride(0), rows, packed.data_ptr(), packed.stride(0), inter,
                                      k, out.data_ptr(), out.stride(0), _lib.stream(x.device))
    if rc == _lib.NQ_ERR_UNSUPPORTED:
        if weight is None:
            raise TypeError("shape not covered by the fused SwiGLU and no unpacked weight given")
        return linear_silu_mul(x, weight, out=out, workspace=workspace)
    _lib.check(rc, "nq_linear_swiglu")
    return out


def linear_fp8_swiglu(q: torch.Tensor, scales: torch.Tensor, packed: torch.Tensor, weight_scales: torch.Tensor,
                      out: torch.Tensor, weight_q: torch.Tensor | None = None,
                      workspace: torch.Tensor | None = None) -> torch.Tensor:
    """silu(gate) * up of the FP8 gate/up projection in one kernel where the shape allows it
    (<= 64 rows, K = 2048), else through linear_fp8 on the unpacked codes ``weight_q``."""

    rows, k = q.shape
    inter = packed.shape[0] // 2
    if out.shape != (rows, inter) or out.dtype != torch.bfloat16 or out.stride(1) != 1:
        raise ValueError(f"out must be bf16 [{rows}, {inter}] with unit inner stride")
    if q.dtype != FP8 or packed.dtype != FP8 or packed.shape[1] != k:
        raise TypeError("FP8 codes expected")
    if scales.shape != (rows, k // 128) or weight_scales.shape != (2 * inter // 128, k // 128):
        raise ValueError("FP8 scales do not match")
    _lib.require_device(q, scales, packed, weight_scales, out)
    rc = _lib.load().nq_linear_fp8_swiglu(q.data_ptr(), q.stride(0), scales.data_ptr(), scales.stride(0), rows,
                                          packed.data_ptr(), packed.stride(0), weight_scales.data_ptr(),
                                          weight_scales.stride(0), inter, k, out.data_ptr(), out.stride(0),
                                          _lib.stream(q.device))
    if rc == _lib.NQ_ERR_UNSUPPORTED:
        if weight_q is None:
            raise TypeError("shape not covered by the fused FP8 SwiGLU and no unpacked codes given")
        return linear_fp8(q, scales, weight_q, weight_scales, epilogue=_lib.NQ_EPI_SILU_MUL, out=out,
                          workspace=workspace)
    _lib.check(rc, "nq_linear_fp8_swiglu")
    return out


__all__ = [
    "linear_swiglu",
    "pack_swiglu",
    "FP8",
    "embed_add_rmsnorm",
    "gather_sum_rows",
    "linear_rows",
    "tgemm",
    "tgemm_add_rmsnorm_fp8",
    "tgemm_fp8_swiglu",
    "tgemm_partials",
    "tgemm_workspace_bytes",
    "prefill_embed_rmsnorm",
    "linear_fp8_swiglu",
    "pack_fp8_swiglu",
    "add_rmsnorm_fp8",
    "linear",
    "linear_add_rmsnorm",
    "linear_add_rmsnorm_fp8",
    "linear_fp8",
    "linear_fp8_workspace_bytes",
    "linear_partials",
    "linear_silu_mul",
    "linear_workspace_bytes",
    "quantize_fp8_rows",
    "quantize_fp8_weight_blocks",
    "add_rmsnorm",
    "qwen3_tts_add_rmsnorm",
    "qwen3_tts_rmsnorm",
    "qwen3_tts_silu_and_mul",
    "rmsnorm",
    "silu_mul",
]
