"""ctypes binding of ``libnq_hip.so`` (the C ABI of include/nq_abi.h).

The library is loaded after ``torch`` so that it binds to the HIP runtime
torch already mapped (both carry the soname ``libamdhip64.so.7``), which makes
torch's streams and device pointers valid inside the library.  There is no
fallback: a missing library raises ``RuntimeError`` on first use.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

from .errors import KVAllocationError

LIBRARY_PATH = Path(__file__).resolve().parent / "libnq_hip.so"

NQ_OK = 0
NQ_ERR_INVALID_ARGUMENT = -1
NQ_ERR_UNSUPPORTED = -2
NQ_ERR_LAUNCH = -3
NQ_ERR_CAPACITY = -4
NQ_ERR_STATE = -5
NQ_F32 = 0
NQ_BF16 = 1
NQ_EPI_NONE = 0
NQ_EPI_ADD_RMSNORM = 1
NQ_EPI_SILU_MUL = 2
NQ_EPI_PARTIALS = 3
NQ_MATMUL_HIGHEST = 0
NQ_MATMUL_HIGH = 1
NQ_ATTN_DECODE = 1
NQ_ATTN_PREFILL = 2
NQ_ATTN_BESIDE_PREFILL = 4
NQ_NOALLOC_SCRATCH_BYTES = 32 << 20
NQ_REPORT_HEAD = 8

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float

# name -> argument types (restype int unless listed in _RESTYPES)
_SIGNATURES: dict[str, list] = {
    "nq_abi_version": [],
    "nq_status_string": [_I],
    "nq_plan_ragged": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _L, _P, _I, _P, _P, _I, _P, _P, _P, _L,
                       _P, _P, _P, _P, _P, _I, _P],
    "nq_free_list_merge": [_P, _I, _P, _I, _P, _P, _P],
    "nq_step_report": [_P, _P, _P, _P, _P, _I, _L, _L, _P, _P],
    "nq_attention_workspace_bytes": [_I, _I, _I, _I, _I, _I],
    "nq_attention_plan": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _L, _P],
    "nq_attention_plan_parts": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P, _L, _P],
    "nq_paged_attention": [_P, _L, _L, _P, _L, _L, _L, _L, _I, _P, _I, _I, _I, _I, _F, _P, _L, _L,
                           _I, _I, _I, _P, _L, _P, _P],
    "nq_paged_attention_noalloc": [_P, _P, _P, _P, _I, _P, _L, _L, _P, _L, _L, _L, _L, _I, _I, _I, _I, _I, _F,
                                   _P, _L, _L, _I, _I, _I, _P, _P],
    "nq_cp_short_attention": [_P, _L, _L, _P, _L, _L, _L, _L, _I, _I, _I, _I, _I, _F, _P, _L, _L, _P],
    "nq_cp_rope_short_attention": [_P, _I, _I, _P, _P, _P, _L, _F, _F, _I, _P, _L, _L, _P, _L, _L, _L, _L, _I, _I, _I, _I,
                                   _F, _P, _L, _L, _P],
    "nq_qk_norm_rope_kv_write": [_P, _L, _L, _P, _L, _L, _P, _L, _L, _P, _P, _P, _L, _I, _I, _I, _I, _F,
                                 _F, _I, _P, _L, _L, _L, _L, _P, _P, _I, _P],
    "nq_qkv_partials_norm_rope_kv_write": [_P, _I, _I, _P, _L, _L, _P, _L, _L, _P, _P, _P, _L, _I, _I, _I, _F, _F,
                                           _I, _P, _L, _L, _L, _L, _P, _P, _I, _P],
    "nq_paged_decode_rope_attention": [_P, _I, _I, _P, _P, _P, _F, _F, _I, _P, _L, _L, _L, _L, _I, _P, _P, _P, _I, _I,
                                       _I, _I, _F, _P, _L, _L, _I, _I, _P, _L, _P, _P],
    "nq_sample": [_P, _I, _L, _I, _I, _P, _P, _P, _P, _P, _L, _P, _I, _I, _P, _I, _P, _P],
    "nq_sample_counter": [_P, _I, _L, _I, _I, _P, _P, _P, _P, _P, _L, _P, _L, _P, _L, _I, _I, _P, _I, _P, _P],
    "nq_sample_counter_planes": [_P, _I, _L, _I, _I, _P, _P, _P, _P, _P, _L, _P, _L, _P, _L, _I, _I, _P, _I, _P, _L,
                                 _P, _P],
    "nq_uniforms_from_counter": [_P, _L, _P, _L, _I, _P, _P],
    "nq_add_rmsnorm": [_P, _P, _P, _I, _I, _F, _P],
    "nq_embed_add_rmsnorm": [_P, _P, _L, _L, _P, _L, _P, _I, _I, _F, _P, _P, _P, _P],
    "nq_prefill_embed_rmsnorm": [_P, _P, _L, _L, _P, _P, _L, _L, _P, _P, _I, _I, _F, _P, _P, _P, _P],
    "nq_gather_sum_rows": [_P, _P, _L, _L, _P, _L, _L, _P, _L, _L, _L, _I, _I, _I, _P, _L, _P, _P],
    "nq_rmsnorm": [_P, _P, _P, _I, _I, _F, _P],
    "nq_silu_mul": [_P, _P, _I, _I, _P],
    "nq_linear_splits": [_I, _I, _I],
    "nq_linear_workspace_bytes": [_I, _I, _I, _I],
    "nq_linear": [_P, _L, _P, _L, _I, _I, _I, _I, _P, _P, _L, _P, _P, _F, _P, _L, _P],
    "nq_quantize_fp8_blocks": [_P, _L, _I, _I, _P, _L, _P, _L, _P],
    "nq_quantize_fp8_rows": [_P, _L, _I, _I, _P, _L, _P, _L, _P],
    "nq_add_rmsnorm_fp8": [_P, _P, _P, _I, _I, _F, _P, _L, _P, _L, _P],
    "nq_linear_add_rmsnorm_fp8": [_P, _L, _P, _L, _I, _I, _I, _P, _P, _F, _P, _L, _P, _L, _P, _L, _P],
    "nq_linear_fp8_splits": [_I, _I, _I],
    "nq_linear_fp8_workspace_bytes": [_I, _I, _I, _I],
    "nq_linear_fp8": [_P, _L, _P, _L, _P, _L, _P, _L, _I, _I, _I, _I, _P, _L, _P, _L, _P],
    "nq_fp8_pack_swiglu": [_P, _L, _I, _I, _P, _L, _P],
    "nq_linear_swiglu": [_P, _L, _I, _P, _L, _I, _I, _P, _L, _P],
    "nq_linear_fp8_swiglu": [_P, _L, _P, _L, _I, _P, _L, _P, _L, _I, _I, _P, _L, _P],
    "nq_sgemm": [_P, _L, _P, _P, _L, _I, _I, _I, _P, _I, _P, _L, _P, _P, _L, _I, _P],
    "nq_row_norm": [_P, _L, _I, _I, _P, _P, _F, _P, _L, _P],
    "nq_codec_last_rows": [_P, _I, _I, _P, _P],
    "nq_tgemm_splits": [_I, _I, _I],
    "nq_tgemm_workspace_bytes": [_I, _I, _I, _I],
    "nq_tgemm": [_P, _L, _P, _L, _I, _I, _I, _I, _P, _L, _P, _P, _F, _P, _L, _P],
    "nq_tgemm_add_rmsnorm_fp8": [_P, _L, _P, _L, _I, _I, _I, _P, _P, _F, _P, _L, _P, _L, _P, _L, _P],
    "nq_tgemm_fp8_swiglu": [_P, _L, _P, _L, _I, _P, _L, _P, _L, _I, _I, _P, _L, _P],
    "nq_codec_embed_sum": [_P, _I, _I, _P, _I, _I, _P, _P, _P],
    "nq_codec_causal_conv": [_P, _L, _L, _P, _I, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _L, _P, _L, _P],
    "nq_codec_residual_unit": [_P, _L, _L, _P, _I, _I, _P, _P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L,
                               _I, _P],
    "nq_codec_causal_transconv": [_P, _L, _L, _P, _I, _I, _I, _P, _P, _P, _P, _I, _I, _P, _P, _P, _L, _P],
    "nq_codec_window_attention": [_P, _P, _P, _L, _I, _I, _I, _P, _P, _F, _F, _P, _I, _P, _P, _P, _P, _P, _L, _I,
                                  _I, _P, _L, _P],
    "nq_codec_advance": [_P, _I, _P, _P, _P, _I, _P],
    "nq_codec_pcm16": [_P, _L, _P, _P, _P],
    "nq_codec_im2col": [_P, _L, _L, _P, _I, _I, _P, _P, _I, _I, _I, _I, _P, _P, _P, _L, _P],
    "nq_codec_history_update": [_P, _L, _P, _I, _I, _P, _P, _I, _I, _P, _P, _P],
    "nq_codec_transconv_overlap": [_P, _I, _I, _I, _P, _P, _P, _I, _P, _L, _P],
}
_RESTYPES = {
    "nq_status_string": ctypes.c_char_p,
    "nq_attention_workspace_bytes": ctypes.c_int64,
    "nq_linear_workspace_bytes": ctypes.c_int64,
    "nq_linear_fp8_workspace_bytes": ctypes.c_int64,
    "nq_tgemm_workspace_bytes": ctypes.c_int64,
}

EXPORTED = tuple(_SIGNATURES)

_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load the library once; raise if it was never built."""

    global _lib
    if _lib is None:
        if not LIBRARY_PATH.exists():
            raise RuntimeError(
                f"HIP library {LIBRARY_PATH} is missing; build it with __graft_entry__.build() "
                "(there is no CPU fallback)"
            )
        lib = ctypes.CDLL(str(LIBRARY_PATH))
        for name, args in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        _lib = lib
    return _lib


def status_string(status: int) -> str:
    return load().nq_status_string(int(status)).decode()


def check(status: int, what: str) -> None:
    """Map an NQ status code to the reference's exception types."""

    if status == NQ_OK:
        return
    message = f"{what}: {status_string(status)} (status {status})"
    if status == NQ_ERR_INVALID_ARGUMENT:
        raise ValueError(message)
    if status == NQ_ERR_UNSUPPORTED:
        raise TypeError(message)
    if status == NQ_ERR_CAPACITY:
        raise KVAllocationError(message)
    raise RuntimeError(message)


_functions: dict[str, object] = {}


def call(name: str, *args) -> None:
    fn = _functions.get(name)
    if fn is None:
        fn = _functions[name] = getattr(load(), name)
    status = fn(*args)
    if status != NQ_OK:
        check(status, name)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream(device: torch.device | None = None) -> int:
    """The hipStream_t of torch's current stream on ``device`` (the current device when it names none):
    the handle ``torch.cuda.current_stream(device).cuda_stream`` gives, without building the Stream
    object (this runs before every launch)."""

    index = device.index if device is not None and device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)


def require_device(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError("HIP kernels need tensors on the GPU (there is no CPU path)")
