"""FP8 block quantization and the block-scaled FP8 GEMM of the talker's gate/up
projection (test infrastructure only).

Weights: model/layers.py:10-25 (``quantize_fp8_weight_blocks``) -- 128 x 128
blocks of the row-major [N, K] matrix, block maximum |w| clamped to >= 1e-4,
scale = 2 ** ceil(log2(max / 448)) (a power of two), codes = e4m3fn(w /
scale) with round-to-nearest-even.  The ceil(log2(.)) is taken exactly here
(the smallest power of two >= max / 448); torch's fp32 log2 can only differ
when max / 448 lies within a few ulps above a power of two.

GEMM: model/layers.py:241-262 hands the bf16 activations and the FP8 weight
blocks to flashinfer 0.6.16.post2 ``fp8_blockscale_gemm_sm90`` (pinned at
pyproject.toml:26, not vendored).  Its published algorithm (the DeepGEMM /
DeepSeek-V3 fine-grained FP8 scheme) quantizes the activations per token and
128 columns -- scale = max |x| / 448, codes = e4m3fn(x / scale) -- and
accumulates in fp32 with both scales applied per 128-wide K block:
y[m, n] = sum_kb s_x[m, kb] * s_w[n / 128, kb] * sum_{k in kb} q_x[m, k] q_w[n, k],
then rounds to bf16.  The activation-side details (no clamp, x / scale rather
than x * (448 / max)) follow the DeepSeek-V3 reference ``act_quant``; the
exact flashinfer kernel is not available here, so that half of the parity is
pinned only by these published rules.

e4m3fn (OCP FP8): 1 sign bit, 4 exponent bits with bias 7, 3 mantissa bits,
no infinities, 0x7F / 0xFF are NaN, largest finite 448, subnormals down to
2 ** -9.
"""

from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0
BLOCK = 128


def e4m3_from_f32(x: np.ndarray) -> np.ndarray:
    """fp32 values -> e4m3fn codes (uint8), round to nearest even, |x| saturated at 448.

    Values in (448, 464) round to 448 as round-to-nearest-even would; values
    at or beyond 464 (which no quantizer here produces) saturate to 448.
    """

    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.int64)
    sign = ((u >> 31) & 1).astype(np.int64) << 7
    a = np.abs(x).astype(np.float32)
    au = a.view(np.uint32).astype(np.int64)
    exp = ((au >> 23) & 0xFF) - 127
    # normal e4m3 range (exponent >= -6): keep 3 mantissa bits with round-to-nearest-even
    mant = au & 0x7FFFFF
    rounded = (mant + 0x7FFFF + ((mant >> 20) & 1)) >> 20  # 0..8 (8 carries into the exponent)
    normal = ((exp + 7) << 3) + rounded
    # subnormal e4m3 (exponent < -6): multiples of 2 ** -9, round-to-nearest-even
    sub = np.rint(a.astype(np.float64) * 512.0).astype(np.int64)
    code = np.where(exp >= -6, normal, sub)
    code = np.minimum(code, 0x7E)
    return (code | sign).astype(np.uint8)


def e4m3_to_f32(code: np.ndarray) -> np.ndarray:
    """e4m3fn codes -> fp32 values (exact; 0x7F / 0xFF give NaN)."""

    c = np.asarray(code, dtype=np.uint8).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    val = np.where((c & 0x7F) == 0x7F, np.nan, val)
    return (sign * val).astype(np.float32)


def _pow2_ceil(v: np.ndarray) -> np.ndarray:
    """Smallest power of two >= v for positive normal fp32 v (exact)."""

    v = np.asarray(v, dtype=np.float32)
    u = v.view(np.uint32).astype(np.int64)
    exp = ((u >> 23) & 0xFF) - 127
    exact = (u & 0x7FFFFF) == 0
    e = np.where(exact, exp, exp + 1)
    return np.exp2(e.astype(np.float64)).astype(np.float32)


def quantize_weight_blocks(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """[N, K] weights (bf16 values as fp32) -> (e4m3fn codes [N, K], fp32 scales [N/128, K/128])."""

    w = np.asarray(w, dtype=np.float32)
    if w.ndim != 2:
        raise ValueError("FP8 block quantization requires a matrix")
    rows, cols = w.shape
    if rows % BLOCK or cols % BLOCK:
        raise ValueError(f"FP8 block quantization requires dimensions divisible by 128, got {w.shape}")
    blocks = w.reshape(rows // BLOCK, BLOCK, cols // BLOCK, BLOCK)
    amax = np.maximum(np.abs(blocks).max(axis=(1, 3)), np.float32(1e-4)).astype(np.float32)
    scales = _pow2_ceil((amax / np.float32(E4M3_MAX)).astype(np.float32))
    q = e4m3_from_f32((blocks / scales[:, None, :, None]).astype(np.float32))
    return q.reshape(rows, cols), scales


def quantize_rows(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """[M, K] activations (fp32 values) -> (e4m3fn codes [M, K], fp32 scales [M, K/128]).

    scale = max |x| / 448 over each 128-column group (1 for an all-zero group),
    codes = e4m3fn(x / scale) in fp32.
    """

    x = np.asarray(x, dtype=np.float32)
    m, k = x.shape
    if k % BLOCK:
        raise ValueError("row quantization requires a multiple of 128 columns")
    g = x.reshape(m, k // BLOCK, BLOCK)
    amax = np.abs(g).max(axis=2)
    scales = np.where(amax > 0, (amax / np.float32(E4M3_MAX)).astype(np.float32), np.float32(1.0)).astype(np.float32)
    q = e4m3_from_f32((g / scales[:, :, None]).astype(np.float32))
    return q.reshape(m, k), scales


def blockscale_gemm(xq: np.ndarray, sx: np.ndarray, wq: np.ndarray, sw: np.ndarray) -> np.ndarray:
    """y[m, n] = sum_kb sx[m, kb] sw[n/128, kb] (q_x[m, kb] . q_w[n, kb]) in float64 (unrounded)."""

    xv = e4m3_to_f32(xq).astype(np.float64)
    wv = e4m3_to_f32(wq).astype(np.float64)
    m, k = xv.shape
    n = wv.shape[0]
    nkb = k // BLOCK
    y = np.zeros((m, n), dtype=np.float64)
    for kb in range(nkb):
        sl = slice(kb * BLOCK, (kb + 1) * BLOCK)
        dot = xv[:, sl] @ wv[:, sl].T
        scale = sx[:, kb].astype(np.float64)[:, None] * np.repeat(sw[:, kb].astype(np.float64), BLOCK)[None, :n]
        y += dot * scale
    return y


def dequantize_weight_blocks(wq: np.ndarray, sw: np.ndarray) -> np.ndarray:
    """Codes and block scales -> fp32 weights (exact: e4m3 values times powers of two)."""

    v = e4m3_to_f32(wq)
    return (v * np.repeat(np.repeat(sw, BLOCK, axis=0), BLOCK, axis=1)).astype(np.float32)
