"""The FP8 oracle pinned against torch's e4m3fn conversion, the reference's
known-answer test for the block quantizer (tests/model_optimization/
test_optimizations.py:35-45) and closed forms of the block-scaled GEMM."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import bf16
from oracle import fp8


def _torch_codes(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_encoder_matches_torch_on_every_bf16_value():
    x = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    x = x[np.isfinite(x) & (np.abs(x) < 464)]
    assert np.array_equal(fp8.e4m3_from_f32(x), _torch_codes(x))


def test_encoder_matches_torch_on_midpoints_and_random_values():
    vals = fp8.e4m3_to_f32(np.arange(256, dtype=np.uint8))
    pos = np.sort(vals[np.isfinite(vals) & (vals >= 0)])
    mids = ((pos[1:].astype(np.float64) + pos[:-1]) / 2).astype(np.float32)
    rng = np.random.default_rng(5)
    rand = (rng.standard_normal(200_000) * rng.choice([1e-4, 1e-2, 1.0, 30.0, 200.0], 200_000)).astype(np.float32)
    y = np.concatenate([mids, -mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e3)), rand])
    y = y[np.abs(y) < 464]
    assert np.array_equal(fp8.e4m3_from_f32(y), _torch_codes(y))


def test_decoder_matches_torch_on_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).float().numpy()
    got = fp8.e4m3_to_f32(codes)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin], want[fin])
    assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9 and got[0x08] == 2.0 ** -6


def test_weight_blocks_reference_known_answer():
    with pytest.raises(ValueError, match="divisible by 128"):
        fp8.quantize_weight_blocks(np.ones((128, 64), np.float32))
    w = np.linspace(-2, 2, 128 * 128, dtype=np.float32).reshape(128, 128)
    q, s = fp8.quantize_weight_blocks(w)
    assert q.shape == w.shape and q.dtype == np.uint8
    assert s.shape == (1, 1)
    # max |w| = 2: 2 / 448 lies in (2^-8, 2^-7], so the scale is 2^-7 and w = 2 maps to 256 exactly
    assert s[0, 0] == 2.0 ** -7
    assert np.all(np.isfinite(fp8.e4m3_to_f32(q)))
    assert fp8.e4m3_to_f32(q[-1:, -1:])[0, 0] == 256.0


def test_weight_block_scales_are_tight_powers_of_two():
    rng = np.random.default_rng(1)
    w = bf16.round_f32((rng.standard_normal((256, 384)) * rng.choice([1e-3, 0.02, 3.0], (256, 1))).astype(np.float32))
    w[:128, :128] = 0.0  # clamp case: max 1e-4
    q, s = fp8.quantize_weight_blocks(w)
    assert s.shape == (2, 3)
    mant, _ = np.frexp(s)
    assert np.all(mant == 0.5), "scales are powers of two"
    amax = np.maximum(np.abs(w.reshape(2, 128, 3, 128)).max(axis=(1, 3)), 1e-4)
    ratio = amax / s
    assert np.all(ratio <= 448.0) and np.all(ratio > 224.0)
    assert np.all(q[:128, :128] == 0)
    # dequantization error is within half an e4m3 step (relative 2^-4 for normal values)
    deq = fp8.dequantize_weight_blocks(q, s)
    step = np.repeat(np.repeat(s, 128, 0), 128, 1) * 2.0 ** -9  # subnormal spacing in real units
    tol = np.maximum(np.abs(w) * 2.0 ** -4, step / 2)
    assert np.all(np.abs(deq - w) <= tol)


def test_row_quantization_maps_group_maximum_to_448():
    rng = np.random.default_rng(2)
    x = bf16.round_f32(rng.standard_normal((7, 256)).astype(np.float32))
    x[3, 128:] = 0.0
    q, s = fp8.quantize_rows(x)
    assert s.shape == (7, 2)
    assert s[3, 1] == 1.0 and np.all(q[3, 128:] == 0)
    v = fp8.e4m3_to_f32(q).reshape(7, 2, 128)
    g = x.reshape(7, 2, 128)
    idx = np.abs(g).argmax(axis=2)
    peak = np.take_along_axis(v, idx[..., None], axis=2)[..., 0]
    live = np.abs(g).max(axis=2) > 0
    assert np.all(np.abs(peak[live]) == 448.0)
    deq = v * s[..., None]
    assert np.all(np.abs(deq - g) <= np.maximum(np.abs(g) * 2.0 ** -4, s[..., None] * 2.0 ** -10) + 1e-12)


def test_blockscale_gemm_exact_on_integer_codes():
    rng = np.random.default_rng(3)
    m, n, k = 5, 256, 384
    # integer-valued codes (|v| <= 8 are exact in e4m3) and power-of-two scales: the result is exact
    xv = rng.integers(-8, 9, (m, k)).astype(np.float32)
    wv = rng.integers(-8, 9, (n, k)).astype(np.float32)
    xq, wq = fp8.e4m3_from_f32(xv), fp8.e4m3_from_f32(wv)
    sx = np.exp2(rng.integers(-3, 4, (m, k // 128))).astype(np.float32)
    sw = np.exp2(rng.integers(-3, 4, (n // 128, k // 128))).astype(np.float32)
    want = np.zeros((m, n), dtype=np.float64)
    for i in range(m):
        for j in range(n):
            for kk in range(k):
                want[i, j] += float(xv[i, kk]) * float(wv[j, kk]) * float(sx[i, kk // 128]) * float(sw[j // 128, kk // 128])
    assert np.array_equal(fp8.blockscale_gemm(xq, sx, wq, sw), want)


def test_blockscale_gemm_equals_dequantized_matmul():
    rng = np.random.default_rng(4)
    x = bf16.round_f32(rng.standard_normal((9, 512)).astype(np.float32))
    w = bf16.round_f32((rng.standard_normal((384, 512)) * 0.02).astype(np.float32))
    xq, sx = fp8.quantize_rows(x)
    wq, sw = fp8.quantize_weight_blocks(w)
    # activation scales are not powers of two: dequantize in float64
    xd = (fp8.e4m3_to_f32(xq).astype(np.float64).reshape(9, 4, 128) * sx.astype(np.float64)[..., None]).reshape(9, 512)
    wd = fp8.dequantize_weight_blocks(wq, sw).astype(np.float64)
    y = fp8.blockscale_gemm(xq, sx, wq, sw)
    assert np.allclose(y, xd @ wd.T, rtol=1e-12, atol=1e-12)
    # and the quantized product tracks the bf16 product to FP8 accuracy
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.abs(y - exact).max() <= 0.06 * np.abs(exact).max()
