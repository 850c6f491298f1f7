"""FP8 gate/up path on the GPU vs the FP8 oracle: the block and row quantizers
bit-exact, the block-scaled GEMM exact on integer-valued codes (which pins the
MFMA operand layout and the e4m3 format) and within fp32-accumulation
tolerance otherwise, and the fused add-RMSNorm quantizer bit-exact against
the unfused kernels."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import to_np
from oracle import bf16 as o_bf16
from oracle import fp8 as o_fp8
from oracle import norms as o_norms

pytestmark = pytest.mark.gpu


def _codes(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.uint8).cpu().numpy()


def _bf16_values(a: np.ndarray) -> np.ndarray:
    return o_bf16.round_f32(a.astype(np.float32))


@pytest.mark.parametrize("n,k,spread", [(128, 128, 1.0), (384, 256, 0.02), (1024, 2048, 0.02)])
def test_weight_blocks_match_oracle(nq, device, n, k, spread):
    from nari_qwen3_tts_amd.layers import FP8, quantize_fp8_weight_blocks

    g = torch.Generator(device=device)
    g.manual_seed(n + k)
    scale_rows = torch.exp2(torch.randint(-12, 3, (n, 1), generator=g, device=device).float())
    w = (torch.randn(n, k, generator=g, device=device) * spread * scale_rows).to(torch.bfloat16)
    w[:128, :128] = 0  # a block below the 1e-4 clamp
    q, s = quantize_fp8_weight_blocks(w)
    torch.cuda.synchronize()
    assert q.dtype is FP8 and q.shape == w.shape and s.shape == (n // 128, k // 128)
    want_q, want_s = o_fp8.quantize_weight_blocks(to_np(w))
    assert np.array_equal(s.cpu().numpy(), want_s)
    assert np.array_equal(_codes(q), want_q)


def test_weight_blocks_reject_bad_shapes(nq, device):
    from nari_qwen3_tts_amd.layers import quantize_fp8_weight_blocks

    with pytest.raises(ValueError, match="divisible by 128"):
        quantize_fp8_weight_blocks(torch.ones((128, 64), dtype=torch.bfloat16, device=device))
    with pytest.raises(ValueError, match="contiguous"):
        quantize_fp8_weight_blocks(torch.ones((256, 256), dtype=torch.bfloat16, device=device)[:, :128])


@pytest.mark.parametrize("m,k", [(64, 2048), (7, 256), (130, 384)])
def test_rows_match_oracle(nq, device, m, k):
    from nari_qwen3_tts_amd.layers import quantize_fp8_rows

    g = torch.Generator(device=device)
    g.manual_seed(m * 31 + k)
    x = (torch.randn(m, k, generator=g, device=device) * torch.exp2(
        torch.randint(-20, 8, (m, 1), generator=g, device=device).float())).to(torch.bfloat16)
    x[min(3, m - 1), :128] = 0
    q, s = quantize_fp8_rows(x)
    torch.cuda.synchronize()
    want_q, want_s = o_fp8.quantize_rows(to_np(x))
    assert np.array_equal(s.cpu().numpy(), want_s)
    assert np.array_equal(_codes(q), want_q)


def _integer_case(device, m, n, k, seed):
    rng = np.random.default_rng(seed)
    xv = rng.integers(-8, 9, (m, k)).astype(np.float32)
    wv = rng.integers(-8, 9, (n, k)).astype(np.float32)
    # block sums stay below 8192 * 4 per block and 2^20 over 16 blocks, on a 2^-4 grid: exact in fp32
    sx = np.exp2(rng.integers(-2, 2, (m, k // 128))).astype(np.float32)
    sw = np.exp2(rng.integers(-2, 2, (n // 128, k // 128))).astype(np.float32)
    xq, wq = o_fp8.e4m3_from_f32(xv), o_fp8.e4m3_from_f32(wv)
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to(device).view(dt)  # noqa: E731
    return (xq, sx, wq, sw), (t(xq, torch.float8_e4m3fn), t(sx, torch.float32), t(wq, torch.float8_e4m3fn),
                              t(sw, torch.float32))


@pytest.mark.parametrize("m,n,k", [(64, 12288, 2048), (1, 256, 1024), (16, 128, 1024), (33, 384, 2048),
                                   (100, 256, 1024), (128, 512, 512), (200, 256, 1024)])
def test_gemm_exact_on_integer_codes(nq, device, m, n, k):
    """Integer codes and power-of-two scales keep every partial sum exact in fp32, so the
    bf16 output must equal the rounded oracle bit for bit."""
    from nari_qwen3_tts_amd.layers import linear_fp8

    ref, dev = _integer_case(device, m, n, k, m + n + k)
    y = linear_fp8(*dev)
    torch.cuda.synchronize()
    want = o_bf16.to_bits(o_fp8.blockscale_gemm(*ref).astype(np.float32))
    assert np.array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), want)


@pytest.mark.parametrize("m", [64, 5, 128])
def test_gemm_and_silu_match_oracle(nq, device, m):
    from nari_qwen3_tts_amd import _lib
    from nari_qwen3_tts_amd.layers import linear_fp8, silu_mul, quantize_fp8_rows, quantize_fp8_weight_blocks

    n, k = 1536, 2048
    g = torch.Generator(device=device)
    g.manual_seed(m)
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
    xq, sx = quantize_fp8_rows(x)
    wq, sw = quantize_fp8_weight_blocks(w)
    y = linear_fp8(xq, sx, wq, sw)
    act = linear_fp8(xq, sx, wq, sw, epilogue=_lib.NQ_EPI_SILU_MUL)
    torch.cuda.synchronize()
    exact = o_fp8.blockscale_gemm(_codes(xq), sx.cpu().numpy(), _codes(wq), sw.cpu().numpy())
    got = y.float().cpu().numpy()
    # fp32 accumulation in another order, then one bf16 rounding
    assert np.all(np.abs(got - exact) <= 2.0 ** -8 * np.abs(exact) + 1e-3)
    # SwiGLU of the bf16 projection in the oracle's own terms (fed the device projection: a one-ulp
    # bf16 flip of both gate and up, which the bound above allows, would compound in silu(g) * u)
    want_act = o_norms.silu_mul(got)
    err = np.abs(act.float().cpu().numpy() - want_act)
    assert np.all(err <= 2.0 ** -8 * np.abs(want_act) + 1e-6)
    # and the split-K planes summed by the fused SwiGLU equal the bf16 projection the NONE path
    # stores: the fused result is the unfused kernel's on that projection, bit for bit
    assert torch.equal(act, silu_mul(y))


def test_fused_add_rmsnorm_quantizes_like_unfused(nq, device):
    from nari_qwen3_tts_amd.layers import (add_rmsnorm_fp8, linear_add_rmsnorm, linear_add_rmsnorm_fp8,
                                           add_rmsnorm, quantize_fp8_rows)

    m, n, k = 64, 2048, 2048
    g = torch.Generator(device=device)
    g.manual_seed(11)
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
    res0 = torch.randn(m, n, generator=g, device=device).to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(n, generator=g, device=device)).to(torch.bfloat16)
    # GEMM + add-RMSNorm -> FP8 == GEMM + add-RMSNorm (bf16) -> row quantizer
    r1, r2 = res0.clone(), res0.clone()
    q1, s1 = linear_add_rmsnorm_fp8(x, w, r1, nw, 1e-6, None, None)
    normed = torch.empty(m, n, dtype=torch.bfloat16, device=device)
    linear_add_rmsnorm(x, w, r2, nw, 1e-6, normed)
    q2, s2 = quantize_fp8_rows(normed)
    # bf16 add-RMSNorm -> FP8 == add_rmsnorm -> row quantizer
    h = torch.randn(m, n, generator=g, device=device).to(torch.bfloat16)
    r3, r4, h4 = res0.clone(), res0.clone(), h.clone()
    q3, s3 = add_rmsnorm_fp8(h, r3, nw, 1e-6)
    add_rmsnorm(h4, r4, nw, 1e-6)
    q4, s4 = quantize_fp8_rows(h4)
    torch.cuda.synchronize()
    assert torch.equal(r1, r2) and torch.equal(s1, s2) and torch.equal(q1.view(torch.uint8), q2.view(torch.uint8))
    assert torch.equal(r3, r4) and torch.equal(s3, s4) and torch.equal(q3.view(torch.uint8), q4.view(torch.uint8))


def test_pack_interleaves_gate_and_up_rows(nq, device):
    from nari_qwen3_tts_amd.layers import pack_fp8_swiglu

    inter, k = 48, 256
    codes = torch.randint(0, 256, (2 * inter, k), dtype=torch.uint8, device=device)
    packed = pack_fp8_swiglu(codes.view(torch.float8_e4m3fn)).view(torch.uint8).cpu().numpy()
    src = codes.cpu().numpy()
    for p in range(2 * inter):
        t, q, e = p // 16, (p % 16) // 4, p % 4
        want = src[8 * t + 2 * q + e] if e < 2 else src[inter + 8 * t + 2 * q + e - 2]
        assert np.array_equal(packed[p], want), p


@pytest.mark.parametrize("m", [64, 1, 37])
def test_fused_swiglu_matches_split_path_and_oracle(nq, device, m):
    from nari_qwen3_tts_amd import _lib
    from nari_qwen3_tts_amd.layers import (linear_fp8, linear_fp8_swiglu, pack_fp8_swiglu, quantize_fp8_rows,
                                           quantize_fp8_weight_blocks)

    inter, k = 6144, 2048
    g = torch.Generator(device=device)
    g.manual_seed(100 + m)
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    w = (torch.randn(2 * inter, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
    xq, sx = quantize_fp8_rows(x)
    wq, sw = quantize_fp8_weight_blocks(w)
    packed = pack_fp8_swiglu(wq)
    fused = torch.empty(m, inter, dtype=torch.bfloat16, device=device)
    linear_fp8_swiglu(xq, sx, packed, sw, fused)
    y = linear_fp8(xq, sx, wq, sw)
    split = linear_fp8(xq, sx, wq, sw, epilogue=_lib.NQ_EPI_SILU_MUL)
    torch.cuda.synchronize()
    # the fused kernel sums K in quarters, the split path in halves: gate / up may differ by one
    # bf16 ulp, so act by about two
    a, b = fused.float().cpu().numpy(), split.float().cpu().numpy()
    assert np.all(np.abs(a - b) <= 2.0 ** -6 * np.abs(b) + 1e-4)
    assert np.mean(a != b) < 0.05
    # against the oracle's SwiGLU of the projection
    exact = o_fp8.blockscale_gemm(_codes(xq), sx.cpu().numpy(), _codes(wq), sw.cpu().numpy())
    want = o_norms.silu_mul(_bf16_values(exact))
    assert np.mean(np.abs(a - want)) <= 2e-3 * np.mean(np.abs(want)) + 1e-6
    assert np.all(np.abs(a - want) <= 2.0 ** -5 * np.abs(want) + 4e-3)
    del y


def test_fused_swiglu_integer_codes_exact(nq, device):
    """Integer codes, power-of-two scales: every sum is exact, so the fused result is the
    oracle's SwiGLU of the exact projection up to the activation's expf."""
    from nari_qwen3_tts_amd.layers import linear_fp8_swiglu, pack_fp8_swiglu

    m, inter, k = 64, 6144, 2048
    ref, dev = _integer_case(device, m, 2 * inter, k, 5)
    packed = pack_fp8_swiglu(dev[2])
    fused = torch.empty(m, inter, dtype=torch.bfloat16, device=device)
    linear_fp8_swiglu(dev[0], dev[1], packed, dev[3], fused)
    torch.cuda.synchronize()
    gu = _bf16_values(o_fp8.blockscale_gemm(*ref))
    want = o_norms.silu_mul(gu)
    got = fused.float().cpu().numpy()
    # gate and up are exact, so only silu's exp rounding separates the two (<= 1 bf16 ulp)
    assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + 1e-6)
