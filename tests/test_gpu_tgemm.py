"""The tiled prefill GEMMs (nq_tgemm, nq_tgemm_fp8_swiglu) against exact references.

- Integer-valued bf16 operands keep every fp32 partial sum exact, so the bf16 product must equal the
  fp32 matmul rounded to bf16 bit for bit, whatever the tile shape and summation order; random
  operands are then held to fp32-accumulation tolerance.  Shapes: the talker projections at the
  prefill captures' token counts (640 tokens for QKV / o / gate_up / down), row tails (37, 129, 300
  rows), one-row and one-stage edge cases.
- The split-K planes, the add-RMSNorm epilogue and its FP8-output form give the bits of the bf16
  product followed by the plane sum in order / the add-RMSNorm kernels.
- The bf16 SwiGLU epilogue on [gate; up] weights equals silu(bf16(g)) * bf16(u) of the exact product
  up to the activation's expf (one bf16 ulp).
- The tiled FP8 gate/up + SwiGLU on integer e4m3 codes with power-of-two scales (exact block sums)
  equals the oracle's SwiGLU of the oracle block-scaled product up to expf, at 640, 300 and 37 rows;
  on random codes it agrees with the decode kernel (nq_linear_fp8_swiglu) within two bf16 ulps."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import bf16 as o_bf16
from oracle import fp8 as o_fp8
from oracle import norms as o_norms

pytestmark = pytest.mark.gpu

SHAPES = [(640, 4096, 2048), (640, 2048, 2048), (640, 2048, 6144), (37, 2048, 2048), (129, 3072, 2048),
          (300, 4096, 2048), (1, 128, 64), (64, 128, 64)]


def _ws(rows, n, k, epilogue=0):
    from nari_qwen3_tts_amd.layers import tgemm_workspace_bytes

    return torch.empty(max(16, tgemm_workspace_bytes(rows, n, k, epilogue)), dtype=torch.uint8, device="cuda:0")


def _int_bf16(shape, gen, device, lo=-4, hi=5):
    return torch.randint(lo, hi, shape, generator=gen).to(torch.bfloat16).to(device)


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_tgemm_exact_on_integer_operands(nq, device, m, n, k):
    from nari_qwen3_tts_amd.layers import tgemm

    gen = torch.Generator().manual_seed(m * 7 + n + k)
    x, w = _int_bf16((m, k), gen, device), _int_bf16((n, k), gen, device)
    out = torch.full((m, n), 7.0, dtype=torch.bfloat16, device=device)
    tgemm(x, w, out, workspace=_ws(m, n, k))
    want = (x.float() @ w.float().t()).to(torch.bfloat16)  # sums below 2^24: exact in fp32
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("m,n,k", SHAPES[:5])
def test_tgemm_random_within_fp32_accumulation(nq, device, m, n, k):
    from nari_qwen3_tts_amd.layers import tgemm

    g = torch.Generator(device=device)
    g.manual_seed(m + n + k)
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
    # a strided x (every other row of a wider buffer) and a strided out
    wide = torch.zeros(m, k + 64, dtype=torch.bfloat16, device=device)
    wide[:, :k] = x
    out_wide = torch.zeros(m, n + 64, dtype=torch.bfloat16, device=device)
    tgemm(wide[:, :k], w, out_wide[:, :n], workspace=_ws(m, n, k))
    ref = x.double() @ w.double().t()
    got = out_wide[:, :n].double()
    torch.cuda.synchronize()
    # one bf16 rounding of a value whose fp32 sum differs from the exact one by < K * 2^-24 relative
    tol = ref.abs() * 2.0 ** -8 + 1e-5 * (k ** 0.5)
    assert bool(((got - ref).abs() <= tol).all()), float((got - ref).abs().max())
    assert bool((out_wide[:, n:] == 0).all())


@pytest.mark.parametrize("m", [640, 300, 37])
def test_tgemm_swiglu_epilogue(nq, device, m):
    from nari_qwen3_tts_amd import _lib
    from nari_qwen3_tts_amd.layers import tgemm

    inter, k = 6144, 2048
    gen = torch.Generator().manual_seed(m)
    x, w = _int_bf16((m, k), gen, device, -2, 3), _int_bf16((2 * inter, k), gen, device, -2, 3)
    act = torch.empty(m, inter, dtype=torch.bfloat16, device=device)
    # operands scaled by 1/8 (exact in bf16) so that silu sees values of order one; sums stay exact
    x8, w8 = (x.float() / 8).to(torch.bfloat16), (w.float() / 8).to(torch.bfloat16)
    tgemm(x8, w8, act, epilogue=_lib.NQ_EPI_SILU_MUL)
    gu = (x8.double() @ w8.double().t()).float().cpu().numpy()
    want = o_norms.silu_mul(o_bf16.round_f32(gu))
    got = act.float().cpu().numpy()
    torch.cuda.synchronize()
    assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + 1e-6)


def _fp8_integer_case(device, m, n, k, seed):
    rng = np.random.default_rng(seed)
    xv = rng.integers(-8, 9, (m, k)).astype(np.float32)
    wv = rng.integers(-8, 9, (n, k)).astype(np.float32)
    sx = np.exp2(rng.integers(-9, -6, (m, k // 128))).astype(np.float32)
    sw = np.exp2(rng.integers(-3, -1, (n // 128, k // 128))).astype(np.float32)
    xq, wq = o_fp8.e4m3_from_f32(xv), o_fp8.e4m3_from_f32(wv)
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to(device).view(dt)  # noqa: E731
    return (xq, sx, wq, sw), (t(xq, torch.float8_e4m3fn), t(sx, torch.float32), t(wq, torch.float8_e4m3fn),
                              t(sw, torch.float32))


# 640 and 300 rows run the 128 x 256 tiles, 768 the 128 x 128 ones (fewer rounds), 1280 two rounds of
# 128 x 256 tiles, 37 the 64 x 64 tiles
@pytest.mark.parametrize("m", [640, 300, 37, 768, 1280])
def test_tgemm_fp8_swiglu_exact_on_integer_codes(nq, device, m):
    from nari_qwen3_tts_amd.layers import pack_fp8_swiglu, tgemm_fp8_swiglu

    inter, k = 6144, 2048
    ref, dev = _fp8_integer_case(device, m, 2 * inter, k, m)
    packed = pack_fp8_swiglu(dev[2])
    out = torch.empty(m, inter, dtype=torch.bfloat16, device=device)
    tgemm_fp8_swiglu(dev[0], dev[1], packed, dev[3], out)
    gu = o_bf16.round_f32(o_fp8.blockscale_gemm(*ref).astype(np.float32))
    want = o_norms.silu_mul(gu)
    got = out.float().cpu().numpy()
    torch.cuda.synchronize()
    assert float(np.abs(want).mean()) > 0.1  # silu sees values of order one
    assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + 1e-6)


def test_tgemm_fp8_swiglu_agrees_with_decode_kernel(nq, device):
    from nari_qwen3_tts_amd.layers import (linear_fp8_swiglu, pack_fp8_swiglu, quantize_fp8_rows,
                                           quantize_fp8_weight_blocks, tgemm_fp8_swiglu)

    m, inter, k = 64, 6144, 2048
    g = torch.Generator(device=device)
    g.manual_seed(17)
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    w = (torch.randn(2 * inter, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
    xq, sx = quantize_fp8_rows(x)
    wq, sw = quantize_fp8_weight_blocks(w)
    packed = pack_fp8_swiglu(wq)
    a = torch.empty(m, inter, dtype=torch.bfloat16, device=device)
    b = torch.empty_like(a)
    tgemm_fp8_swiglu(xq, sx, packed, sw, a)
    linear_fp8_swiglu(xq, sx, packed, sw, b)
    torch.cuda.synchronize()
    a, b = a.float().cpu().numpy(), b.float().cpu().numpy()
    # K summed block by block here, in quarters there: gate / up may differ by one bf16 ulp
    assert np.all(np.abs(a - b) <= 2.0 ** -6 * np.abs(b) + 1e-4)
    assert np.mean(a != b) < 0.05


@pytest.mark.parametrize("m,n,k", [(640, 2048, 2048), (300, 2048, 6144), (640, 4096, 2048), (129, 2048, 2048)])
def test_tgemm_planes_and_norm_epilogues(nq, device, m, n, k):
    from nari_qwen3_tts_amd import _lib
    from nari_qwen3_tts_amd.layers import add_rmsnorm, add_rmsnorm_fp8, tgemm, tgemm_add_rmsnorm_fp8, tgemm_partials

    g = torch.Generator(device=device)
    g.manual_seed(m + 3 * n + k)
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
    res0 = torch.randn(m, n, generator=g, device=device).to(torch.bfloat16)
    norm = (torch.rand(n, generator=g, device=device) + 0.5).to(torch.bfloat16)
    y = torch.empty(m, n, dtype=torch.bfloat16, device=device)
    tgemm(x, w, y, workspace=_ws(m, n, k))
    # planes: summed in plane order and rounded, they are the bf16 product
    ws = _ws(m, n, k, _lib.NQ_EPI_PARTIALS)
    splits = tgemm_partials(x, w, ws)
    planes = ws[: splits * m * n * 4].view(torch.float32).view(splits, m, n)
    acc = planes[0].clone()
    for s_ in range(1, splits):
        acc += planes[s_]
    assert torch.equal(acc.to(torch.bfloat16), y)
    # add-RMSNorm epilogue == product, then the add-RMSNorm kernel
    r_a, r_b = res0.clone(), res0.clone()
    h = torch.empty_like(y)
    tgemm(x, w, h, _lib.NQ_EPI_ADD_RMSNORM, r_a, norm, 1e-6, _ws(m, n, k, _lib.NQ_EPI_ADD_RMSNORM))
    y2 = y.clone()
    add_rmsnorm(y2, r_b, norm, 1e-6)
    assert torch.equal(r_a, r_b) and torch.equal(h, y2)
    if n % 128 == 0:
        r_a, r_b = res0.clone(), res0.clone()
        qa, sa = tgemm_add_rmsnorm_fp8(x, w, r_a, norm, 1e-6, None, None, _ws(m, n, k, _lib.NQ_EPI_ADD_RMSNORM))
        qb, sb = add_rmsnorm_fp8(y.clone(), r_b, norm, 1e-6)
        assert torch.equal(r_a, r_b)
        assert torch.equal(qa.view(torch.uint8), qb.view(torch.uint8)) and torch.equal(sa, sb)
    torch.cuda.synchronize()
