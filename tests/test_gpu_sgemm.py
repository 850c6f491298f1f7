"""The codec decoder's fp32 GEMM (nq_sgemm) and row norms (nq_row_norm) against torch on the CPU in
float64, at the decoder's shapes (transformer / ConvNeXt linears over ~960 frames, the im2col
convolutions and transposed convolutions of the decoder blocks, the per-stream overlap rows), at
both product precisions (torch's float32 matmul precisions by name).

- Integer-valued operands (including K and N tails of the small decoder: 48 / 40 / 20): every fp32
  sum is exact and every small integer is its own bf16 high part (low part zero), so at both
  precisions the product equals the float64 one bit for bit (pins the tiling, the K order
  permutation inside a lane and the row gather).
- Random operands with every epilogue (bias, GELU, per-column scale, residual, in place): "highest"
  within the fp32 accumulation bound 2e-5 x sum |x w| of the float64 reference; "high" within
  8e-5 x sum |x w|: v = hi + lo + e with |v - hi| <= 2^-8 |v| and |e| <= 2^-16 |v|, so each of the
  three dropped terms lo*lo', e*w, x*e' is at most 2^-16 |x w| (4.6e-5 together), plus the same
  accumulation bound.
- "high" really drops those terms: on random operands it is not bit-equal to "highest", and its
  error is above the fp32 one (a "high" that fell back to fp32 products fails this).
- RMSNorm and LayerNorm rows within 2e-6 relative of torch (float64)."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

SHAPES = [(960, 512, 512), (960, 1536, 512), (960, 512, 1536), (3840, 128, 3584), (3840, 320, 256),
          (19200, 64, 448), (19200, 160, 128), (37, 1024, 512), (5, 64, 64), (37, 40, 48), (200, 48, 20)]


HIGHEST, HIGH = 0, 1
BOUND = {HIGHEST: 2e-5, HIGH: 8e-5}


def _call(device, x, w, *, x_rows=None, bias=None, act=0, res=None, scale=None, out=None, precision=HIGHEST):
    from nari_qwen3_tts_amd import _lib

    rows = x.shape[0] if x_rows is None else x_rows.shape[0]
    out = torch.empty(rows, w.shape[0], dtype=torch.float32, device=device) if out is None else out
    _lib.call("nq_sgemm", x.data_ptr(), x.stride(0), _lib.ptr(x_rows), w.data_ptr(), w.stride(0), rows, w.shape[0],
              w.shape[1], _lib.ptr(bias), act, _lib.ptr(res), res.stride(0) if res is not None else 0, _lib.ptr(scale),
              out.data_ptr(), out.stride(0), precision, _lib.stream(device))
    return out


@pytest.mark.parametrize("precision", [HIGHEST, HIGH])
@pytest.mark.parametrize("m,n,k", SHAPES)
def test_sgemm_exact_on_integer_operands(nq, device, m, n, k, precision):
    gen = torch.Generator().manual_seed(m + n + k)
    x = torch.randint(-8, 9, (m, k), generator=gen).float()
    w = torch.randint(-8, 9, (n, k), generator=gen).float()
    got = _call(device, x.to(device), w.to(device), precision=precision).cpu()
    assert torch.equal(got.double(), x.double() @ w.double().t())
    # gathered rows (the per-stream overlap product): every third row, reversed
    rows = torch.arange(m - 1, -1, -3, dtype=torch.int32)
    got = _call(device, x.to(device), w.to(device), x_rows=rows.to(device), precision=precision).cpu()
    assert torch.equal(got.double(), x[rows.long()].double() @ w.double().t())


@pytest.mark.parametrize("precision", [HIGHEST, HIGH])
@pytest.mark.parametrize("m,n,k", SHAPES[:6])
@pytest.mark.parametrize("epi", ["bias", "bias_gelu", "scale_res", "bias_scale_res_inplace"])
def test_sgemm_epilogues(nq, device, m, n, k, epi, precision):
    g = torch.Generator().manual_seed(7 * m + n + k)
    x = torch.randn(m, k, generator=g)
    w = torch.randn(n, k, generator=g) / k ** 0.5
    b = torch.randn(n, generator=g) * 0.1
    sc = torch.rand(n, generator=g) + 0.05
    r = torch.randn(m, n, generator=g)
    xd, wd = x.to(device), w.to(device)
    y = x.double() @ w.double().t()
    bound = x.double().abs() @ w.double().abs().t()
    p = dict(precision=precision)
    if epi == "bias":
        got = _call(device, xd, wd, bias=b.to(device), **p)
        want = y + b.double()
    elif epi == "bias_gelu":
        got = _call(device, xd, wd, bias=b.to(device), act=1, **p)
        want = F.gelu(y + b.double())
    elif epi == "scale_res":
        got = _call(device, xd, wd, scale=sc.to(device), res=r.to(device), **p)
        want = r.double() + sc.double() * y
    else:
        rd = r.to(device)
        got = _call(device, xd, wd, bias=b.to(device), scale=sc.to(device), res=rd, out=rd, **p)
        assert got.data_ptr() == rd.data_ptr()
        want = r.double() + sc.double() * (y + b.double())
        bound = bound * sc.double()
    err = (got.cpu().double() - want).abs()
    tol = BOUND[precision]
    assert bool((err <= tol * bound + 1e-6).all()), float((err - tol * bound).max())


@pytest.mark.parametrize("m,n,k", [(960, 1536, 512), (3840, 128, 3584)])
def test_high_precision_takes_the_split_products(nq, device, m, n, k):
    g = torch.Generator().manual_seed(m * 3 + k)
    x = torch.randn(m, k, generator=g)
    w = torch.randn(n, k, generator=g) / k ** 0.5
    xd, wd = x.to(device), w.to(device)
    want = x.double() @ w.double().t()
    full = _call(device, xd, wd, precision=HIGHEST).cpu().double()
    split = _call(device, xd, wd, precision=HIGH).cpu().double()
    assert not torch.equal(full, split)
    e_full, e_split = float((full - want).abs().mean()), float((split - want).abs().mean())
    # split: about 2^-16 relative per product against about 2^-24 for fp32 products
    assert e_split > 4 * e_full, (e_split, e_full)
    bound = x.double().abs() @ w.double().abs().t()
    assert bool(((split - want).abs() <= BOUND[HIGH] * bound + 1e-6).all())


@pytest.mark.parametrize("rows,width", [(960, 512), (3840, 512), (3, 1024), (7, 64)])
def test_row_norms(nq, device, rows, width):
    from nari_qwen3_tts_amd import _lib

    g = torch.Generator().manual_seed(rows + width)
    x = torch.randn(rows, width, generator=g) * 3 + 0.5
    w = torch.rand(width, generator=g) + 0.5
    b = torch.randn(width, generator=g)
    xd, wd, bd = x.to(device), w.to(device), b.to(device)  # held: the kernel reads them after the call
    for layer in (False, True):
        out = torch.empty(rows, width, device=device)
        _lib.call("nq_row_norm", xd.data_ptr(), xd.stride(0), rows, width, wd.data_ptr(), _lib.ptr(bd if layer else None),
                  1e-6, out.data_ptr(), out.stride(0), _lib.stream(device))
        xx = x.double()
        if layer:
            want = F.layer_norm(xx, (width,), w.double(), b.double(), 1e-6)
        else:
            want = xx * torch.rsqrt(xx.pow(2).mean(-1, keepdim=True) + 1e-6) * w.double()
        err = (out.cpu().double() - want).abs()
        assert bool((err <= 2e-6 * want.abs().clamp(min=1.0)).all()), (layer, float(err.max()))
