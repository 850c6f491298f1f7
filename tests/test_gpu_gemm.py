"""Skinny HIP projection (nq_linear) vs a torch fp32 reference of the same product, and its fused
epilogues vs the unfused kernels (bit-exact: the split-K planes are summed in one fixed order)."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

# talker decode shapes (packed QKV, o_proj, gate_up, down, codec head), the
# code-predictor shapes at 128 rows, and ragged / single-slice edge cases
SHAPES = [
    (64, 4096, 2048),
    (64, 2048, 2048),
    (64, 12288, 2048),
    (64, 2048, 6144),
    (16, 2048, 6144),  # 768-column K slices with one and two 16-row tiles
    (32, 2048, 6144),
    (7, 4096, 3072),
    (64, 3072, 2048),
    (128, 4096, 1024),
    (128, 1024, 2048),
    (1, 64, 512),
    (37, 192, 1024),
    (16, 128, 512),
    (100, 320, 768),
    # more than 64 rows, as row blocks: 768-column slices in 32-row blocks (the code predictor's down),
    # in 64-row blocks with a 36-row last block; 256-column slices in 32-row blocks (its o projection),
    # in 64-row blocks with a 26-row and with a one-row last block
    (128, 1024, 3072),
    (100, 2048, 6144),
    (128, 1024, 1024),
    (90, 1024, 3072),
    (65, 2048, 2048),
]


def _reference(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    return x.float() @ w.float().t()


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_linear_matches_fp32_reference(nq, device, m, n, k):
    from nari_qwen3_tts_amd.layers import linear

    g = torch.Generator(device=device)
    g.manual_seed(m * 7 + n + k)
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
    y = linear(x, w)
    torch.cuda.synchronize()
    ref = _reference(x, w)
    err = (y.float() - ref).abs()
    # fp32 accumulation in another order, then one bf16 rounding of the result
    bound = 8e-3 * ref.abs() + 2e-3
    assert bool((err <= bound).all()), f"max err {err.max().item():.3g}"


def test_linear_strided_rows_and_determinism(nq, device):
    from nari_qwen3_tts_amd.layers import linear

    g = torch.Generator(device=device)
    g.manual_seed(5)
    m, n, k = 64, 2048, 2048
    xbuf = torch.randn(m, k + 64, generator=g, device=device).to(torch.bfloat16)
    x = xbuf[:, 32 : 32 + k]  # row stride k + 64, 64-byte offset
    w = (torch.randn(n, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
    obuf = torch.full((m, n + 128), 7.0, dtype=torch.bfloat16, device=device)
    out = obuf[:, :n]
    linear(x, w, out=out)
    first = out.clone()
    linear(x, w, out=out)
    torch.cuda.synchronize()
    assert torch.equal(first, out), "split-K reduction must be deterministic"
    assert bool((obuf[:, n:] == 7.0).all()), "columns past N must stay untouched"
    ref = _reference(x, w)
    assert bool(((out.float() - ref).abs() <= 8e-3 * ref.abs() + 2e-3).all())


def test_linear_rejects_unsupported_shapes(nq, device):
    from nari_qwen3_tts_amd.layers import linear

    x = torch.zeros(8, 500, dtype=torch.bfloat16, device=device)
    w = torch.zeros(64, 500, dtype=torch.bfloat16, device=device)
    with pytest.raises(TypeError):
        linear(x, w)
    with pytest.raises(TypeError):
        linear(torch.zeros(200, 512, dtype=torch.bfloat16, device=device),
               torch.zeros(64, 512, dtype=torch.bfloat16, device=device))


@pytest.mark.parametrize("m", [64, 37, 128])
def test_fused_add_rmsnorm_equals_unfused(nq, device, m):
    from nari_qwen3_tts_amd.layers import linear, linear_add_rmsnorm, add_rmsnorm

    g = torch.Generator(device=device)
    g.manual_seed(11 + m)
    k, n = (6144, 2048) if m != 128 else (1024, 1024)
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
    res = torch.randn(m, n, generator=g, device=device).to(torch.bfloat16)
    nw = (torch.rand(n, generator=g, device=device) + 0.5).to(torch.bfloat16)
    # unfused: projection, then the add-RMSNorm kernel
    y = linear(x, w)
    res_a = res.clone()
    add_rmsnorm(y, res_a, nw, 1e-6)
    # fused
    res_b = res.clone()
    out = torch.empty(m, n, dtype=torch.bfloat16, device=device)
    linear_add_rmsnorm(x, w, res_b, nw, 1e-6, out)
    torch.cuda.synchronize()
    assert torch.equal(res_a, res_b)
    assert torch.equal(y, out)


@pytest.mark.parametrize("m,k,inter", [(64, 2048, 6144), (5, 2048, 6144), (128, 1024, 3072), (128, 2048, 6144),
                                       (100, 1024, 3072)])
def test_fused_silu_mul_equals_unfused(nq, device, m, k, inter):
    """The talker (2048 -> 2 x 6144) and code-predictor (1024 -> 2 x 3072) gate/up shapes up to 128 rows."""
    from nari_qwen3_tts_amd import _lib
    from nari_qwen3_tts_amd.layers import linear, linear_silu_mul, silu_mul

    if _lib.load().nq_linear_splits(m, 2 * inter, k) <= 0:
        pytest.skip(f"no HIP projection for {m} x {k} -> {2 * inter}")
    g = torch.Generator(device=device)
    g.manual_seed(21 + m)
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    w = (torch.randn(2 * inter, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
    want = silu_mul(linear(x, w))
    got = linear_silu_mul(x, w)
    torch.cuda.synchronize()
    assert torch.equal(want, got)


def test_partials_epilogue_sums_to_the_projection(nq, device):
    from nari_qwen3_tts_amd import _lib
    from nari_qwen3_tts_amd.layers import linear, linear_workspace_bytes

    g = torch.Generator(device=device)
    g.manual_seed(31)
    m, n, k = 64, 4096, 2048
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
    splits = int(_lib.load().nq_linear_splits(m, n, k))
    ws = torch.empty(linear_workspace_bytes(m, n, k, _lib.NQ_EPI_PARTIALS), dtype=torch.uint8, device=device)
    _lib.call("nq_linear", x.data_ptr(), k, w.data_ptr(), k, m, n, k, _lib.NQ_EPI_PARTIALS, None, None, 0, None,
              None, 0.0, ws.data_ptr(), ws.numel(), _lib.stream(device))
    planes = ws.view(torch.float32)[: splits * m * n].view(splits, m, n)
    total = planes[0].clone()
    for s in range(1, splits):
        total += planes[s]
    torch.cuda.synchronize()
    assert torch.equal(total.to(torch.bfloat16), linear(x, w))


@pytest.mark.parametrize("m,n,k", [(128, 1024, 2048), (8, 128, 512)])
def test_linear_bias_single_rounding(nq, device, m, n, k):
    from nari_qwen3_tts_amd.layers import linear

    g = torch.Generator(device=device)
    g.manual_seed(41 + m)
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
    b = torch.randn(n, generator=g, device=device).to(torch.bfloat16)
    y = linear(x, w, bias=b)
    torch.cuda.synchronize()
    ref = _reference(x, w) + b.float()
    assert bool(((y.float() - ref).abs() <= 8e-3 * ref.abs() + 2e-3).all())


_PACKED_OFF = pytest.mark.skip(reason="the packed projection weight layout (nq_pack_linear_weight) was taken out of the library: the GPU run that exercised it ended in a device fault whose cause was not found (index arithmetic emulated in bounds); these tests of it stay, skipped")


@_PACKED_OFF
@pytest.mark.parametrize("m,n,k", SHAPES)
def test_packed_weights_give_identical_results(nq, device, m, n, k):
    from nari_qwen3_tts_amd.layers import linear, pack_linear_weight

    g = torch.Generator(device=device)
    g.manual_seed(m * 11 + n + 3 * k)
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
    packed = pack_linear_weight(w)
    # the layout: fragment (row group, 32-k step), lane (k group, row) of 8 consecutive k
    want = w.view(n // 16, 16, k // 32, 4, 8).permute(0, 2, 3, 1, 4).reshape(-1)
    assert torch.equal(packed.data, want)
    # the same lanes see the same operands in the same order: bit-identical products
    assert torch.equal(linear(x, packed), linear(x, w))


@_PACKED_OFF
def test_packed_weights_in_fused_epilogues(nq, device):
    from nari_qwen3_tts_amd.layers import (
        linear_add_rmsnorm, linear_add_rmsnorm_fp8, linear_partials, linear_workspace_bytes, pack_linear_weight,
    )
    from nari_qwen3_tts_amd import _lib

    g = torch.Generator(device=device)
    g.manual_seed(5)
    m, n, k = 64, 2048, 6144
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    # a weight view with a row stride wider than K packs like its contiguous copy
    wide = (torch.randn(n, k + 64, generator=g, device=device) * 0.02).to(torch.bfloat16)
    w = wide[:, :k]
    packed = pack_linear_weight(w)
    assert torch.equal(packed.data, pack_linear_weight(w.contiguous()).data)
    res = torch.randn(m, n, generator=g, device=device).to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(n, generator=g, device=device)).to(torch.bfloat16)
    ws = torch.empty(linear_workspace_bytes(m, n, k, _lib.NQ_EPI_ADD_RMSNORM), dtype=torch.uint8, device=device)
    ws2 = torch.empty_like(ws)
    s1 = linear_partials(x, w, ws)
    s2 = linear_partials(x, packed, ws2)
    assert s1 == s2 and torch.equal(ws, ws2)
    outs = []
    for weight in (w, packed):
        r = res.clone()
        out = torch.empty(m, n, dtype=torch.bfloat16, device=device)
        linear_add_rmsnorm(x, weight, r, nw, 1e-6, out, ws)
        r8 = res.clone()
        q, sc = linear_add_rmsnorm_fp8(x, weight, r8, nw, 1e-6, None, None, ws)
        outs.append((r, out, r8, q.view(torch.uint8).clone(), sc.clone()))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@_PACKED_OFF
def test_pack_rejects_unsupported_shapes(nq, device):
    from nari_qwen3_tts_amd.layers import pack_linear_weight

    with pytest.raises(TypeError):
        pack_linear_weight(torch.zeros(24, 64, dtype=torch.bfloat16, device=device))
    with pytest.raises(TypeError):
        pack_linear_weight(torch.zeros(32, 48, dtype=torch.bfloat16, device=device))


@pytest.mark.parametrize("m,inter", [(128, 3072), (64, 3072), (37, 96), (1, 96), (200, 3072)])
def test_fused_bf16_swiglu_equals_split_k_silu_mul(nq, device, m, inter):
    """One kernel over interleaved gate/up rows (K = 1024): at 128 rows (the code predictor's batch,
    where the split-K projection cuts K into the same four 256-wide slices) the bits of the split-K
    projection followed by the SiLU-mul kernel; at every row count within fp32-summation-order
    rounding of a float32 torch reference (gate and up rounded to bf16 first)."""

    from nari_qwen3_tts_amd.layers import linear_silu_mul, linear_swiglu, pack_swiglu

    print(f"case m {m} inter {inter}", flush=True)
    k = 1024
    g = torch.Generator(device=device)
    g.manual_seed(m * 7 + inter)
    x = (torch.randn(m, k, generator=g, device=device) * 0.5).to(torch.bfloat16)
    w = (torch.randn(2 * inter, k, generator=g, device=device) * 0.05).to(torch.bfloat16)
    packed = pack_swiglu(w)
    out = torch.full((m, inter), float("nan"), dtype=torch.bfloat16, device=device)
    linear_swiglu(x, packed, out)
    torch.cuda.synchronize()
    y = x.float() @ w.float().t()
    gate, up = y[:, :inter].bfloat16().float(), y[:, inter:].bfloat16().float()
    want = gate / (1.0 + torch.exp(-gate)) * up
    err = (out.float() - want).abs()
    # one bf16 rounding of the product plus a rare one-ulp flip of gate or up
    assert bool((err <= want.abs() * 2.0 ** -6 + 1e-5).all()), f"max err {err.max().item():.3g}"
    if m == 128:
        assert torch.equal(out, linear_silu_mul(x, w))
    # the packed rows are a permutation of the original rows
    assert torch.equal(packed.sort(dim=0).values, w.sort(dim=0).values)


def test_fused_bf16_swiglu_falls_back_outside_its_shape(nq, device):
    from nari_qwen3_tts_amd.layers import linear_silu_mul, linear_swiglu, pack_swiglu

    g = torch.Generator(device=device)
    g.manual_seed(5)
    x = (torch.randn(16, 512, generator=g, device=device) * 0.5).to(torch.bfloat16)
    w = (torch.randn(2 * 96, 512, generator=g, device=device) * 0.05).to(torch.bfloat16)
    out = torch.empty(16, 96, dtype=torch.bfloat16, device=device)
    linear_swiglu(x, pack_swiglu(w), out, weight=w)
    assert torch.equal(out, linear_silu_mul(x, w))
    with pytest.raises(TypeError):
        linear_swiglu(x, pack_swiglu(w), out)
