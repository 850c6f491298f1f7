"""The norm / SwiGLU drop-ins called with the reference's exact arguments (model/layers.py:28-100,
264-270): the RMSNorm module as ``norm``, the ``use_cuda_kernel`` keyword.  Inputs that the
reference keeps off its kernels (CPU tensors, fp32, ``use_cuda_kernel=False``) take its torch math;
bf16 device tensors run the HIP kernels (the ``-m gpu`` case below)."""

from __future__ import annotations

import pytest
import torch


class RMSNorm(torch.nn.Module):
    """The reference module's interface (weight, variance_epsilon, fp32 forward; model/layers.py:103-115)."""

    def __init__(self, hidden: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.variance_epsilon = eps
        self.weight = torch.nn.Parameter(torch.ones(hidden))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        v = x.float()
        return (v * torch.rsqrt(v.square().mean(-1, keepdim=True) + self.variance_epsilon)
                * self.weight.float()).to(x.dtype)


def _layers(nq):
    from nari_qwen3_tts_amd import layers

    return layers


def test_shims_take_the_reference_arguments_on_cpu(nq):
    L = _layers(nq)
    g = torch.Generator().manual_seed(3)
    norm = RMSNorm(64)
    with torch.no_grad():
        norm.weight.copy_(torch.rand(64, generator=g) + 0.5)
    h = torch.randn(4, 64, generator=g)
    r = torch.randn(4, 64, generator=g)
    # model/layers.py:42-78 fallback: residual + hidden, then norm(residual); new tensors returned
    out_h, out_r = L.qwen3_tts_add_rmsnorm(h, r, norm, use_cuda_kernel=True)
    torch.testing.assert_close(out_r, r + h)
    torch.testing.assert_close(out_h, norm(r + h))
    out_h2, _ = L.qwen3_tts_add_rmsnorm(h, r, norm)
    torch.testing.assert_close(out_h2, out_h)
    torch.testing.assert_close(L.qwen3_tts_rmsnorm(h, norm, use_cuda_kernel=False), norm(h))
    gu = torch.randn(4, 2 * 32, generator=g)
    gate, up = gu.chunk(2, dim=-1)
    torch.testing.assert_close(L.qwen3_tts_silu_and_mul(gu, use_cuda_kernel=True),
                               torch.nn.functional.silu(gate) * up)
    # keyword-only, as GatedMLP.forward passes it (model/layers.py:264-270)
    with pytest.raises(TypeError):
        L.qwen3_tts_silu_and_mul(gu, True)
    with pytest.raises(TypeError):
        L.qwen3_tts_add_rmsnorm(h, r, norm, True)


@pytest.mark.gpu
def test_shims_run_the_kernels_on_bf16_device_tensors(nq, device):
    L = _layers(nq)
    g = torch.Generator(device=device).manual_seed(4)
    width = 2048
    norm = RMSNorm(width).to(device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_(torch.rand(width, generator=g, device=device) + 0.5)
    h = torch.randn(64, width, generator=g, device=device).to(torch.bfloat16)
    r = torch.randn(64, width, generator=g, device=device).to(torch.bfloat16)
    h2, r2 = h.clone(), r.clone()
    out_h, out_r = L.qwen3_tts_add_rmsnorm(h, r, norm, use_cuda_kernel=True)
    # in place on both tensors, the same bits as the (weight, eps) kernel entry
    assert out_h.data_ptr() == h.data_ptr() and out_r.data_ptr() == r.data_ptr()
    L.add_rmsnorm(h2, r2, norm.weight.detach(), norm.variance_epsilon)
    assert torch.equal(h, h2) and torch.equal(r, r2)
    # against the reference module's own math, within bf16 rounding of its output
    rr = (r2.float()).to(torch.bfloat16)
    assert (norm(rr).float() - h.float()).abs().max().item() <= 2e-2
    x = torch.randn(8, 3, width, generator=g, device=device).to(torch.bfloat16)
    y = L.qwen3_tts_rmsnorm(x, norm, use_cuda_kernel=True)
    assert y.shape == x.shape
    assert torch.equal(y, L.rmsnorm(x, norm.weight.detach(), norm.variance_epsilon))
    gu = torch.randn(64, 2 * 6144, generator=g, device=device).to(torch.bfloat16)
    assert torch.equal(L.qwen3_tts_silu_and_mul(gu, use_cuda_kernel=True), L.silu_mul(gu))
    # a strided view (the reference guard sends non-contiguous add-norm inputs to its torch math)
    hs, rs = h[:, ::2], r[:, ::2].contiguous()
    n2 = RMSNorm(width // 2).to(device=device, dtype=torch.bfloat16)
    out_h, out_r = L.qwen3_tts_add_rmsnorm(hs, rs, n2)
    torch.testing.assert_close(out_r, rs + hs)
    # fp16 device tensors: the reference would use its kernel; ours is bf16 only and says so
    with pytest.raises(TypeError):
        L.qwen3_tts_silu_and_mul(gu.to(torch.float16))
