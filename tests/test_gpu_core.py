"""GPU parity of fused RMSNorm-SiLU (fused_rmsnorm_silu).

Tolerances: fp32 forward 2e-5 (tests/cuda/test_core_cuda.py:73), inverse rms
2e-6 relative (.colab_run_existing.py:122), backward 3e-4
(test_core_cuda.py:94-95). bf16 (C2, C3): every output is within 1 bf16 ulp of
the float64 oracle rounded to bf16 (the kernel computes in fp32 and rounds
once), counted and printed.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from koemi_amd import core, loader, workloads

pytestmark = pytest.mark.gpu


def bf16_ulps(got_bf16: torch.Tensor, want64: np.ndarray) -> np.ndarray:
    """Distance in bf16 ulps between kernel output and the f64 oracle rounded to bf16."""

    got_bits = got_bf16.view(torch.int16).cpu().numpy().astype(np.int32)
    want_bits = oracle.f32_to_bf16(want64.astype(np.float32)).astype(np.int16).astype(np.int32)
    # map sign-magnitude bf16 bit patterns to a monotone integer line
    def line(b):
        return np.where(b < 0, -(b & 0x7FFF), b)
    return np.abs(line(got_bits) - line(want_bits))


def test_forward_matches_torch_fp32(device):
    torch.manual_seed(11)
    x = torch.randn((5, 257), device=device)
    w = torch.randn((257,), device=device)
    expected = F.silu(x * torch.rsqrt(x.square().mean(dim=-1, keepdim=True) + 1e-6) * w)
    got = core.fused_rmsnorm_silu(x, w, 1e-6)
    torch.testing.assert_close(got, expected, atol=2e-5, rtol=2e-5)


@pytest.mark.parametrize("shape", [(3, 129), (8, 128), (64, 512), (17, 1000)])
def test_backward_matches_autograd(device, shape):
    torch.manual_seed(12)
    x0 = torch.randn(shape)
    w0 = torch.randn((shape[1],))
    up = torch.randn(shape)
    x = x0.to(device).requires_grad_()
    w = w0.to(device).requires_grad_()
    out = core.fused_rmsnorm_silu(x, w, 1e-6)
    (out * up.to(device)).sum().backward()
    xr, wr = x0.double().requires_grad_(), w0.double().requires_grad_()
    ref = F.silu(xr * torch.rsqrt(xr.square().mean(dim=-1, keepdim=True) + 1e-6) * wr)
    (ref * up.double()).sum().backward()
    torch.testing.assert_close(out.detach().cpu(), ref.detach().float(), atol=2e-5, rtol=2e-5)
    torch.testing.assert_close(x.grad.cpu(), xr.grad.float(), atol=3e-4, rtol=3e-4)
    torch.testing.assert_close(w.grad.cpu(), wr.grad.float(), atol=3e-4, rtol=3e-4)


def test_native_op_surface_and_inverse_rms(device):
    ext = core.load_core_extension(device=device)
    assert ext.KOEMI_CUDA_ABI_VERSION == 1
    torch.manual_seed(101)
    x = torch.randn((8, 128), device=device)
    w = torch.randn((128,), device=device)
    y, inv = ext.rmsnorm_silu_forward(x, w, 1e-6)
    torch.testing.assert_close(inv, torch.rsqrt(x.square().mean(dim=-1) + 1e-6), rtol=2e-5, atol=2e-6)
    dx, dw = ext.rmsnorm_silu_backward(torch.randn_like(y), x, w, inv, 1e-6)
    assert dx.shape == x.shape and dw.shape == w.shape


def test_gpu_contracts(device):
    x = torch.ones((2, 8), device=device)
    w = torch.ones((8,), device=device)
    with pytest.raises(loader.CudaExtensionValidationError, match="contiguous"):
        core.fused_rmsnorm_silu(x[:, ::2], w[:4])
    with pytest.raises(loader.CudaExtensionValidationError, match="same dtype"):
        core.fused_rmsnorm_silu(x, w.to(torch.float16))
    empty = core.fused_rmsnorm_silu(torch.empty((0, 8), device=device), w)
    assert empty.shape == (0, 8)


@pytest.mark.parametrize("dtype,hidden", [(torch.bfloat16, 100), (torch.float16, 512), (torch.bfloat16, 4096), (torch.float32, 2048), (torch.bfloat16, 8200)])
def test_low_precision_and_generic_widths(device, dtype, hidden):
    g = torch.Generator().manual_seed(hidden)
    x = torch.randn((37, hidden), generator=g).to(dtype)
    w = (1 + 0.02 * torch.randn((hidden,), generator=g)).to(dtype)
    got = core.fused_rmsnorm_silu(x.to(device), w.to(device), 1e-6)
    want, _ = oracle.rmsnorm_silu_f64(x.float().numpy(), w.float().numpy())
    if dtype == torch.bfloat16:
        assert bf16_ulps(got, want).max() <= 1
    else:
        tol = 2e-5 if dtype == torch.float32 else 1e-3
        np.testing.assert_allclose(got.float().cpu().numpy(), want, atol=tol, rtol=tol)


def test_config2_norm_full_within_one_bf16_ulp(device):
    c = workloads.config2()
    y, inv = core.rmsnorm_silu_forward(c.x.to(device), c.gamma.to(device), c.eps)
    want, want_inv = oracle.rmsnorm_silu_f64(c.x.float().numpy(), c.gamma.float().numpy(), c.eps)
    ulps = bf16_ulps(y, want)
    print(f"C2 norm bf16: max_ulp={ulps.max()} frac_off_by_one={np.mean(ulps > 0):.2e}", flush=True)
    assert ulps.max() <= 1
    np.testing.assert_allclose(inv.cpu().numpy(), want_inv, rtol=2e-6)


def test_config3_norm_sampled_within_one_bf16_ulp(device):
    g = torch.Generator().manual_seed(1003)
    h = (0.5 * torch.randn((131072, 1024), generator=g)).to(torch.bfloat16)
    gamma = (1 + 0.02 * torch.randn((1024,), generator=g)).to(torch.bfloat16)
    y, _ = core.rmsnorm_silu_forward(h.to(device), gamma.to(device), 1e-6)
    rows = torch.randperm(131072, generator=g)[:8192]
    want, _ = oracle.rmsnorm_silu_f64(h[rows].float().numpy(), gamma.float().numpy())
    assert bf16_ulps(y[rows.to(device)], want).max() <= 1
