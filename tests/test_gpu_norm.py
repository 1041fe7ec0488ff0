"""GPU parity of the RMSNorm kernels (``llattn_rmsnorm_fwd/bwd``) against torch's ``F.rms_norm`` in float64.

Floating-point kernel: compared with a float64 torch reference of the same op on the same inputs --
fp32 storage within 1e-4 (max-abs scaled by max(1, max|ref|)), bf16 storage within 2e-2 max-abs and 1e-2
mean-relative.  The bf16 cases feed the reference the bf16-rounded inputs the kernel reads.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from gpu_helpers import assert_bf16_close, assert_fp32_close, require_cuda

pytestmark = pytest.mark.gpu

SHAPES = [(7, 64), (1, 1408), (513, 1000), (64, 4096), (300, 4), (2048, 1408)]


def _ref(x, w, dy, eps):
    xd = x.detach().double().requires_grad_(True)
    wd = w.detach().double().requires_grad_(True)
    y = F.rms_norm(xd, (x.shape[-1],), wd, eps)
    y.backward(dy.double())
    return y.detach(), xd.grad, wd.grad


@pytest.mark.parametrize("M,D", SHAPES)
@pytest.mark.parametrize("xdt,ydt", [(torch.float32, torch.float32), (torch.float32, torch.bfloat16),
                                     (torch.bfloat16, torch.bfloat16)])
def test_rmsnorm_matches_torch(M, D, xdt, ydt):
    from llattn_amd.norm import _RMSNorm
    dev = require_cuda()
    g = torch.Generator(device=dev).manual_seed(M * 7 + D)
    x = (torch.randn(M, D, device=dev, generator=g) * 3.0 + 0.5).to(xdt)
    w = torch.randn(D, device=dev, generator=g) * 0.5 + 1.0
    dy = torch.randn(M, D, device=dev, generator=g).to(ydt)
    eps = 1e-6
    xg = x.clone().requires_grad_(True)
    wg = w.clone().requires_grad_(True)
    y = _RMSNorm.apply(xg, wg, eps, ydt)
    assert y.dtype == ydt and y.shape == (M, D)
    y.backward(dy)
    y_ref, dx_ref, dw_ref = _ref(x, w, dy, eps)
    close = assert_fp32_close if ydt == torch.float32 else assert_bf16_close
    close(y.detach().float().cpu().double().numpy(), y_ref.cpu().numpy(), "y")
    dx_close = assert_fp32_close if xdt == torch.float32 else assert_bf16_close
    assert xg.grad.dtype == xdt
    dx_close(xg.grad.float().cpu().double().numpy(), dx_ref.cpu().numpy(), "dx")
    assert_fp32_close(wg.grad.cpu().double().numpy(), dw_ref.cpu().numpy(), "dw")


def test_rmsnorm_backward_is_deterministic_at_lm_shape():
    from llattn_amd.norm import _RMSNorm
    dev = require_cuda()
    g = torch.Generator(device=dev).manual_seed(1)
    x = torch.randn(32768, 1408, device=dev, generator=g)
    w = torch.randn(1408, device=dev, generator=g)
    dy = torch.randn(32768, 1408, device=dev, generator=g).to(torch.bfloat16)
    outs = []
    for _ in range(2):
        xg, wg = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
        _RMSNorm.apply(xg, wg, 1e-6, torch.bfloat16).backward(dy)
        outs.append((xg.grad.clone(), wg.grad.clone()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    _, dx_ref, dw_ref = _ref(x[:512], w, dy[:512], 1e-6)
    assert_fp32_close(outs[0][0][:512].cpu().double().numpy(), dx_ref.cpu().numpy(), "dx rows")


def test_rms_norm_autocast_output_dtype():
    from llattn_amd.norm import rms_norm
    dev = require_cuda()
    x = torch.randn(4, 5, 64, device=dev)
    w = torch.ones(64, device=dev)
    assert rms_norm(x, w, 1e-6).dtype == torch.float32
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        y = rms_norm(x, w, 1e-6)
    assert y.dtype == torch.bfloat16 and y.shape == x.shape
