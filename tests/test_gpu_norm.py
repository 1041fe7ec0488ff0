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


@pytest.mark.parametrize("M,D", [(7, 64), (513, 1000), (2048, 1408)])
@pytest.mark.parametrize("rdt", [torch.float32, torch.bfloat16])
def test_add_rms_norm_matches_torch(M, D, rdt):
    """Fused residual add + norm: s = x + res and y = rms_norm(s) forward; the backward with gradients arriving at
    both s (the residual stream) and y, against float64 autograd of the unfused ops."""
    print(f"add_rms_norm M={M} D={D} res={rdt}", flush=True)
    from llattn_amd.norm import add_rms_norm
    dev = require_cuda()
    g = torch.Generator(device="cpu").manual_seed(M + D)
    x = torch.randn(M, D, generator=g).to(dev)
    r = torch.randn(M, D, generator=g).to(dev).to(rdt)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(dev)
    ds, dy = torch.randn(M, D, generator=g).to(dev), torch.randn(M, D, generator=g).to(dev)
    xg, rg, wg = x.clone().requires_grad_(True), r.clone().requires_grad_(True), w.clone().requires_grad_(True)
    s, y = add_rms_norm(xg, rg, wg, 1e-6)
    (s * ds).sum().backward(retain_graph=True)
    (y * dy).sum().backward()
    xd, rd, wd = (t.detach().double().requires_grad_(True) for t in (x, r.float(), w))
    sd = xd + rd
    yd = F.rms_norm(sd, (D,), wd, 1e-6)
    ((sd * ds.double()).sum() + (yd * dy.double()).sum()).backward()
    assert s.dtype == torch.float32 and y.dtype == torch.float32
    c = lambda t: t.detach().float().cpu()  # noqa: E731
    assert_fp32_close(c(s), c(sd))
    assert_fp32_close(c(y), c(yd))
    assert_fp32_close(c(xg.grad), c(xd.grad))
    if rdt == torch.float32:
        assert_fp32_close(c(rg.grad), c(rd.grad))
    else:
        assert rg.grad.dtype == torch.bfloat16
        assert_bf16_close(c(rg.grad), c(rd.grad))
    assert_fp32_close(c(wg.grad), c(wd.grad))


def test_lm_fused_residual_norms_match_unfused():
    """The LM with every residual add inside the following norm gives the same loss and gradients as the
    unfused block order (same kernels, same fp32 sums): bitwise, forward and backward."""
    from llattn_amd.lm import build_model
    dev = require_cuda()
    torch.manual_seed(0)
    kw = dict(vocab_size=512, max_seq_len=256, d_model=192, n_heads=2, n_layers=2, d_ff=384, local_window=32,
              local_block_size=64, latent_tokens=8, latent_d_model=64, latent_heads=2)
    model = build_model(**kw).to(dev)
    inputs = torch.randint(0, 512, (2, 256), device=dev)
    targets = torch.randint(0, 512, (2, 256), device=dev)
    runs = []
    for fused in (True, False):
        model.fuse_residual_norms = fused
        model.zero_grad(set_to_none=True)
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            loss, _ = model.loss(inputs, targets)
            loss.backward()
        runs.append((loss.detach(), {n: p.grad.clone() for n, p in model.named_parameters()}))
    assert torch.equal(runs[0][0], runs[1][0])
    for n, g in runs[0][1].items():
        assert torch.equal(g, runs[1][1][n]), n
