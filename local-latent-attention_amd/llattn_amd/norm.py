"""RMSNorm of the residual stream on the gfx950 kernels (``llattn_rmsnorm_fwd/bwd`` of the C ABI).

:func:`rms_norm` computes ``F.rms_norm(x, (D,), weight, eps)`` (reference
models.py:40-47) in one pass over ``x``.  Under bf16 autocast it returns the
normalised rows in bf16 -- the dtype every consumer (the block's projections,
the feed-forward ``w1``) casts them to -- so no separate cast runs; the
backward takes that bf16 gradient and returns ``dx`` in ``x``'s dtype and the
weight gradient in fp32 (deterministic order, no atomics).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib as L


def _rows(t: torch.Tensor, D: int) -> torch.Tensor:
    t2 = t.reshape(-1, D)
    if t2.stride(1) != 1 or t2.data_ptr() % 16 or (t2.stride(0) * t2.element_size()) % 16:
        t2 = t2.contiguous()
        if t2.data_ptr() % 16:
            t2 = t2.clone()
    return t2


class _RMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, eps, out_dtype):
        L.require_gpu(x, weight)
        D = x.shape[-1]
        x2 = _rows(x, D)
        M = x2.shape[0]
        w = weight.detach().to(torch.float32).contiguous()
        y = torch.empty((M, D), dtype=out_dtype, device=x.device)
        rstd = torch.empty((M,), dtype=torch.float32, device=x.device)
        from .ops import _call
        _call("llattn_rmsnorm_fwd", x2.data_ptr(), L.dtype_code(x2.dtype), x2.stride(0), w.data_ptr(), M, D,
              ctypes.c_float(eps), y.data_ptr(), L.dtype_code(out_dtype), y.stride(0), rstd.data_ptr(), None, 0, 0,
              None, 0, L.stream_ptr(x.device), work=M * D * (x2.element_size() + y.element_size()) + 4 * M)
        ctx.save_for_backward(x2, w, rstd)
        ctx.meta = (tuple(x.shape), weight.dtype)
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy):
        x2, w, rstd = ctx.saved_tensors
        shape, wdt = ctx.meta
        M, D = x2.shape
        dy2 = _rows(dy, D)
        if dy2.dtype not in (torch.float32, torch.bfloat16):
            dy2 = dy2.float()
        dx = torch.empty_like(x2)
        dw = torch.empty((D,), dtype=torch.float32, device=x2.device)
        lib = L.load()
        nws = lib.llattn_rmsnorm_workspace_size(M, D)
        ws = torch.empty((nws,), dtype=torch.uint8, device=x2.device)
        from .ops import _call
        _call("llattn_rmsnorm_bwd", dy2.data_ptr(), L.dtype_code(dy2.dtype), dy2.stride(0), x2.data_ptr(),
              L.dtype_code(x2.dtype), x2.stride(0), rstd.data_ptr(), w.data_ptr(), M, D, dx.data_ptr(), dx.stride(0),
              dw.data_ptr(), None, 0, ws.data_ptr(), nws, L.stream_ptr(x2.device),
              work=M * D * (dy2.element_size() + 2 * x2.element_size()) + 4 * M)
        return dx.view(shape), dw.to(wdt), None, None


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``F.rms_norm(x, (D,), weight, eps)`` on the GPU kernels; bf16 output under bf16 autocast, else
    ``x``'s dtype.  Raises for tensors that are not on a GPU (there is no CPU path)."""
    bf16 = torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16
    out_dtype = torch.bfloat16 if bf16 else x.dtype
    return _RMSNorm.apply(x, weight, float(eps), out_dtype)


def _copy_as(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """``t`` in ``dtype`` as a tensor of its own: the two inputs of a sum get equal gradients, and autograd may
    accumulate into either one in place, so they must not share storage."""
    return t.to(dtype, copy=True)


class _AddRMSNorm(torch.autograd.Function):
    """``s = x + res`` (fp32) and ``y = rms_norm(s)`` in one pass; the backward adds the gradient arriving at ``s``
    through the residual stream to the norm's input gradient in the same pass."""

    @staticmethod
    def forward(ctx, x, res, weight, eps, out_dtype):
        L.require_gpu(x, res, weight)
        D = x.shape[-1]
        x2 = _rows(x, D)
        r2 = _rows(res, D)
        if r2.dtype not in (torch.float32, torch.bfloat16):
            r2 = r2.float()
        M = x2.shape[0]
        w = weight.detach().to(torch.float32).contiguous()
        s = torch.empty((M, D), dtype=torch.float32, device=x.device)
        y = torch.empty((M, D), dtype=out_dtype, device=x.device)
        rstd = torch.empty((M,), dtype=torch.float32, device=x.device)
        from .ops import _call
        _call("llattn_rmsnorm_fwd", x2.data_ptr(), L.F32, x2.stride(0), w.data_ptr(), M, D, ctypes.c_float(eps),
              y.data_ptr(), L.dtype_code(out_dtype), y.stride(0), rstd.data_ptr(), r2.data_ptr(),
              L.dtype_code(r2.dtype), r2.stride(0), s.data_ptr(), s.stride(0), L.stream_ptr(x.device),
              work=M * D * (4 + r2.element_size() + 4 + y.element_size()) + 4 * M)
        ctx.save_for_backward(s, w, rstd)
        ctx.meta = (tuple(x.shape), res.dtype, weight.dtype)
        return s.view(x.shape), y.view(x.shape)

    @staticmethod
    def backward(ctx, ds, dy):
        s2, w, rstd = ctx.saved_tensors
        shape, rdt, wdt = ctx.meta
        M, D = s2.shape
        dev = s2.device
        if dy is None:  # only the sum is used further on: its gradient passes through unchanged
            g = ds.reshape(M, D).float()
            return g.view(shape), _copy_as(g, rdt).view(shape), torch.zeros_like(w).to(wdt), None, None
        dy2 = _rows(dy, D)
        if dy2.dtype not in (torch.float32, torch.bfloat16):
            dy2 = dy2.float()
        dres = _rows(ds, D).float() if ds is not None else None
        if dres is not None and dres.data_ptr() % 16:
            dres = dres.clone()
        dx = torch.empty((M, D), dtype=torch.float32, device=dev)
        dw = torch.empty((D,), dtype=torch.float32, device=dev)
        lib = L.load()
        nws = lib.llattn_rmsnorm_workspace_size(M, D)
        ws = torch.empty((nws,), dtype=torch.uint8, device=dev)
        from .ops import _call
        _call("llattn_rmsnorm_bwd", dy2.data_ptr(), L.dtype_code(dy2.dtype), dy2.stride(0), s2.data_ptr(), L.F32,
              s2.stride(0), rstd.data_ptr(), w.data_ptr(), M, D, dx.data_ptr(), dx.stride(0), dw.data_ptr(),
              dres.data_ptr() if dres is not None else None, dres.stride(0) if dres is not None else 0,
              ws.data_ptr(), nws, L.stream_ptr(dev),
              work=M * D * (dy2.element_size() + 8 + (4 if dres is not None else 0)) + 4 * M)
        return dx.view(shape), _copy_as(dx, rdt).view(shape), dw.to(wdt), None, None


def add_rms_norm(x: torch.Tensor, res: torch.Tensor, weight: torch.Tensor, eps: float):
    """``s = x + res`` and ``F.rms_norm(s, (D,), weight, eps)`` in one pass over the rows: the residual add of an LM
    block followed by the next norm (reference models.py:499-502).  ``x`` fp32; ``res`` fp32 or bf16.  Returns
    ``(s, y)`` with ``y`` in bf16 under bf16 autocast, else fp32.  GPU only."""
    if x.dtype != torch.float32:
        raise ValueError("add_rms_norm: the residual stream x must be fp32")
    bf16 = torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16
    out_dtype = torch.bfloat16 if bf16 else torch.float32
    return _AddRMSNorm.apply(x, res, weight, float(eps), out_dtype)
