"""The LM's FeedForward ``w2(gelu(w1 x))`` (reference models.py:50-58) on the gfx950 MFMA GEMM under bf16
autocast, with the GELU in the GEMM epilogues:

* forward: one GEMM forms ``h = x W1^T + b1`` and writes ``gelu(h)`` (the input of ``w2``) and ``gelu'(h)``
  (what the backward multiplies by; the epilogue has both from one evaluation of Phi and phi), a second one
  ``y = gelu(h) W2^T + b2``;
* backward: the input gradient of ``w2`` leaves its GEMM already multiplied by ``gelu'(h)``, so no separate
  elementwise pass reads or writes the ``[tokens, d_ff]`` gradients; weight gradients in fp32 with the bias
  gradients from the same passes (or the column-sum kernel where the width does not allow it).

Numerics are those of the reference under bf16 autocast: bf16 operands, fp32 accumulation, ``h`` rounded to
bf16 before the exact (erf) GELU, ``gelu(h)`` rounded to bf16, the GELU backward on the bf16 upstream
gradient, except that ``gelu'(h)`` is kept in bf16 (one rounding more than autocast's backward makes) and
weight gradients are accumulated in fp32 instead of being rounded to bf16.
"""
from __future__ import annotations

import torch

from . import gemm
from .linear import pack_params, weight_grad

BF16 = torch.bfloat16


def _bias(b: torch.Tensor | None) -> torch.Tensor | None:
    if b is None:
        return None
    b = b.detach().float().contiguous()
    return b if b.data_ptr() % 16 == 0 else b.clone()


class _FeedForward(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w1, b1, w2, b2):
        lead, D = tuple(x.shape[:-1]), x.shape[-1]
        with torch.autocast(device_type="cuda", enabled=False):
            x2 = x.reshape(-1, D).to(BF16)
            if not x2.is_contiguous():
                x2 = x2.contiguous()
            # the autocast casts, one launch; w1 also transposed for the input gradient
            (w1b, w1t), w2b = pack_params([([w1], BF16, True), ([w2], BF16)])
            g, gp = gemm.linear_gelu(x2, w1b, _bias(b1))
            y = gemm.linear(g, w2b, _bias(b2))
        ctx.save_for_backward(x2, gp, g, w1b, w1t, w2b)
        ctx.meta = (lead, x.dtype, w1.dtype, w2.dtype, None if b1 is None else b1.dtype,
                    None if b2 is None else b2.dtype)
        return y.view(*lead, w2.shape[0])

    @staticmethod
    def backward(ctx, dy):
        x2, gp, g, w1b, w1t, w2b = ctx.saved_tensors
        lead, xdt, w1dt, w2dt, b1dt, b2dt = ctx.meta
        has_b1, has_b2 = b1dt is not None, b2dt is not None
        with torch.autocast(device_type="cuda", enabled=False):
            dy2 = dy.reshape(-1, dy.shape[-1]).to(BF16)
            if not dy2.is_contiguous():
                dy2 = dy2.contiguous()
            dh = gemm.matmul_nn_scaled(dy2, w2b, gp)         # (dy W2) * gelu'(h), bf16
            dw2, db2 = weight_grad(dy2, g, has_b2)           # fp32
            dx = gemm.input_grad(dh, w1b, w_t=w1t) if ctx.needs_input_grad[0] else None
            dw1, db1 = weight_grad(dh, x2, has_b1)
        return (None if dx is None else dx.view(*lead, x2.shape[1]).to(xdt), dw1.to(w1dt),
                None if db1 is None else db1.to(b1dt), dw2.to(w2dt), None if db2 is None else db2.to(b2dt))


def feed_forward(x: torch.Tensor, w1: torch.nn.Linear, w2: torch.nn.Linear) -> torch.Tensor:
    """bf16 ``w2(gelu(w1(x)))`` on the GEMM kernels (GPU only; widths multiples of 8)."""
    return _FeedForward.apply(x, w1.weight, w1.bias, w2.weight, w2.bias)
