"""Tied LM head and cross entropy in row chunks, on the gfx950 kernels (``llattn_xent`` and ``llattn_gemm``).

The reference training step (reference models.py:516-517, 576; train.py:354-370)
computes ``logits = lm_head(norm(x))`` -- a bf16 ``[B*T, V]`` tensor under autocast
(2 GB at B16 T2048 V32000) -- then ``F.cross_entropy`` in fp32 (an fp32 copy, log
softmax, its backward) and ``logits.argmax(-1)`` for the accuracy metric.

:func:`lm_head_loss` gives the same loss and argmax without the full logits: for
each chunk of rows it computes the chunk's bf16 logits (``llattn_gemm``), one
``llattn_xent`` pass turns them into per-row losses, argmaxes and -- in place --
the bf16 logit gradient ``(softmax - onehot) / valid_rows``, and two more GEMMs
take the hidden-state gradient of the chunk and add the chunk's share of the
head weight gradient (fp32 accumulation over the chunks).  The gradients are
formed during the forward (for the unit upstream gradient of the loss; the
backward scales them by the actual one), so the logits buffer lives for one
chunk only.
"""
from __future__ import annotations

import torch

from . import _lib as L
from . import gemm

IGNORE_INDEX = -100


def xent_rows(logits: torch.Tensor, targets: torch.Tensor, ignore_index: int = IGNORE_INDEX,
              grad_scale: torch.Tensor | None = None, dlogits: torch.Tensor | None = None):
    """Per-row cross entropy of bf16 ``logits [R, V]`` against int64 ``targets [R]``: returns fp32 ``loss [R]``
    (``logsumexp - x[target]``, 0 for ignored rows) and int32 ``pred [R]`` (first argmax).  With ``dlogits``
    (bf16 ``[R, V]``, may be ``logits`` itself) and a device fp32 scalar ``grad_scale``, also writes
    ``(softmax - onehot) * grad_scale`` there."""
    L.require_gpu(logits, targets)
    if logits.dtype != torch.bfloat16 or logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("xent_rows: logits must be bf16 [R, V] with unit column stride")
    R, V = logits.shape
    t = targets.reshape(-1).to(torch.int64).contiguous()
    if t.numel() != R:
        raise ValueError(f"xent_rows: {t.numel()} targets for {R} rows")
    loss = torch.empty((R,), dtype=torch.float32, device=logits.device)
    pred = torch.empty((R,), dtype=torch.int32, device=logits.device)
    if dlogits is not None:
        if grad_scale is None or dlogits.dtype != torch.bfloat16 or dlogits.shape != logits.shape \
                or dlogits.stride(1) != 1:
            raise ValueError("xent_rows: dlogits must be bf16 like logits, with a grad_scale")
        grad_scale = grad_scale.reshape(()).to(torch.float32).contiguous()
    from .ops import _call
    _call("llattn_xent", logits.data_ptr(), logits.stride(0), R, V, t.data_ptr(), ignore_index, loss.data_ptr(),
          pred.data_ptr(), dlogits.data_ptr() if dlogits is not None else None,
          dlogits.stride(0) if dlogits is not None else 0,
          grad_scale.data_ptr() if dlogits is not None else None, L.stream_ptr(logits.device),
          work=R * V * (4 if dlogits is not None else 2))
    return loss, pred


class _HeadLoss(torch.autograd.Function):
    @staticmethod
    def forward(ctx, h, weight, targets, ignore_index, chunk_rows, grad_enabled):
        L.require_gpu(h, weight, targets)
        D = h.shape[-1]
        V = weight.shape[0]
        hb = h.detach().reshape(-1, D).to(torch.bfloat16).contiguous()
        N = hb.shape[0]
        wb = weight.detach().to(torch.bfloat16).contiguous()  # the autocast cast of the head weight
        t = targets.reshape(-1).to(torch.int64).contiguous()
        if t.numel() != N:
            raise ValueError(f"lm_head_loss: {t.numel()} targets for {N} rows")
        dev = h.device
        valid = (t != ignore_index).sum()
        scale = 1.0 / valid.to(torch.float32)  # mean over the rows that count (NaN loss when none do)
        # under no_grad needs_input_grad still reports the leaves' requires_grad: the caller's grad mode decides
        want_h, want_w = grad_enabled and ctx.needs_input_grad[0], grad_enabled and ctx.needs_input_grad[1]
        grad = want_h or want_w
        loss_rows = torch.empty((N,), dtype=torch.float32, device=dev)
        pred = torch.empty((N,), dtype=torch.int32, device=dev)
        dh = torch.empty_like(hb) if want_h else None
        dw = torch.empty((V, D), dtype=torch.float32, device=dev) if want_w else None
        step = max(64, chunk_rows // 64 * 64)
        logits = torch.empty((min(step, N), V), dtype=torch.bfloat16, device=dev)
        from .ops import _call
        for r0 in range(0, N, step):
            r1 = min(N, r0 + step)
            n = r1 - r0
            lc = logits[:n]
            gemm.linear(hb[r0:r1], wb, None, out=lc)
            _call("llattn_xent", lc.data_ptr(), V, n, V, t[r0:].data_ptr(), ignore_index, loss_rows[r0:].data_ptr(),
                  pred[r0:].data_ptr(), lc.data_ptr() if grad else None, V if grad else 0,
                  scale.data_ptr() if grad else None, L.stream_ptr(dev), work=n * V * (4 if grad else 2))
            if want_h:
                gemm.matmul_nn(lc, wb, out=dh[r0:r1])
            if want_w:
                gemm.matmul_tn(lc, hb[r0:r1], out=dw, accumulate=r0 > 0)
        loss = loss_rows.sum() * scale
        ctx.save_for_backward(dh, dw)
        ctx.shape = h.shape
        ctx.mark_non_differentiable(pred)
        return loss, pred.view(targets.shape)

    @staticmethod
    def backward(ctx, gl, _gpred):
        dh, dw = ctx.saved_tensors
        gh = (dh * gl.to(dh.dtype)).view(ctx.shape) if dh is not None else None
        gw = dw * gl if dw is not None else None
        return gh, gw, None, None, None, None


def head_supported(V: int, D: int) -> bool:
    """Vocabulary and hidden sizes the chunked head loss takes: multiples of 8 (16-byte rows for the GEMMs and
    the cross-entropy kernel), V at most 65536."""
    return V % 8 == 0 and D % 8 == 0 and 0 < V <= 65536


def lm_head_loss(h: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor, ignore_index: int = IGNORE_INDEX,
                 chunk_rows: int = 8192):
    """Mean cross entropy of ``h [..., D] @ weight [V, D]^T`` against ``targets [...]`` (``ignore_index`` rows
    excluded) and the first argmax of every logit row, without materialising the ``[rows, V]`` logits: chunks
    of ``chunk_rows`` rows (a multiple of 64).  Returns ``(loss, pred)``; ``pred`` has ``targets``' shape.
    V and D must be multiples of 8 and V at most 65536 (:func:`head_supported`).  GPU only."""
    D = h.shape[-1]
    V = weight.shape[0]
    if weight.dim() != 2 or weight.shape[1] != D:
        raise ValueError(f"lm_head_loss: weight {tuple(weight.shape)} does not match hidden size {D}")
    if not head_supported(V, D):
        raise ValueError(f"lm_head_loss: V={V} (multiple of 8, at most 65536) and D={D} (multiple of 8) unsupported")
    return _HeadLoss.apply(h, weight, targets, int(ignore_index), int(chunk_rows), torch.is_grad_enabled())
