"""bf16 projections of the block with fp32 master weights (the autocast training path).

:func:`project` computes ``x @ cat(W_i)^T + cat(b_i)`` for one or more
``nn.Linear`` parameter pairs that read the same input (the block's ``qkv_proj``
and token-wise ``rq_proj``, reference models.py:315, 348) as ONE bf16 GEMM, and
its backward writes every weight gradient in fp32 straight from the gfx950
split-K MFMA kernel (:func:`llattn_amd.gemm.matmul_tn`), so no bf16 weight
gradient is materialised and cast.  It is what ``F.linear`` under
``torch.autocast(dtype=bfloat16)`` computes (bf16 operands, fp32 accumulation,
bf16 output), with the weight gradient accumulated in fp32 instead of being
rounded to bf16 first.
"""
from __future__ import annotations

import torch

from . import gemm

BF16 = torch.bfloat16
MAX_SEGS = 8  # LLATTN_CAST_MAX_SEGS


def pack_params(groups):
    """``groups``: ``[(tensors, dtype), ...]`` of fp32 parameters, or ``(tensors, torch.bfloat16, True)`` for a
    group of 2-D weights that also wants its transposed copy.  Returns one new contiguous tensor per group,
    ``torch.cat(tensors)`` converted to ``dtype`` (bf16: round to nearest even, as ``.to(torch.bfloat16)``), or
    for a transposed group the pair ``(cat, cat.t().contiguous())`` -- ``(cat, None)`` when a weight's rows or
    columns are not multiples of 8, which the tiled copy needs; all written by one ``llattn_cast_transposed``
    launch (per 8 arrays): the weight casts bf16 autocast makes once per forward, and the ``W^T`` copies that the
    input gradients run on (:func:`llattn_amd.gemm.input_grad`)."""
    import ctypes

    from . import _lib as L
    from .ops import _call
    outs, segs = [], []
    for group in groups:
        tensors, dtype = group[0], group[1]
        ts = [t.detach() for t in tensors]
        if any(t.shape[1:] != ts[0].shape[1:] for t in ts):
            raise ValueError("the tensors of one group must share their trailing dimensions")
        want_t = len(group) > 2 and group[2]
        pair = want_t
        if want_t and (dtype != BF16 or any(t.dim() != 2 for t in ts)):
            raise ValueError("transposed copies are made of 2-D weights cast to bf16")
        want_t = want_t and all(t.shape[0] % 8 == 0 and t.shape[1] % 8 == 0 for t in ts)
        lead = sum(t.shape[0] for t in ts)
        out = torch.empty((lead, *ts[0].shape[1:]), dtype=dtype, device=ts[0].device)
        out_t = None
        if want_t:
            out_t = torch.empty((ts[0].shape[1], lead), dtype=dtype, device=ts[0].device)
        o = 0
        for t in ts:
            if t.dtype != torch.float32 or not t.is_contiguous():
                t = t.float().contiguous()
            if want_t and t.data_ptr() % 16:
                t = t.clone()  # the tiled copy reads 16-byte rows
            n = t.shape[0]
            # segment i of W^T: columns o .. o + n of [cols, lead]
            tr = (out_t[:, o:].data_ptr(), lead, n) if want_t else (None, 0, 0)
            segs.append((t, out[o:o + n], t.numel(), L.dtype_code(dtype), *tr))
            o += n
        outs.append((out, out_t) if pair else out)
    L.require_gpu(*[sg[0] for sg in segs])
    for i in range(0, len(segs), MAX_SEGS):
        chunk = segs[i:i + MAX_SEGS]
        k = len(chunk)
        src = (ctypes.c_void_p * k)(*[sg[0].data_ptr() for sg in chunk])
        dst = (ctypes.c_void_p * k)(*[sg[1].data_ptr() for sg in chunk])
        n = (ctypes.c_int64 * k)(*[sg[2] for sg in chunk])
        dt = (ctypes.c_int32 * k)(*[sg[3] for sg in chunk])
        if any(sg[4] is not None for sg in chunk):
            tdst = (ctypes.c_void_p * k)(*[sg[4] for sg in chunk])
            tld = (ctypes.c_int64 * k)(*[sg[5] for sg in chunk])
            rows = (ctypes.c_int32 * k)(*[sg[6] for sg in chunk])
            _call("llattn_cast_transposed", k, src, dst, n, dt, tdst, tld, rows, L.stream_ptr(chunk[0][0].device))
        else:
            _call("llattn_cast", k, src, dst, n, dt, L.stream_ptr(chunk[0][0].device))
    return outs


def linear_fwd(x2: torch.Tensor, w: torch.Tensor, b32: torch.Tensor | None, heads=None) -> torch.Tensor:
    """bf16 ``x2 @ w^T + b`` (fp32 bias added before the bf16 rounding of the output) on the MFMA GEMM
    (``heads``: the output stored split-head, see :mod:`llattn_amd.gemm`)."""
    return gemm.linear(x2, w, b32, heads=heads)


def input_grad(dy2: torch.Tensor, w: torch.Tensor, rowadd=(), w_t: torch.Tensor | None = None,
               heads=None) -> torch.Tensor:
    """bf16 ``dy2 @ w`` (w [N, K] read row-major), plus the broadcast ``rowadd`` pooling gradients
    added in the GEMM's epilogue (:func:`llattn_amd.gemm.input_grad`; ``w_t``: ``w``'s transposed copy from
    :func:`pack_params`, if made; ``heads``: the output stored split-head)."""
    return gemm.input_grad(dy2, w, rowadd=rowadd, w_t=w_t, heads=heads)


def weight_grad(dy2: torch.Tensor, x2: torch.Tensor, bias_grad: bool = False):
    """fp32 ``dy2^T @ x2`` for bf16 ``dy2 [K, N]``, ``x2 [K, D]`` (K = tokens, any count), and with ``bias_grad``
    also the fp32 column sums of ``dy2`` (the bias gradient): returns ``(dW, db)``.  The bias gradient comes
    from the weight-gradient pass itself: ``dy2`` contracted against ones (:func:`llattn_amd.gemm.matmul_tn`)."""
    N = dy2.shape[1]
    if bias_grad:
        db = torch.empty((N,), dtype=torch.float32, device=dy2.device)
        return gemm.matmul_tn(dy2, x2, rowsum=db), db
    return gemm.matmul_tn(dy2, x2), None


class _Project(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, pools, packed, heads, grad_heads, *params):
        # packed: (bf16 weights, fp32 biases[, bf16 transposed weights]) already concatenated by pack_params,
        # or None
        ctx.set_materialize_grads(False)
        ws, bs = params[0::2], params[1::2]
        has_bias = bs[0] is not None
        K = x.shape[-1]
        rows = [w.shape[0] for w in ws]
        with torch.autocast(device_type="cuda", enabled=False):
            x2 = x.reshape(-1, K).to(BF16)
            if not x2.is_contiguous():
                x2 = x2.contiguous()
            wcat_t = None
            if packed is not None:
                wcat, bcat = packed[0], packed[1]
                wcat_t = packed[2] if len(packed) > 2 else None
            elif len(ws) == 1:
                wcat = ws[0].detach().to(BF16)
                b = bs[0]
                bcat = None if b is None else (b.detach() if b.dtype == torch.float32 and b.is_contiguous()
                                               and b.data_ptr() % 16 == 0 else b.detach().float().contiguous().clone())
            else:
                packs = pack_params([(ws, BF16)] + ([(bs, torch.float32)] if has_bias else []))
                wcat, bcat = packs[0], (packs[1] if has_bias else None)
            y = linear_fwd(x2, wcat, bcat, heads)
            pooled = []
            if pools:
                from . import _lib as L
                from .ops import _contig, pool_fwd_into
                xc = x2.view(x.shape) if x.dtype == BF16 else _contig(x)
                means = (L.DIV_COUNT, L.DIV_SEG)
                for seg, n_seg, divisor in pools:
                    # with every segment full, the token-count mean and the segment mean are the same values
                    # (one formula, sum * (1 / seg)): such a pooling is computed once and returned again as a
                    # view, which keeps its gradient apart from the first one's
                    twin = next((p for p, (s2, n2, d2) in zip(pooled, pools) if (s2, n2) == (seg, n_seg)
                                 and n_seg * seg <= x.shape[1] and d2 in means and divisor in means), None)
                    if twin is not None:
                        pooled.append(twin.view(twin.shape))
                        continue
                    p = torch.empty((x.shape[0], n_seg, K), dtype=x.dtype, device=x.device)
                    pool_fwd_into(xc, p, seg, n_seg, divisor)
                    pooled.append(p)
        ctx.save_for_backward(x2, wcat, wcat_t)
        ctx.meta = (tuple(x.shape[:-1]), rows, has_bias, [w.dtype for w in ws], [None if b is None else b.dtype
                                                                                 for b in bs], x.dtype, tuple(pools))
        ctx.grad_heads = grad_heads
        return (y.view(*x.shape[:-1], sum(rows)), *pooled)

    @staticmethod
    def backward(ctx, dy, *dpooled):
        x2, wcat, wcat_t = ctx.saved_tensors
        lead, rows, has_bias, wdt, bdt, xdt, pools = ctx.meta
        N = sum(rows)
        K = x2.shape[1]
        dx = dw = db = None
        with torch.autocast(device_type="cuda", enabled=False):
            if dy is not None:
                dy2 = dy.reshape(-1, N).to(BF16)
                if not dy2.is_contiguous():
                    dy2 = dy2.contiguous()
                if ctx.needs_input_grad[0]:
                    # the poolings' gradients (bf16) join the input gradient in the GEMM's epilogue
                    fuse = xdt == BF16 and len(lead) == 2 and all(g is None or g.dtype == BF16 for g in dpooled)
                    rowadd = []
                    if fuse:
                        from .ops import _contig
                        for g, (seg, n_seg, divisor) in zip(dpooled, pools):
                            if g is not None:
                                rowadd.append((_contig(g).view(-1, K), lead[1], seg, n_seg, divisor))
                        dpooled = ()
                    dx = input_grad(dy2, wcat, rowadd, wcat_t, heads=ctx.grad_heads).view(*lead, K).to(xdt)
                dw, db = weight_grad(dy2, x2, has_bias)
            if ctx.needs_input_grad[0] and any(g is not None for g in dpooled):
                # pooling backward accumulates straight into the projection's input gradient
                from .ops import _contig, pool_bwd_into
                if dx is None:
                    dx = torch.zeros((*lead, K), dtype=xdt, device=x2.device)
                elif not dx.is_contiguous():
                    dx = dx.contiguous()
                for g, (seg, n_seg, divisor) in zip(dpooled, pools):
                    if g is not None:
                        pool_bwd_into(_contig(g.to(xdt)), dx, seg, n_seg, divisor, accumulate=True)
        grads = []
        o = 0
        for n, wd, bd in zip(rows, wdt, bdt):
            grads.append(None if dw is None else dw[o:o + n].to(wd))
            grads.append(None if db is None else db[o:o + n].to(bd))
            o += n
        return (dx, None, None, None, None, *grads)


def project(x: torch.Tensor, *linears: torch.nn.Linear, pools=(), packed=None, heads=None, grad_heads=None):
    """bf16 ``x @ [W_1; W_2; ...]^T + [b_1; b_2; ...]`` (all layers share the input width); backward gives
    fp32 weight and bias gradients in the parameters' dtypes.  Every product (forward, input and weight
    gradient) runs on the gfx950 MFMA GEMM; shapes it does not take raise.

    ``pools``: ``(seg, n_seg, divisor)`` segment poolings of the same ``x [B, T, K]`` (as
    :func:`llattn_amd.ops.pool`) returned after the projection, ``(y, pooled_1, ...)``; their backward adds
    into the projection's input gradient in place, so the block's input gradient is formed once.  Without
    ``pools`` the projection alone is returned.  ``packed``: ``(bf16 [sum N_i, K] weights, fp32 biases or None)``
    already cast and concatenated (:func:`pack_params`), so a caller casts all its weights in one launch; a
    third entry, the bf16 ``[K, sum N_i]`` transposed weights (or None), feeds the input gradient.
    ``heads``: ``(T, dh, n[, tail_dh])`` -- the output ``[B, T, N]`` is stored split-head (its first ``n * dh``
    columns as ``[B][n][T][dh]`` slabs, the rest after them, packed or as slabs of ``tail_dh`` columns;
    :mod:`llattn_amd.gemm`), for a consumer that reads it by strides (:class:`llattn_amd.ops.LLAttnCore`); its
    gradient comes back as a plain row-major tensor.  ``grad_heads``: the input gradient (bf16, on the
    persistent kernel's route of :func:`llattn_amd.gemm.input_grad`, no poolings) is stored split-head that way
    instead, for a producer of ``x`` whose backward reads its output gradient by strides (``dy_heads`` of
    :class:`llattn_amd.ops.LLAttnCore`)."""
    params = []
    for lin in linears:
        params += [lin.weight, lin.bias]
    if grad_heads is not None and pools:
        raise ValueError("grad_heads: a split-head input gradient takes no pooling gradients")
    out = _Project.apply(x, tuple(pools), packed, heads, grad_heads, *params)
    return out if pools else out[0]


class _ProjectF32(torch.autograd.Function):
    """fp32 ``x @ cat(W_i)^T + cat(b_i)`` with its gradients on ``llattn_gemm_f32``: the fp32 module's
    projections (reference models.py:80-84, 315, 333-353, 395, 462 without autocast)."""

    @staticmethod
    def forward(ctx, x, *params):
        ctx.set_materialize_grads(False)
        ws, bs = params[0::2], params[1::2]
        has_bias = bs[0] is not None
        K = x.shape[-1]
        rows = [w.shape[0] for w in ws]
        x2 = x.reshape(-1, K)
        if x2.dtype != torch.float32 or not x2.is_contiguous():
            x2 = x2.float().contiguous()
        # one copy kernel concatenates the projections that share the input (llattn_cast, fp32 -> fp32)
        groups = [(ws, torch.float32)] + ([(bs, torch.float32)] if has_bias else [])
        if len(ws) == 1 and all(t.is_contiguous() and t.dtype == torch.float32 for t in (ws[0], bs[0]) if t is not None):
            wcat, bcat = ws[0].detach(), (bs[0].detach() if has_bias else None)
        else:
            packs = pack_params(groups)
            wcat, bcat = packs[0], (packs[1] if has_bias else None)
        y = gemm.linear_f32(x2, wcat, bcat)
        ctx.save_for_backward(x2, wcat)
        ctx.meta = (tuple(x.shape[:-1]), rows, has_bias, [w.dtype for w in ws],
                    [None if b is None else b.dtype for b in bs], x.dtype)
        return y.view(*x.shape[:-1], sum(rows))

    @staticmethod
    def backward(ctx, dy):
        x2, wcat = ctx.saved_tensors
        lead, rows, has_bias, wdt, bdt, xdt = ctx.meta
        N, K = sum(rows), x2.shape[1]
        if dy is None:
            return (None, *([None] * (2 * len(rows))))
        dy2 = dy.reshape(-1, N)
        if dy2.dtype != torch.float32 or not dy2.is_contiguous():
            dy2 = dy2.float().contiguous()
        dx = gemm.matmul_nn_f32(dy2, wcat).view(*lead, K).to(xdt) if ctx.needs_input_grad[0] else None
        db = torch.empty((N,), dtype=torch.float32, device=dy2.device) if has_bias else None
        dw = gemm.matmul_tn_f32(dy2, x2, rowsum=db)
        grads = []
        o = 0
        for n, wd, bd in zip(rows, wdt, bdt):
            grads.append(dw[o:o + n].to(wd))
            grads.append(None if db is None else db[o:o + n].to(bd))
            o += n
        return (dx, *grads)


def project_f32(x: torch.Tensor, *linears: torch.nn.Linear) -> torch.Tensor:
    """fp32 ``x @ [W_1; W_2; ...]^T + [b_1; b_2; ...]`` for ``nn.Linear`` layers that read the same input; every
    product of the forward and the backward runs on ``llattn_gemm_f32`` (GPU only)."""
    params = []
    for lin in linears:
        params += [lin.weight, lin.bias]
    return _ProjectF32.apply(x, *params)

