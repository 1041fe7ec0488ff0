"""Autograd ops over the gfx950 HIP kernels.

* :func:`pool` -- segment pooling (chunk means, zero-padded query-block means)
  with its broadcast backward.
* :class:`LLAttnCore` -- the fused core of one block: latent attention,
  ``r_out``, windowed local attention and the gate mix, reading q/k/v (and the
  token-wise latent queries) straight out of the packed projection output and
  returning its gradient as one packed tensor.
* :class:`LLAttnFunction` -- the reference op surface
  (``LLAttnFunction.apply(Q, K, V, GQ, GK, GV, gate_local_w, gate_remote_w,
  r_out_w, window, chunk_size, ...)``, reference kernels/llattn_op.py:184-238)
  with the semantics of the reference PyTorch path (models.py:61-462).

All device work is HIP kernels from ``libllattn_gfx950.so``; under bf16 autocast
``r_out`` runs on its MFMA GEMM as well.  Without autocast (the fp32 module, kept
for the fp32 parity gate) ``r_out`` is a torch fp32 product, like the block's other
fp32 projections.  Nothing here runs on the CPU: CPU tensors raise.
"""
from __future__ import annotations

import ctypes
import time

import torch

from . import _lib as L
from .gemm import input_grad_persistent, linear_f32, matmul_nn_f32, matmul_tn_f32
from .linear import input_grad, linear_fwd, weight_grad

_byref = ctypes.byref

# When set to a list, every C-ABI call appends (entry point, start event, end event, work) recorded on
# the stream the call launches on; a benchmark turns this on to time kernels inside its timed region.
# `work` is the call's algorithmic FLOPs (GEMMs) or bytes (column sums) when the caller states it.
EVENT_LOG = None


def _call(name: str, *args, work=None) -> None:
    fn = getattr(L.load(), name)
    if EVENT_LOG is None:
        rc = fn(*args)
    else:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        rc = fn(*args)
        end.record()
        EVENT_LOG.append((name, start, end, work))
    L.check(rc, name)


def _empty(shape, dtype, device):
    return torch.empty(shape, dtype=dtype, device=device)


def _aligned_f32(t: torch.Tensor) -> torch.Tensor:
    t = t.detach().to(torch.float32).contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def _contig(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


# ---------------------------------------------------------------------------
# pooling
# ---------------------------------------------------------------------------

def pool_fwd_into(x: torch.Tensor, out: torch.Tensor, seg: int, n_seg: int, divisor: int) -> None:
    """out[b, n] = sum of x[b, n*seg : (n+1)*seg] / divisor (x: [B, T, D], out: [B, n_seg, D])."""
    B, T, D = x.shape
    _call("llattn_pool_fwd", x.data_ptr(), x.stride(0), x.stride(1), out.data_ptr(), out.stride(0), out.stride(1),
          B, T, D, seg, n_seg, divisor, L.dtype_code(x.dtype), L.stream_ptr(x.device))


def pool_bwd_into(dpooled: torch.Tensor, dx: torch.Tensor, seg: int, n_seg: int, divisor: int,
                  accumulate: bool) -> None:
    B, T, D = dx.shape
    _call("llattn_pool_bwd", dpooled.data_ptr(), dpooled.stride(0), dpooled.stride(1), dx.data_ptr(),
          dx.stride(0), dx.stride(1), B, T, D, seg, n_seg, divisor, int(accumulate),
          L.dtype_code(dx.dtype), L.stream_ptr(dx.device))


class _Pool(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, seg, n_seg, divisor):
        L.require_gpu(x)
        x = _contig(x)
        B, T, D = x.shape
        out = _empty((B, n_seg, D), x.dtype, x.device)
        pool_fwd_into(x, out, seg, n_seg, divisor)
        ctx.meta = (seg, n_seg, divisor, T)
        return out

    @staticmethod
    def backward(ctx, g):
        seg, n_seg, divisor, T = ctx.meta
        g = _contig(g)
        B, _, D = g.shape
        dx = _empty((B, T, D), g.dtype, g.device)
        pool_bwd_into(g, dx, seg, n_seg, divisor, accumulate=False)
        return dx, None, None, None


def pool(x: torch.Tensor, seg: int, n_seg: int, divisor: int = L.DIV_COUNT) -> torch.Tensor:
    """Segment pooling of x [B, T, D] into [B, n_seg, D] (differentiable).

    ``divisor``: ``DIV_COUNT`` -- mean over the real tokens (``_pool_to_latents``,
    reference models.py:159-214); ``DIV_SEG`` -- sum / seg, the zero-padded mean of
    ``_pool_query_blocks`` (reference models.py:216-230); ``DIV_ONE`` -- sum.
    """
    return _Pool.apply(x, seg, n_seg, divisor)


# ---------------------------------------------------------------------------
# shared forward / backward of the core
# ---------------------------------------------------------------------------

class _Prof:
    """Optional per-stage wall clock (device-synchronised), as the reference's
    ``set_profile`` instrumentation does (reference models.py:131-157, 309-461)."""

    def __init__(self, enabled: bool, device):
        self.enabled = enabled
        self.device = device
        self.t = {}
        self._last = None

    def start(self):
        if self.enabled:
            torch.cuda.synchronize(self.device)
            self._last = time.perf_counter()

    def lap(self, key):
        if self.enabled:
            torch.cuda.synchronize(self.device)
            now = time.perf_counter()
            self.t[key] = self.t.get(key, 0.0) + (now - self._last) * 1000.0
            self._last = now


def _remote_heads(lay: L.Layout, dt) -> bool:
    """Whether ``r_out``'s output R [B, n_q, D] is stored split-head ([B][H][n_q][Dh] slabs): in bf16, where its
    persistent GEMM writes it so (latent width above 64, below 2 GiB).  Only the local-attention kernels read R,
    by strides, so each head of a sequence streams as one contiguous run."""
    return dt == torch.bfloat16 and lay.Lh * lay.Ldh > 64 and lay.Dh % 8 == 0 and \
        lay.B * lay.n_q * lay.H * lay.Dh * 2 < (1 << 31)


def grad_heads_ok(M: int, N: int, K: int, dh: int) -> bool:
    """Whether a bf16 input gradient ``dy [M, N] @ w [N, K]`` can be stored split-head with heads of ``dh``
    columns: on the persistent kernel with at least 224 output tiles of 256 x 256 (row-major it then runs there
    unsplit too, so both layouts hold the same bits; with fewer tiles a row-major product is split over k),
    below 2 GiB."""
    return input_grad_persistent(M, N, K) and dh % 8 == 0 and N > 64 and M * K * 2 < (1 << 31) and \
        ((M + 255) // 256) * ((K + 255) // 256) >= 224


def _latent_grad_heads(lay: L.Layout) -> bool:
    """Whether the bf16 gradient of the latent output [B, n_q, Ld] (``r_out``'s input gradient) is stored
    split-head, as [B][Lh][n_q][Ldh] slabs."""
    return grad_heads_ok(lay.B * lay.n_q, lay.H * lay.Dh, lay.Lh * lay.Ldh, lay.Ldh)


def _remote_view(lay: L.Layout, R: torch.Tensor, heads: bool) -> L.LlattnTensor:
    if heads:
        return L.view(R, lay.H * lay.n_q * lay.Dh, lay.Dh, lay.n_q * lay.Dh)
    return L.view(R, R.stride(0), R.stride(1), lay.Dh)


def _core_forward(lay: L.Layout, q, k, v, rq, gk, gv, gate_l, gate_r, r_w, r_b, dt, device, prof=None,
                  saved: bool = True):
    """Latent attention -> r_out -> local attention + gate.  q/k/v/rq/gk/gv are
    LlattnTensor views; returns (y, o_local, lse, w, lat, lse_lat, R).  ``saved=False`` (no backward
    follows): the kernels skip o_local, lse, w and the latent lse, returned as None (w is kept when
    profiling, for the gate mean)."""
    B, T, H, Dh, Lh, Ldh = lay.B, lay.T, lay.H, lay.Dh, lay.Lh, lay.Ldh
    D, Ld = H * Dh, Lh * Ldh
    per_head = gate_l.dim() == 2 and gate_l.shape[0] > 1
    shape = lay.shape(dt, per_head)
    stream = L.stream_ptr(device)
    if prof is not None:
        prof.start()
    lat = _empty((B, lay.n_q, Lh, Ldh), dt, device)
    lse_lat = _empty((B, Lh, lay.n_q), torch.float32, device) if saved else None
    _call("llattn_latent_fwd", _byref(shape), _byref(rq), _byref(gk), _byref(gv), _byref(L.view_bnhd(lat)),
          None if lse_lat is None else lse_lat.data_ptr(), stream)
    with torch.autocast(device_type="cuda", enabled=False):
        if dt == torch.bfloat16:
            rh = (lay.n_q, Dh, H) if _remote_heads(lay, dt) else None
            R = linear_fwd(lat.view(B * lay.n_q, Ld), r_w.to(dt), None if r_b is None else r_b.float(),
                           rh).view(B, lay.n_q, D)
        else:  # fp32: the fp32 GEMM
            R = linear_f32(lat.view(B * lay.n_q, Ld), _contig(r_w.detach().float()),
                           None if r_b is None else _contig(r_b.detach().float())).view(B, lay.n_q, D)
    if prof is not None:
        prof.lap("latent_attention_ms")
    y = _empty((B, T, H, Dh), dt, device)
    keep = saved or prof is not None
    # o_local is the op's own: head-major [B, H, T, Dh], so that a head's rows are one contiguous run
    ol = _empty((B, H, T, Dh), dt, device) if keep else None
    lse = _empty((B, H, T), torch.float32, device) if keep else None
    w = _empty((B, H, T), torch.float32, device) if keep else None
    _call("llattn_local_gate_fwd", _byref(shape), _byref(q), _byref(k), _byref(v),
          _byref(_remote_view(lay, R, _remote_heads(lay, dt))), gate_l.data_ptr(),
          gate_r.data_ptr(), _byref(L.view_bnhd(y)), None if ol is None else _byref(L.view_bhnd(ol)),
          None if lse is None else lse.data_ptr(), None if w is None else w.data_ptr(), stream)
    if prof is not None:
        prof.lap("local_attention_ms")
    return y, ol, lse, w, lat, lse_lat, R


def _core_backward(lay: L.Layout, dy, q, k, v, rq, gk, gv, gate_l, gate_r, r_w, has_rb, lat, lse_lat, R, ol, lse,
                   w, dq, dk, dv, drq, dgk, dgv, dt, device, r_wt=None):
    """Writes dq/dk/dv/drq/dgk/dgv (LlattnTensor views) and returns (dgate_l, dgate_r, dr_w, dr_b): the gate
    gradients per head ([H, Dh]) or, for a shared gate, already summed over heads ([Dh]); r_out's bias
    gradient comes from the local backward (the column sums of dremote).  ``dy``: [B, T, H, Dh] with any
    16-byte strides (packed rows or head slabs), Dh contiguous."""
    B, T, H, Dh, Lh, Ldh = lay.B, lay.T, lay.H, lay.Dh, lay.Lh, lay.Ldh
    D, Ld = H * Dh, Lh * Ldh
    per_head = gate_l.dim() == 2 and gate_l.shape[0] > 1
    shape = lay.shape(dt, per_head)
    stream = L.stream_ptr(device)
    drem = _empty((B, T, D), dt, device)
    dgl = _empty((H, Dh) if per_head else (Dh,), torch.float32, device)
    dgr = _empty((H, Dh) if per_head else (Dh,), torch.float32, device)
    dr_b = _empty((D,), torch.float32, device) if has_rb else None
    ws = _empty((L.workspace_bytes(shape, L.WS_LOCAL_BWD),), torch.uint8, device)
    _call("llattn_local_gate_bwd",
          _byref(shape), _byref(q), _byref(k), _byref(v), _byref(_remote_view(lay, R, _remote_heads(lay, dt))),
          gate_l.data_ptr(), gate_r.data_ptr(), _byref(L.view_bhnd(ol)), lse.data_ptr(), w.data_ptr(),
          _byref(L.view(dy, dy.stride(0), dy.stride(1), dy.stride(2))), _byref(dq), _byref(dk), _byref(dv),
          _byref(L.view(drem, drem.stride(0), drem.stride(1), Dh)), dgl.data_ptr(), dgr.data_ptr(),
          None if dr_b is None else dr_b.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    if lay.macro:
        dR = _empty((B, lay.n_q, D), dt, device)
        pool_fwd_into(drem, dR, lay.q_block, lay.n_q, L.DIV_ONE)
    else:
        dR = drem
    with torch.autocast(device_type="cuda", enabled=False):
        dR2 = dR.view(B * lay.n_q, D)
        # bf16: the latent output's gradient stored as [B][Lh][n_q][Ldh] slabs, so that the latent backward reads
        # each latent head of a sequence as one contiguous run
        lh = dt == torch.bfloat16 and _latent_grad_heads(lay)
        if dt == torch.bfloat16:
            dlat = input_grad(dR2, r_w.to(dt), w_t=r_wt, heads=(lay.n_q, Ldh, Lh) if lh else None)
        else:
            dlat = matmul_nn_f32(dR2, _contig(r_w.float()))
        dlat_v = L.view(dlat, Lh * lay.n_q * Ldh, Ldh, lay.n_q * Ldh) if lh else L.view_bnhd(dlat.view(B, lay.n_q, Lh, Ldh))
        if dt == torch.bfloat16:
            dr_w, _ = weight_grad(dR2, lat.view(B * lay.n_q, Ld), False)
        else:
            dr_w = matmul_tn_f32(dR2, lat.view(B * lay.n_q, Ld))
    ws2 = _empty((L.workspace_bytes(shape, L.WS_LATENT_BWD),), torch.uint8, device)
    _call("llattn_latent_bwd", _byref(shape), _byref(rq), _byref(gk), _byref(gv), lse_lat.data_ptr(),
          _byref(dlat_v), _byref(drq), _byref(dgk), _byref(dgv), ws2.data_ptr(), ws2.numel(), stream)
    return dgl, dgr, dr_w, dr_b


def _gate_grad(dg: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    return dg.reshape(like.shape).to(like.dtype)


# ---------------------------------------------------------------------------
# packed core used by the module
# ---------------------------------------------------------------------------

def _qkv_views(lay: L.Layout, qkv: torch.Tensor, token_rq: bool, heads: bool):
    """q, k, v (and, for token-wise latent queries, rq) views of the projection output ``qkv`` [B, T, 3D (+Ld)]:
    packed rows (``view(B, T, 3, H, Dh)``, reference models.py:315-316, 348-353) or, with ``heads``, split-head
    storage -- the 3H heads as ``[B][3H][T][Dh]`` slabs, then the latent queries as ``[B][Lh][T][Ldh]`` slabs."""
    B, T, H, Dh, Ldh = lay.B, lay.T, lay.H, lay.Dh, lay.Ldh
    D, Ld = H * Dh, lay.Lh * Ldh
    if not heads:
        sb, sn = qkv.stride(0), qkv.stride(1)
        q, k, v = (L.view(qkv, sb, sn, Dh, i * D) for i in range(3))
        return q, k, v, (L.view(qkv, sb, sn, Ldh, 3 * D) if token_rq else None)
    q, k, v = (L.view(qkv, 3 * H * T * Dh, Dh, T * Dh, i * H * T * Dh) for i in range(3))
    return q, k, v, (L.view(qkv, T * Ld, Ldh, T * Ldh, B * T * 3 * D) if token_rq else None)


def heads_layout_ok(lay: L.Layout, d_model: int, token_rq: bool) -> bool:
    """Whether the block's q|k|v projection can be stored split-head (``heads`` of :class:`LLAttnCore`): the
    GEMM writes it from its persistent kernel (d_model > 64), all of it below 2 GiB."""
    D = lay.H * lay.Dh
    width = 3 * D + (lay.Lh * lay.Ldh if token_rq else 0)
    return d_model > 64 and lay.Dh % 8 == 0 and lay.Ldh % 8 == 0 and width % 8 == 0 and \
        lay.B * lay.T * width * 2 < (1 << 31)


class LLAttnCore(torch.autograd.Function):
    """Fused core of ``LocalLatentAttention`` over packed projections.

    Inputs: ``qkv`` [B, T, 3D (+Ld)] -- q|k|v in ``view(B, T, 3, H, Dh)`` order
    (reference models.py:315) followed, when ``rq`` is None, by the token-wise
    latent queries ``rq_proj(x)`` [Ld]; ``rq`` [B, n_q, Ld] (macro-block
    queries) or None; ``gkgv`` [B, n_chunks, 2*Ld] = ``rkv_proj(pooled)``
    (reference models.py:333-342); the shared gate weights [1, Dh] (or per-head
    [H, Dh]); ``r_out`` weight [D, Ld] and bias [D].  Returns the gate-mixed
    heads [B, T, D] ready for the output projection (reference models.py:438).
    ``heads``: ``qkv`` is stored split-head (``project(..., heads=(T, Dh, 3H, Ldh))``); the gradient returned for
    it is a plain row-major [B, T, 3D (+Ld)] tensor either way.  ``dy_heads``: the gradient that the backward
    receives for the output is stored as [B][H][T][Dh] slabs in its [B, T, D] tensor (``project(y, out,
    grad_heads=(T, Dh, H))`` writes it so), so that the local backward reads each head as one contiguous run.
    """

    @staticmethod
    def forward(ctx, qkv, rq, gkgv, gate_l, gate_r, r_w, r_b, lay: L.Layout, prof=None, r_w_cast=None,
                saved: bool = True, heads: bool = False, dy_heads: bool = False):
        L.require_gpu(qkv, rq, gkgv)
        dt, device = qkv.dtype, qkv.device
        H, Dh, Lh, Ldh = lay.H, lay.Dh, lay.Lh, lay.Ldh
        D, Ld = H * Dh, Lh * Ldh
        qkv = _contig(qkv)
        width = 3 * D + (Ld if rq is None else 0)
        if tuple(qkv.shape) != (lay.B, lay.T, width):
            raise ValueError(f"qkv must be [B, T, {width}], got {tuple(qkv.shape)}")
        if rq is not None:
            rq = _contig(rq.to(dt))
            if tuple(rq.shape) != (lay.B, lay.n_q, Ld):
                raise ValueError(f"rq must be [B, {lay.n_q}, {Ld}], got {tuple(rq.shape)}")
        gkgv = _contig(gkgv.to(dt))
        if tuple(gkgv.shape) != (lay.B, lay.n_chunks, 2 * Ld):
            raise ValueError(f"gkgv must be [B, {lay.n_chunks}, {2 * Ld}], got {tuple(gkgv.shape)}")
        gl, gr = _aligned_f32(gate_l), _aligned_f32(gate_r)
        q, k, v, rqv = _qkv_views(lay, qkv, rq is None, heads)
        if rq is not None:
            rqv = L.view(rq, rq.stride(0), rq.stride(1), Ldh)
        gk = L.view(gkgv, gkgv.stride(0), gkgv.stride(1), Ldh)
        gv = L.view(gkgv, gkgv.stride(0), gkgv.stride(1), Ldh, Ld)
        # cast once (or given cast, with or without its transposed copy): the backward's input gradient reuses it
        r_wt = None
        if isinstance(r_w_cast, (tuple, list)):
            r_w_cast, r_wt = r_w_cast
        if r_w_cast is None or r_w_cast.dtype != dt:
            r_w_cast, r_wt = None, None
        r_wd = r_w_cast if r_w_cast is not None else r_w.detach().to(dt)
        y, ol, lse, w, lat, lse_lat, R = _core_forward(lay, q, k, v, rqv, gk, gv, gl, gr, r_wd, r_b, dt, device, prof,
                                                       saved=saved)
        if saved:
            ctx.save_for_backward(qkv, rq, gkgv, gl, gr, r_wd, r_wt, lat, lse_lat, R, ol, lse, w)
        ctx.lay, ctx.has_rb, ctx.packed, ctx.heads, ctx.dy_heads = lay, r_b is not None, rq is None, heads, dy_heads
        ctx.r_w_dtype = r_w.dtype
        ctx.gate_like = (gate_l, gate_r)
        ctx.r_b_dtype = None if r_b is None else r_b.dtype
        if prof is not None:
            prof.gate_mean = w
        return y.view(lay.B, lay.T, D)

    @staticmethod
    def backward(ctx, dy):
        qkv, rq, gkgv, gl, gr, r_w, r_wt, lat, lse_lat, R, ol, lse, w = ctx.saved_tensors
        lay = ctx.lay
        dt, device = qkv.dtype, qkv.device
        H, Dh, Lh, Ldh = lay.H, lay.Dh, lay.Lh, lay.Ldh
        D, Ld = H * Dh, Lh * Ldh
        if ctx.dy_heads:  # [B][H][T][Dh] slabs in the storage of a contiguous [B, T, D] tensor
            if dy.dtype != dt or not dy.is_contiguous() or tuple(dy.shape) != (lay.B, lay.T, D):
                raise ValueError("dy_heads: the output gradient must be the contiguous split-head tensor that its "
                                 f"consumer's backward wrote (got {dy.dtype}, {tuple(dy.shape)}, {dy.stride()})")
            dy = dy.view(lay.B, H, lay.T, Dh).permute(0, 2, 1, 3)
        else:
            dy = _contig(dy.to(dt)).view(lay.B, lay.T, H, Dh)
        q, k, v, rqv = _qkv_views(lay, qkv, rq is None, ctx.heads)
        if rq is not None:
            rqv = L.view(rq, rq.stride(0), rq.stride(1), Ldh)
        gk = L.view(gkgv, gkgv.stride(0), gkgv.stride(1), Ldh)
        gv = L.view(gkgv, gkgv.stride(0), gkgv.stride(1), Ldh, Ld)
        # the gradient in plain rows whatever the storage of qkv: the projection's backward GEMMs read it as
        # their row-major operand
        dqkv = torch.empty_like(qkv)
        dq, dk, dv, drq = _qkv_views(lay, dqkv, rq is None, False)
        if rq is None:
            drq_t = None
        else:
            drq_t = torch.empty_like(rq)
            drq = L.view(drq_t, drq_t.stride(0), drq_t.stride(1), Ldh)
        dgkgv = torch.empty_like(gkgv)
        dgk = L.view(dgkgv, dgkgv.stride(0), dgkgv.stride(1), Ldh)
        dgv = L.view(dgkgv, dgkgv.stride(0), dgkgv.stride(1), Ldh, Ld)
        dgl, dgr, dr_w, dr_b = _core_backward(lay, dy, q, k, v, rqv, gk, gv, gl, gr, r_w, ctx.has_rb, lat, lse_lat,
                                              R, ol, lse, w, dq, dk, dv, drq, dgk, dgv, dt, device, r_wt)
        gate_l, gate_r = ctx.gate_like
        return (dqkv, drq_t, dgkgv, _gate_grad(dgl, gate_l), _gate_grad(dgr, gate_r), dr_w.to(ctx.r_w_dtype),
                None if dr_b is None else dr_b.to(ctx.r_b_dtype), None, None, None, None, None, None)


# ---------------------------------------------------------------------------
# reference op surface
# ---------------------------------------------------------------------------

class LLAttnFunction(torch.autograd.Function):
    """Drop-in for the reference autograd op (reference kernels/llattn_op.py:184-238).

    ``LLAttnFunction.apply(Q, K, V, GQ, GK, GV, gate_local_w, gate_remote_w,
    r_out_w, window, chunk_size[, r_out_b, local_block_size, q_block])``

    Same leading positional arguments as the reference; the math is the
    reference PyTorch path's (models.py:61-462), so:

    * Q, K, V: [B, Nh, S, Dh] (any strides, Dh contiguous); GQ: [B, Lh, Q, Ldh]
      latent queries (Q = S token-wise, or ceil(S/q_block) macro-block
      queries); GK, GV: [B, Lh, Nc, Ldh] with Nc = ceil(S / chunk_size);
    * gate_local_w / gate_remote_w: [Nh, Dh] per-head or [1, Dh] shared (pass
      ``gate_local.weight`` to get the reference's shared gate; an
      ``expand(Nh, Dh)`` view of it also works and autograd sums the heads);
    * r_out_w: the full [Nh*Dh, Lh*Ldh] matrix, r_out_b its bias (optional);
    * local_block_size: the reference's local query block (default 256);
      q_block: latent query block (0/1 token-wise).

    Returns the gate-mixed heads as [B, Nh, S, Dh] (a permuted view of a
    [B, S, Nh, Dh] buffer, so ``out.permute(0, 2, 1, 3).reshape(B, S, D)`` is free).
    ``backward`` returns gradients for the nine tensors (and r_out_b) in their
    input dtypes.
    """

    @staticmethod
    def forward(ctx, Q, K, V, GQ, GK, GV, gate_local_w, gate_remote_w, r_out_w, window, chunk_size, r_out_b=None,
                local_block_size=256, q_block=0):
        L.require_gpu(Q, K, V, GQ, GK, GV)
        B, H, S, Dh = Q.shape
        _, Lh, nq, Ldh = GQ.shape
        n_chunks = GK.shape[2]
        if K.shape != Q.shape or V.shape != Q.shape:
            raise ValueError("Q, K, V must share the shape [B, Nh, S, Dh]")
        if GK.shape != GV.shape or GK.shape[:2] != (B, Lh) or GK.shape[3] != Ldh:
            raise ValueError("GK, GV must be [B, Lh, Nc, Ldh] matching GQ")
        if chunk_size <= 0 or n_chunks != -(-S // chunk_size):
            raise ValueError(f"GK has {n_chunks} latents but ceil(S / chunk_size) = {-(-S // max(chunk_size, 1))}")
        if window <= 0:
            raise ValueError("local_window must be positive")
        qb = min(S, q_block) if q_block > 1 else 1
        if nq != -(-S // qb):
            raise ValueError(f"GQ has {nq} queries; expected {-(-S // qb)} for q_block={q_block}")
        lay = L.Layout(B, S, H, Dh, Lh, Ldh, window, min(S, max(window, local_block_size)), chunk_size, n_chunks, qb, nq)
        dt, device = Q.dtype, Q.device
        Q, K, V, GQ, GK, GV = (_contig_last(t.to(dt)) for t in (Q, K, V, GQ, GK, GV))
        gl, gr = _aligned_f32(gate_local_w), _aligned_f32(gate_remote_w)
        y, ol, lse, w, lat, lse_lat, R = _core_forward(
            lay, L.view_bhnd(Q), L.view_bhnd(K), L.view_bhnd(V), L.view_bhnd(GQ), L.view_bhnd(GK), L.view_bhnd(GV),
            gl, gr, r_out_w, r_out_b, dt, device)
        ctx.save_for_backward(Q, K, V, GQ, GK, GV, gl, gr, r_out_w, lat, lse_lat, R, ol, lse, w)
        ctx.lay, ctx.has_rb = lay, r_out_b is not None
        ctx.like = (gate_local_w, gate_remote_w)
        ctx.r_b_dtype = None if r_out_b is None else r_out_b.dtype
        return y.permute(0, 2, 1, 3)

    @staticmethod
    def backward(ctx, dOut):
        Q, K, V, GQ, GK, GV, gl, gr, r_w, lat, lse_lat, R, ol, lse, w = ctx.saved_tensors
        lay = ctx.lay
        dt, device = Q.dtype, Q.device
        B, H, S, Dh = Q.shape
        dy = _contig_last(dOut.to(dt).permute(0, 2, 1, 3))  # [B, S, H, Dh], read by its strides
        dQ, dK, dV = (_empty((B, S, H, Dh), dt, device) for _ in range(3))
        dGQ = _empty((B, lay.n_q, lay.Lh, lay.Ldh), dt, device)
        dGK = _empty((B, lay.n_chunks, lay.Lh, lay.Ldh), dt, device)
        dGV = _empty((B, lay.n_chunks, lay.Lh, lay.Ldh), dt, device)
        dgl, dgr, dr_w, dr_b = _core_backward(
            lay, dy, L.view_bhnd(Q), L.view_bhnd(K), L.view_bhnd(V), L.view_bhnd(GQ),
            L.view_bhnd(GK), L.view_bhnd(GV), gl, gr, r_w, ctx.has_rb, lat, lse_lat, R, ol, lse, w,
            L.view_bnhd(dQ), L.view_bnhd(dK), L.view_bnhd(dV), L.view_bnhd(dGQ), L.view_bnhd(dGK), L.view_bnhd(dGV),
            dt, device)
        like_l, like_r = ctx.like
        t = lambda x: x.permute(0, 2, 1, 3)  # noqa: E731
        return (t(dQ), t(dK), t(dV), t(dGQ), t(dGK), t(dGV), _gate_grad(dgl, like_l), _gate_grad(dgr, like_r),
                dr_w.to(r_w.dtype), None, None, None if dr_b is None else dr_b.to(ctx.r_b_dtype), None, None)


def _contig_last(t: torch.Tensor) -> torch.Tensor:
    """Keep any strides whose innermost dimension is contiguous and 16-byte aligned; copy otherwise."""
    es = t.element_size()
    ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all((s * es) % 16 == 0 for s in t.stride()[:-1])
    return t if ok else t.contiguous()
