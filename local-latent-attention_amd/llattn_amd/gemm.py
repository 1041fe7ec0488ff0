"""Projection GEMMs on the gfx950 MFMA kernel (``llattn_gemm`` of the C ABI).

Three products cover every projection of the block and its backward without a
transpose copy (all operands bf16, fp32 accumulation):

* :func:`linear` -- ``y = x W^T (+ b)`` (``nn.Linear`` forward; reference models.py:315, 348, 395, 462);
* :func:`matmul_nn` -- ``dx = dy W`` (input gradient);
* :func:`matmul_tn` -- ``dW = dy^T x`` (weight gradient, fp32 output, split over tokens).

Each takes 2-D views whose innermost dimension is contiguous; outputs may be
passed in (``out=``) and accumulated into (``accumulate=True``).

Split-head output: ``linear(..., heads=(T, dh, n[, tail_dh]))`` stores the ``[tokens, width]`` product with its
first ``n * dh`` columns as per-sequence head slabs ``[batch][n][T][dh]`` followed by the other columns, packed
or (``tail_dh``) as slabs ``[batch][(width - n dh) / tail_dh][T][tail_dh]`` (``llattn_heads_layout`` of the C ABI).  The tensor returned is the ``[tokens, width]`` view of that storage;
it is read by strides (the local-attention kernels), not as a row-major matrix.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib as L


def _check2d(name: str, t: torch.Tensor) -> None:
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a 2-D view with a contiguous inner dimension, got shape "
                         f"{tuple(t.shape)} strides {t.stride()}")
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16 (got {t.dtype})")


def _heads(h) -> L.LlattnHeadsLayout:
    return L.LlattnHeadsLayout(0, 0, 0, 0) if h is None else L.LlattnHeadsLayout(*h)


def _run(M: int, N: int, K: int, A: torch.Tensor, a_trans: bool, B: torch.Tensor, b_trans: bool, C: torch.Tensor,
         bias: torch.Tensor | None, accumulate: bool, split_k: int = 0, rowsum: torch.Tensor | None = None,
         rowadd=(), act: int = 0, aux: torch.Tensor | None = None, c_heads=None) -> None:
    L.require_gpu(A, B, C)
    if rowsum is not None and (rowsum.dtype != torch.float32 or not rowsum.is_contiguous() or rowsum.numel() != M):
        raise ValueError(f"rowsum must be a contiguous fp32 vector of {M} elements")
    if C.dim() != 2 or C.stride(1) != 1 or C.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("output must be a 2-D bf16 / fp32 view with a contiguous inner dimension")
    if bias is not None and (bias.dtype != torch.float32 or not bias.is_contiguous() or bias.numel() != N):
        raise ValueError(f"bias must be a contiguous fp32 vector of {N} elements")
    desc = L.LlattnGemmDesc(M, N, K, int(a_trans), int(b_trans), A.data_ptr(), A.stride(0), B.data_ptr(),
                            B.stride(0), C.data_ptr(), C.stride(0), L.dtype_code(C.dtype), int(accumulate),
                            None if bias is None else bias.data_ptr(), split_k,
                            None if rowsum is None else rowsum.data_ptr())
    if len(rowadd) > 2:
        raise ValueError("at most two row addends")
    if act:
        if aux is None or aux.dtype != torch.bfloat16 or aux.dim() != 2 or aux.stride(1) != 1 \
                or tuple(aux.shape) != (M, N):
            raise ValueError(f"the activation's aux must be a bf16 [{M}, {N}] view with a contiguous inner dimension")
        L.require_gpu(aux)
        desc.act, desc.aux, desc.ld_aux = act, aux.data_ptr(), aux.stride(0)
    desc.c_heads = _heads(c_heads)
    for q, (rows, per_seq, seg, n_seg, divisor) in enumerate(rowadd):
        if rows.dtype != torch.bfloat16 or rows.stride(-1) != 1 or rows.shape[-1] != N:
            raise ValueError(f"row addend {q} must be bf16 rows of {N} contiguous elements")
        desc.rowadd[q] = L.LlattnGemmRowadd(rows.data_ptr(), rows.stride(-2), per_seq, seg, n_seg, divisor)
    lib = L.load()
    nws = lib.llattn_gemm_workspace_size(ctypes.byref(desc))
    ws = torch.empty((max(nws, 1),), dtype=torch.uint8, device=C.device) if nws else None
    from .ops import _call
    _call("llattn_gemm", ctypes.byref(desc), None if ws is None else ws.data_ptr(), nws, L.stream_ptr(C.device),
          work=2 * M * N * K)


def linear(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None = None, out: torch.Tensor | None = None,
           accumulate: bool = False, heads=None, rowadd=()) -> torch.Tensor:
    """``x [M, K] @ w [N, K]^T (+ bias fp32 [N])`` -> bf16 ``[M, N]`` (``heads``: stored split-head; ``rowadd``:
    the broadcast row addends of :func:`matmul_nn`, on the persistent kernel only)."""
    _check2d("x", x)
    _check2d("w", w)
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"x is [{M}, {K}] but w is {tuple(w.shape)}")
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    _run(M, N, K, x, False, w, False, out, bias, accumulate, c_heads=heads, rowadd=rowadd)
    return out


def linear_gelu(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None = None):
    """With ``h = x [M, K] @ w [N, K]^T (+ bias)`` rounded to bf16: ``(gelu(h), gelu'(h))`` (exact GELU and its
    derivative) from one GEMM, both bf16 ``[M, N]``."""
    _check2d("x", x)
    _check2d("w", w)
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"x is [{M}, {K}] but w is {tuple(w.shape)}")
    g = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    gp = torch.empty_like(g)
    _run(M, N, K, x, False, w, False, g, bias, False, act=L.ACT_GELU, aux=gp)
    return g, gp


def matmul_nn_scaled(a: torch.Tensor, b: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """``bf16(a [M, K] @ b [K, N]) * s`` elementwise in bf16 (``s`` bf16 ``[M, N]``): with ``s = gelu'(h)`` from
    :func:`linear_gelu`, the input gradient of a projection whose input was ``gelu(h)``, through the GELU."""
    _check2d("a", a)
    _check2d("b", b)
    M, K = a.shape
    N = b.shape[1]
    if b.shape[0] != K:
        raise ValueError(f"a is [{M}, {K}] but b is {tuple(b.shape)}")
    out = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    _run(M, N, K, a, False, b, True, out, None, False, act=L.ACT_MUL_AUX, aux=s)
    return out


def matmul_nn(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor | None = None,
              accumulate: bool = False, rowadd=()) -> torch.Tensor:
    """``a [M, K] @ b [K, N]`` -> bf16 ``[M, N]`` (b read row-major, no transpose copy).  ``rowadd``: up to two
    ``(rows, rows_per_seq, seg, n_seg, divisor)`` -- bf16 ``[n_seq * n_seg, N]`` rows added to every output row of
    their segment before the rounding, as ``llattn_pool_bwd`` adds a pooling's gradient into its input gradient."""
    _check2d("a", a)
    _check2d("b", b)
    M, K = a.shape
    N = b.shape[1]
    if b.shape[0] != K:
        raise ValueError(f"a is [{M}, {K}] but b is {tuple(b.shape)}")
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    _run(M, N, K, a, False, b, True, out, None, accumulate, rowadd=rowadd)
    return out


def transpose(w: torch.Tensor) -> torch.Tensor:
    """bf16 ``w [R, C]`` -> a new contiguous ``[C, R]`` (``llattn_transpose``)."""
    _check2d("w", w)
    L.require_gpu(w)
    R, C = w.shape
    out = torch.empty((C, R), dtype=torch.bfloat16, device=w.device)
    from .ops import _call
    _call("llattn_transpose", w.data_ptr(), w.stride(0), R, C, out.data_ptr(), out.stride(0), L.stream_ptr(w.device),
          work=4 * R * C)
    return out


# input gradients with row addends through the transposed weight and the persistent kernel (else matmul_nn)
ROWADD_PERSISTENT = True


def input_grad_persistent(M: int, N: int, K: int, rowadd=()) -> bool:
    """Whether :func:`input_grad` of ``dy [M, N]`` and ``w [N, K]`` runs on the persistent kernel."""
    return (not rowadd or ROWADD_PERSISTENT) and M >= 4096 and K % 8 == 0 and N % 8 == 0 and N > 64


def input_grad(dy: torch.Tensor, w: torch.Tensor, rowadd=(), w_t: torch.Tensor | None = None,
               heads=None) -> torch.Tensor:
    """``dy [M, N] @ w [N, K]`` (+ the ``rowadd`` addends of :func:`matmul_nn`) -> bf16 ``[M, K]``, the input
    gradient of ``y = x w^T``.  For large M (:func:`input_grad_persistent`) as ``dy (w^T)^T`` on the persistent
    kernel with a transposed copy of ``w`` (both operands k-contiguous: plain LDS fragment reads, the epilogue
    overlapped with the next tile): ``w_t`` when the caller has it (``llattn_cast_transposed`` writes it with the
    weight cast), else made here; otherwise :func:`matmul_nn` (transposing fragment reads of ``w``).  All routes
    give the same bits.  ``heads``: the output stored split-head as :func:`linear` does (persistent route only)."""
    M, N = dy.shape
    K = w.shape[1]
    if input_grad_persistent(M, N, K, rowadd):
        if w_t is None:
            w_t = transpose(w)
        elif tuple(w_t.shape) != (K, N):
            raise ValueError(f"w_t is {tuple(w_t.shape)}, expected the transpose of w {tuple(w.shape)}")
        return linear(dy, w_t, rowadd=rowadd, heads=heads)
    if heads is not None:
        raise ValueError(f"a split-head input gradient needs the persistent kernel (M={M}, N={N}, K={K})")
    return matmul_nn(dy, w, rowadd=rowadd)


def matmul_tn(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor | None = None, accumulate: bool = False,
              split_k: int = 0, rowsum: torch.Tensor | None = None) -> torch.Tensor:
    """``a [K, M]^T @ b [K, N]`` -> fp32 ``[M, N]`` (weight gradients: K = tokens).  With ``rowsum`` (fp32 ``[M]``,
    overwritten) also ``a.sum(0)`` -- the bias gradient -- from the same pass: contracted against a column of ones
    in place of the unused column ``N`` of the last 256-wide tile, or, when ``N`` is a multiple of 256, by one
    more product per A fragment block in the first tile column."""
    _check2d("a", a)
    _check2d("b", b)
    K, M = a.shape
    N = b.shape[1]
    if b.shape[0] != K:
        raise ValueError(f"a is [{K}, {M}] but b is {tuple(b.shape)}")
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=a.device)
    _run(M, N, K, a, True, b, True, out, None, accumulate, split_k, rowsum)
    return out


def colsum(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 ``x.sum(0)`` of a bf16 ``[M, N]`` view (the bias gradient of a projection)."""
    _check2d("x", x)
    L.require_gpu(x)
    M, N = x.shape
    if out is None:
        out = torch.empty((N,), dtype=torch.float32, device=x.device)
    lib = L.load()
    nws = lib.llattn_colsum_workspace_size(M, N)
    ws = torch.empty((max(nws, 1),), dtype=torch.uint8, device=x.device)
    from .ops import _call
    _call("llattn_colsum", x.data_ptr(), x.stride(0), M, N, out.data_ptr(), ws.data_ptr(), nws, L.stream_ptr(x.device),
          work=M * N * 2 + N * 4)
    return out


# ---------------------------------------------------------------------------
# fp32 products (``llattn_gemm_f32``): the fp32 module's projections
# ---------------------------------------------------------------------------

def _check2d_f32(name: str, t: torch.Tensor) -> None:
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a 2-D view with a contiguous inner dimension, got shape "
                         f"{tuple(t.shape)} strides {t.stride()}")
    if t.dtype != torch.float32:
        raise ValueError(f"{name} must be float32 (got {t.dtype})")


def _run_f32(M: int, N: int, K: int, A: torch.Tensor, a_trans: bool, B: torch.Tensor, b_trans: bool,
             C: torch.Tensor, bias: torch.Tensor | None = None, accumulate: bool = False,
             rowsum: torch.Tensor | None = None) -> None:
    L.require_gpu(A, B, C)
    if C.dim() != 2 or C.stride(1) != 1 or C.dtype != torch.float32:
        raise ValueError("output must be a 2-D fp32 view with a contiguous inner dimension")
    if bias is not None and (bias.dtype != torch.float32 or not bias.is_contiguous() or bias.numel() != N):
        raise ValueError(f"bias must be a contiguous fp32 vector of {N} elements")
    if rowsum is not None and (rowsum.dtype != torch.float32 or not rowsum.is_contiguous() or rowsum.numel() != M):
        raise ValueError(f"rowsum must be a contiguous fp32 vector of {M} elements")
    desc = L.LlattnGemmDesc(M, N, K, int(a_trans), int(b_trans), A.data_ptr(), A.stride(0), B.data_ptr(),
                            B.stride(0), C.data_ptr(), C.stride(0), L.F32, int(accumulate),
                            None if bias is None else bias.data_ptr(), 0,
                            None if rowsum is None else rowsum.data_ptr())
    from .ops import _call
    _call("llattn_gemm_f32", ctypes.byref(desc), L.stream_ptr(C.device), work=2 * M * N * K)


def linear_f32(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 ``x [M, K] @ w [N, K]^T (+ bias [N])`` -> ``[M, N]`` (``nn.Linear`` in fp32)."""
    _check2d_f32("x", x)
    _check2d_f32("w", w)
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"x is [{M}, {K}] but w is {tuple(w.shape)}")
    out = torch.empty((M, N), dtype=torch.float32, device=x.device)
    _run_f32(M, N, K, x, False, w, False, out, bias)
    return out


def matmul_nn_f32(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """fp32 ``a [M, K] @ b [K, N]`` (an input gradient ``dy W``)."""
    _check2d_f32("a", a)
    _check2d_f32("b", b)
    M, K = a.shape
    N = b.shape[1]
    if b.shape[0] != K:
        raise ValueError(f"a is [{M}, {K}] but b is {tuple(b.shape)}")
    out = torch.empty((M, N), dtype=torch.float32, device=a.device)
    _run_f32(M, N, K, a, False, b, True, out)
    return out


def matmul_tn_f32(a: torch.Tensor, b: torch.Tensor, rowsum: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 ``a [K, M]^T @ b [K, N]`` (a weight gradient ``dy^T x``); with ``rowsum`` (fp32 ``[M]``,
    overwritten) also ``a.sum(0)``, the bias gradient, from the same pass."""
    _check2d_f32("a", a)
    _check2d_f32("b", b)
    K, M = a.shape
    N = b.shape[1]
    if b.shape[0] != K:
        raise ValueError(f"a is [{K}, {M}] but b is {tuple(b.shape)}")
    out = torch.empty((M, N), dtype=torch.float32, device=a.device)
    _run_f32(M, N, K, a, True, b, True, out, rowsum=rowsum)
    return out

