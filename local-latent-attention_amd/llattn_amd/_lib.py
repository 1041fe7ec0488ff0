"""ctypes binding of the C ABI declared in ``include/llattn.h``.

This is the only place that touches the shared library.  Every call checks the
returned status and raises: ``ValueError`` for shape / dtype / layout /
unsupported-size errors, ``RuntimeError`` for workspace and launch errors.
There is no fallback: without the built library, or with tensors that are not
on a GPU, the op raises.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libllattn_gfx950.so"
ABI_VERSION = 8

OK, ERR_SHAPE, ERR_DTYPE, ERR_LAYOUT, ERR_UNSUPPORTED, ERR_WORKSPACE, ERR_LAUNCH = range(7)
F32, BF16 = 0, 1
DIV_COUNT, DIV_SEG, DIV_ONE = 0, 1, 2
ACT_NONE, ACT_GELU, ACT_MUL_AUX = 0, 1, 2
WS_LOCAL_BWD, WS_LATENT_BWD = 0, 1
NOALLOC_SCRATCH_BYTES = 8 << 20  # LLATTN_NOALLOC_SCRATCH_BYTES

_DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16}


class LlattnTensor(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("sb", ctypes.c_int64), ("sn", ctypes.c_int64), ("sh", ctypes.c_int64)]


class LlattnShape(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "B", "T", "H", "Dh", "Lh", "Ldh", "window", "block", "chunk", "n_chunks", "q_block", "n_q", "dtype",
        "gate_per_head")]


class LlattnGemmRowadd(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("ld", ctypes.c_int64), ("rows_per_seq", ctypes.c_int32),
                ("seg", ctypes.c_int32), ("n_seg", ctypes.c_int32), ("divisor", ctypes.c_int32)]


class LlattnHeadsLayout(ctypes.Structure):
    """Split-head storage of a token-row matrix (include/llattn.h llattn_heads_layout); T = 0: row-major."""
    _fields_ = [("T", ctypes.c_int32), ("dh", ctypes.c_int32), ("n", ctypes.c_int32), ("tail_dh", ctypes.c_int32)]


class LlattnGemmDesc(ctypes.Structure):
    _fields_ = [("M", ctypes.c_int32), ("N", ctypes.c_int32), ("K", ctypes.c_int32), ("a_trans", ctypes.c_int32),
                ("b_trans", ctypes.c_int32), ("A", ctypes.c_void_p), ("lda", ctypes.c_int64), ("B", ctypes.c_void_p),
                ("ldb", ctypes.c_int64), ("C", ctypes.c_void_p), ("ldc", ctypes.c_int64), ("c_dtype", ctypes.c_int32),
                ("accumulate", ctypes.c_int32), ("bias", ctypes.c_void_p), ("split_k", ctypes.c_int32),
                ("a_rowsum", ctypes.c_void_p), ("rowadd", LlattnGemmRowadd * 2), ("act", ctypes.c_int32),
                ("aux", ctypes.c_void_p), ("ld_aux", ctypes.c_int64), ("c_heads", LlattnHeadsLayout)]


_P = ctypes.c_void_p
_T = ctypes.POINTER(LlattnTensor)
_G = ctypes.POINTER(LlattnGemmDesc)
_S = ctypes.POINTER(LlattnShape)
_I32, _I64, _SZ = ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/llattn.h
SIGNATURES = {
    "llattn_abi_version": (_I32, []),
    "llattn_last_error": (ctypes.c_char_p, []),
    "llattn_workspace_size": (_SZ, [_S, _I32]),
    "llattn_pool_fwd": (_I32, [_P, _I64, _I64, _P, _I64, _I64, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _P]),
    "llattn_pool_bwd": (_I32, [_P, _I64, _I64, _P, _I64, _I64, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _P]),
    "llattn_latent_fwd": (_I32, [_S, _T, _T, _T, _T, _P, _P]),
    "llattn_latent_bwd": (_I32, [_S, _T, _T, _T, _P, _T, _T, _T, _T, _P, _SZ, _P]),
    "llattn_local_gate_fwd": (_I32, [_S, _T, _T, _T, _T, _P, _P, _T, _T, _P, _P, _P]),
    "llattn_local_gate_bwd": (_I32, [_S, _T, _T, _T, _T, _P, _P, _T, _P, _P, _T, _T, _T, _T, _T, _P, _P, _P, _P, _SZ,
                                     _P]),
    "llattn_local_gate_bwd_noalloc": (_I32, [_S, _T, _T, _T, _T, _P, _P, _T, _P, _P, _T, _T, _T, _T, _T, _P, _P, _P,
                                             _P]),
    "llattn_gemm_workspace_size": (_SZ, [_G]),
    "llattn_gemm": (_I32, [_G, _P, _SZ, _P]),
    "llattn_gemm_f32": (_I32, [_G, _P]),
    "llattn_colsum_workspace_size": (_SZ, [_I32, _I32]),
    "llattn_colsum": (_I32, [_P, _I64, _I32, _I32, _P, _P, _SZ, _P]),
    "llattn_cast": (_I32, [_I32, _P, _P, _P, _P, _P]),
    "llattn_cast_transposed": (_I32, [_I32, _P, _P, _P, _P, _P, _P, _P, _P]),
    "llattn_transpose": (_I32, [_P, _I64, _I32, _I32, _P, _I64, _P]),
    "llattn_rmsnorm_fwd": (_I32, [_P, _I32, _I64, _P, _I32, _I32, ctypes.c_float, _P, _I32, _I64, _P, _P, _I32, _I64,
                                  _P, _I64, _P]),
    "llattn_rmsnorm_workspace_size": (_SZ, [_I32, _I32]),
    "llattn_rmsnorm_bwd": (_I32, [_P, _I32, _I64, _P, _I32, _I64, _P, _P, _I32, _I32, _P, _I64, _P, _P, _I64, _P, _SZ,
                                  _P]),
    "llattn_xent": (_I32, [_P, _I64, _I32, _I32, _P, _I64, _P, _P, _P, _I64, _P, _P]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it is missing or stale."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"llattn HIP library not built ({LIB_PATH} missing); run __graft_entry__.build() "
                           "or `python -m llattn_amd._build` on a machine with ROCm hipcc")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    v = lib.llattn_abi_version()
    if v != ABI_VERSION:
        raise RuntimeError(f"llattn library ABI version {v} != expected {ABI_VERSION}; rebuild it")
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc == OK:
        return
    msg = load().llattn_last_error().decode(errors="replace")
    text = f"{what}: {msg}"
    if rc in (ERR_SHAPE, ERR_DTYPE, ERR_LAYOUT, ERR_UNSUPPORTED):
        raise ValueError(text)
    raise RuntimeError(text)


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise ValueError(f"llattn supports float32 and bfloat16 activations, got {dtype}") from None


def require_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError("llattn runs on MI355X (gfx950) GPUs only; got a tensor on "
                               f"{t.device} (there is no CPU path)")


def stream_ptr(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def view(t: torch.Tensor, sb: int, sn: int, sh: int, offset: int = 0) -> LlattnTensor:
    """A [b][n][h][d] view of ``t`` starting ``offset`` elements past its data pointer."""
    return LlattnTensor(t.data_ptr() + offset * t.element_size(), sb, sn, sh)


def view_bnhd(t: torch.Tensor) -> LlattnTensor:
    """View of a [B, N, H, d] tensor (d contiguous)."""
    assert t.dim() == 4 and t.stride(3) == 1
    return LlattnTensor(t.data_ptr(), t.stride(0), t.stride(1), t.stride(2))


def view_bhnd(t: torch.Tensor) -> LlattnTensor:
    """View of a [B, H, N, d] tensor (d contiguous), e.g. the reference op's [B, Nh, S, Dh]."""
    assert t.dim() == 4 and t.stride(3) == 1
    return LlattnTensor(t.data_ptr(), t.stride(0), t.stride(2), t.stride(1))


@dataclass(frozen=True)
class Layout:
    """Integer index maps of one call (all host-side; reference models.py:175-230, 249)."""

    B: int
    T: int
    H: int
    Dh: int
    Lh: int
    Ldh: int
    window: int
    block: int
    chunk: int
    n_chunks: int
    q_block: int
    n_q: int

    @property
    def macro(self) -> bool:
        return self.q_block > 1 or self.n_q != self.T

    def shape(self, dtype: torch.dtype, gate_per_head: bool = False) -> LlattnShape:
        return LlattnShape(self.B, self.T, self.H, self.Dh, self.Lh, self.Ldh, self.window, self.block, self.chunk,
                           self.n_chunks, self.q_block, self.n_q, dtype_code(dtype), int(gate_per_head))


def resolve_layout(B: int, T: int, d_model: int, n_heads: int, latent_d_model: int, latent_heads: int,
                   window: int, local_block_size: int, latent_tokens: int, latent_query_block_size: int) -> Layout:
    """Resolve sizes exactly as the reference forward does, raising the same errors.

    * ``seq_len must be positive`` / ``latent_tokens must be positive`` (reference models.py:171-177)
    * ``local_window must be positive`` (reference models.py:246-247)
    * chunk = ceil(T / min(latent_tokens, T)), latent count = ceil(T / chunk) (reference models.py:175-208)
    * local block = min(T, max(W, local_block_size)) (reference models.py:249)
    * macro-block queries only when latent_query_block_size > 1, block = min(T, qbs) (reference models.py:218, 343)
    """
    if T <= 0:
        raise ValueError("seq_len must be positive")
    target = min(latent_tokens, T)
    if target <= 0:
        raise ValueError("latent_tokens must be positive")
    if window <= 0:
        raise ValueError("local_window must be positive")
    if d_model % n_heads != 0:
        raise ValueError("d_model must be divisible by n_heads")
    if latent_d_model % latent_heads != 0:
        raise ValueError("latent_dim must be divisible by latent_heads")
    chunk = math.ceil(T / target)
    n_chunks = math.ceil(T / chunk)
    block = min(T, max(window, local_block_size))
    if latent_query_block_size > 1:
        q_block = min(T, latent_query_block_size)
        n_q = math.ceil(T / q_block)
    else:
        q_block, n_q = 1, T
    return Layout(B, T, n_heads, d_model // n_heads, latent_heads, latent_d_model // latent_heads, window, block,
                  chunk, n_chunks, q_block, n_q)


def workspace_bytes(shape: LlattnShape, kind: int) -> int:
    n = load().llattn_workspace_size(ctypes.byref(shape), kind)
    if n == 0:
        check(ERR_SHAPE, "llattn_workspace_size")
    return n
