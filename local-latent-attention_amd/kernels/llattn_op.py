"""Drop-in for the reference module ``kernels.llattn_op`` (reference kernels/llattn_op.py:184-238).

``LLAttnFunction`` here runs the gfx950 HIP kernels with the semantics of the
reference PyTorch path; see :class:`llattn_amd.ops.LLAttnFunction`.
"""
from llattn_amd.ops import LLAttnFunction  # noqa: F401

__all__ = ["LLAttnFunction"]
