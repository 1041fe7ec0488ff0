"""Drop-in replacement for the reference module ``llattn_triton`` (reference llattn_triton.py).

The reference dispatcher imports ``llattn_triton.LocalLatentAttentionTriton`` by
module name (reference models.py:466-479); putting this directory on
``sys.path`` ahead of the reference makes it load the gfx950 HIP block.
"""
from llattn_amd.module import LocalLatentAttentionTriton  # noqa: F401

__all__ = ["LocalLatentAttentionTriton"]
