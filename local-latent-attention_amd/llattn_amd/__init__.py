"""MI355X-native (gfx950 HIP) local+latent attention: drop-in for the reference's fused block.

Public surface:

* :class:`LocalLatentAttentionTriton` -- the attention module (reference
  llattn_triton.py:33-176 surface, reference models.py:61-462 math);
* :class:`LLAttnFunction` -- the autograd op surface (reference kernels/llattn_op.py:184-238);
* :func:`build_attention` -- the dispatcher (reference models.py:465-488);
* :func:`pool` -- segment pooling op.
"""
from ._lib import DIV_COUNT, DIV_ONE, DIV_SEG, Layout, resolve_layout
from .config import ModelConfig, build_attention
from .module import LocalLatentAttentionHIP, LocalLatentAttentionTriton
from .ops import LLAttnCore, LLAttnFunction, pool

__all__ = [
    "DIV_COUNT", "DIV_ONE", "DIV_SEG", "Layout", "resolve_layout", "ModelConfig", "build_attention",
    "LocalLatentAttentionHIP", "LocalLatentAttentionTriton", "LLAttnCore", "LLAttnFunction", "pool",
]
