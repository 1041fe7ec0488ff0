"""Drop-in for the reference package ``kernels`` (reference kernels/__init__.py)."""
from .llattn_op import LLAttnFunction  # noqa: F401

__all__ = ["LLAttnFunction"]
