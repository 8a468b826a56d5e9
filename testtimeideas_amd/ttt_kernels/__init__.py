"""Reference-compatible surface: ``from ttt_kernels import triton_attention``
(reference: ttt_kernels/__init__.py:1-3)."""
from .triton_attention import triton_attention

__all__ = ["triton_attention"]
