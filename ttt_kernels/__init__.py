"""Import name of the reference package, so callers written against
``ttt_kernels`` (``from ttt_kernels import triton_attention``,
``from ttt_kernels.triton_attention import TritonAttentionFn``) run unchanged.
As in the reference's ttt_kernels/__init__.py:1-3, the submodule is imported
first and the package attribute ``triton_attention`` is then the function.
The implementation lives in ``testtimeideas_amd.ttt_kernels``."""
from . import backward_stubs  # noqa: F401
from .triton_attention import triton_attention

__all__ = ["triton_attention"]
