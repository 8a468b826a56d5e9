"""Import name of the reference package, so callers written against
``ttt_kernels`` (``from ttt_kernels import triton_attention``,
``from ttt_kernels.triton_attention import TritonAttentionFn``) run unchanged.
The implementation lives in ``testtimeideas_amd.ttt_kernels``."""
from testtimeideas_amd.ttt_kernels import backward_stubs  # noqa: F401
from testtimeideas_amd.ttt_kernels.triton_attention import triton_attention

__all__ = ["triton_attention"]
