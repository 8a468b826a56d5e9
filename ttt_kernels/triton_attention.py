"""``ttt_kernels.triton_attention`` import path; see testtimeideas_amd.ttt_kernels.triton_attention."""
from testtimeideas_amd.ttt_kernels.triton_attention import (  # noqa: F401
    BWD_MODES, RECOMPUTE_MODES, SAVE_P_MODES, TritonAttentionFn, mode_kind, triton_attention)
from testtimeideas_amd.ttt_kernels import backward_stubs  # noqa: F401
