"""``ttt_kernels.backward_stubs`` import path; see testtimeideas_amd.ttt_kernels.backward_stubs."""
from testtimeideas_amd.ttt_kernels.backward_stubs import (  # noqa: F401
    TritonDqDkFn, TritonDvFn, TritonRowSumFn, triton_attn_bwd2, triton_attn_bwd2_dk, triton_attn_bwd2_dq,
    triton_attn_bwd2_dv, triton_attn_bwd_dk, triton_attn_bwd_dq, triton_attn_bwd_dqdk_from_p,
    triton_attn_bwd_dv, triton_attn_bwd_dv_from_p, triton_attn_rowsum_from_p)
