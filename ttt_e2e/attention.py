"""``ttt_e2e.attention`` import path; see testtimeideas_amd.ttt_e2e.attention."""
from testtimeideas_amd.ttt_e2e.attention import (  # noqa: F401
    GradGradAttentionFn, WindowedSelfAttention, gradgrad_attention, windowed_attention)
from testtimeideas_amd.ttt_e2e.utils import local_window_mask as _local_window_mask  # noqa: F401
