"""The reference TTT model's attention (``cloud_ttt_e2e/ttt_e2e``) on the HIP
kernels: ``GradGradAttentionFn`` with an additive mask and
``WindowedSelfAttention``, whose chunked window runs as one problem with a
structured mask.  The model, its meta step and its data, the callers of this
attention, live outside the library package (top-level ``ttt_e2e``)."""
from .attention import GradGradAttentionFn, WindowedSelfAttention, gradgrad_attention, windowed_attention
from .utils import local_window_mask, make_window_mask

__all__ = ["GradGradAttentionFn", "WindowedSelfAttention", "gradgrad_attention", "windowed_attention",
           "make_window_mask", "local_window_mask"]
