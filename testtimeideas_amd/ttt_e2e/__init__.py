"""Drop-ins for the attention of the reference's TTT model
(``cloud_ttt_e2e/ttt_e2e/attention.py``): ``GradGradAttentionFn`` with an
additive mask, and ``WindowedSelfAttention``, whose chunked window runs as one
problem with a structured mask."""
from .attention import GradGradAttentionFn, WindowedSelfAttention, gradgrad_attention, windowed_attention
from .utils import local_window_mask, make_window_mask

__all__ = ["GradGradAttentionFn", "WindowedSelfAttention", "gradgrad_attention", "windowed_attention",
           "make_window_mask", "local_window_mask"]
