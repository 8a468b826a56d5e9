"""The reference's TTT model (``cloud_ttt_e2e/ttt_e2e``) on the HIP attention:
``GradGradAttentionFn`` with an additive mask, ``WindowedSelfAttention``
(whose chunked window runs as one problem with a structured mask), and, as
the callers of the attention, the model (``model``), its meta-learning step
(``meta``) and its synthetic key-value data (``data``)."""
from .attention import GradGradAttentionFn, WindowedSelfAttention, gradgrad_attention, windowed_attention
from .utils import local_window_mask, make_window_mask

__all__ = ["GradGradAttentionFn", "WindowedSelfAttention", "gradgrad_attention", "windowed_attention",
           "make_window_mask", "local_window_mask"]
