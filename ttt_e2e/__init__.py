"""Import name of the reference's TTT model package for its attention
(``from ttt_e2e.attention import GradGradAttentionFn, WindowedSelfAttention``,
``from ttt_e2e.utils import make_window_mask``).  The implementation lives in
``testtimeideas_amd.ttt_e2e``; the model, data and training code of the
reference package are not part of this library."""
