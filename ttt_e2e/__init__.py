"""The reference TTT model package's import name (cloud_ttt_e2e/ttt_e2e).

``attention`` and ``utils`` re-export the library's drop-in attention
(``testtimeideas_amd.ttt_e2e``: GradGradAttentionFn, WindowedSelfAttention,
make_window_mask).  ``model``, ``meta`` and ``data`` are the model, its
test-time-training meta step and its synthetic key-value data, written here
as the callers of that attention for the benchmark and the tests; they are
not part of the library package."""
