"""``ttt_e2e.utils`` import path for the mask helpers; see testtimeideas_amd.ttt_e2e.utils."""
from testtimeideas_amd.ttt_e2e.utils import local_window_mask, make_window_mask  # noqa: F401
