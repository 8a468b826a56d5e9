"""``ttt_e2e.meta`` import path; see testtimeideas_amd.ttt_e2e.meta."""
from testtimeideas_amd.ttt_e2e.meta import inner_update, meta_step  # noqa: F401
