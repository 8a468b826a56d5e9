"""``ttt_e2e.data`` import path; see testtimeideas_amd.ttt_e2e.data."""
from testtimeideas_amd.ttt_e2e.data import KVBatch, generate_kv_batch  # noqa: F401
