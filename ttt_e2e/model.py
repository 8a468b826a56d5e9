"""``ttt_e2e.model`` import path; see testtimeideas_amd.ttt_e2e.model."""
from testtimeideas_amd.ttt_e2e.model import ModelConfig, PrefixBlock, SuffixBlock, TTTModel  # noqa: F401
