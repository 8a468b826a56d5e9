"""Additive masks of the reference's TTT model, as torch tensors on the
caller's device (0 where a key is visible, -inf where it is masked).  They
are what callers hand to ``GradGradAttentionFn``; the kernels never read them
when a structured window is given instead."""
from __future__ import annotations

from typing import Optional

import torch


def make_window_mask(seq_len: int, window_size: Optional[int], device, dtype) -> torch.Tensor:
    """[T, T]: query i sees keys j with i - window < j <= i (all j <= i when
    window_size is None).  Reference: cloud_ttt_e2e/ttt_e2e/utils.py:40-54."""
    return local_window_mask(0, seq_len, 0, seq_len, window_size, device, dtype)


def local_window_mask(q_start: int, q_end: int, k_start: int, k_end: int, window_size: Optional[int], device,
                      dtype) -> torch.Tensor:
    """[q_end - q_start, k_end - k_start] for absolute query positions
    q_start.. and key positions k_start..: key j is visible to query i when
    j <= i and (no window, or i - j < window).  Reference:
    cloud_ttt_e2e/ttt_e2e/attention.py:56-69."""
    qi = torch.arange(q_start, q_end, device=device).unsqueeze(1)
    kj = torch.arange(k_start, k_end, device=device).unsqueeze(0)
    hidden = kj > qi
    if window_size is not None:
        hidden = hidden | (qi - kj >= window_size)
    out = torch.zeros(hidden.shape, device=device, dtype=dtype)
    return out.masked_fill(hidden, float("-inf"))
