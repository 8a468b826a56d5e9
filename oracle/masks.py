"""Masks and the chunked window loop of the reference's TTT model, restated
in numpy float64 — TEST INFRASTRUCTURE ONLY.

  window_bias(T, W)           make_window_mask (cloud_ttt_e2e/ttt_e2e/utils.py:40-54):
                              0 where key j <= query i and i - j < W, else -inf
                              (W None: causal only).
  local_chunk_bias(qs, qe, ks, ke, W)
                              _local_window_mask (attention.py:56-69) for absolute
                              query rows qs..qe-1 and key rows ks..ke-1.
  chunked_loop(q, k, v, W, ...)
                              WindowedSelfAttention.forward's attention for T > W
                              (attention.py:111-128): query chunks [s, e) of W rows,
                              keys [max(0, e - W), e), each chunk on its own with its
                              rectangular local mask; the outputs concatenated, and
                              the gradients of every chunk scattered back onto the
                              full q, k, v (the chunks share keys only through the
                              overlap of a last partial chunk).
  local_bias(T, W)            the same layout as one [T, T] mask: query i sees keys
                              from min(T, (i // W + 1) W) - W to i.
"""
from __future__ import annotations

from typing import Dict, Optional

import numpy as np

from . import closed_form


def local_chunk_bias(q_start: int, q_end: int, k_start: int, k_end: int, window: Optional[int]) -> np.ndarray:
    qi = np.arange(q_start, q_end)[:, None]
    kj = np.arange(k_start, k_end)[None, :]
    hidden = kj > qi
    if window is not None:
        hidden = hidden | (qi - kj >= window)
    return np.where(hidden, -np.inf, 0.0)


def window_bias(t: int, window: Optional[int]) -> np.ndarray:
    return local_chunk_bias(0, t, 0, t, window)


def local_bias(t: int, window: int) -> np.ndarray:
    i = np.arange(t)[:, None]
    j = np.arange(t)[None, :]
    lo = np.maximum(0, np.minimum(t, (i // window + 1) * window) - window)
    return np.where((j > i) | (j < lo), -np.inf, 0.0)


def chunks(t: int, window: int):
    """(start, end, kv_start) of each query chunk (attention.py:111-115)."""
    out = []
    for start in range(0, t, window):
        end = min(t, start + window)
        out.append((start, end, max(0, end - window)))
    return out


def chunked_loop(q, k, v, window: int, scale: float, do=None, gq=None, gk=None, gv=None) -> Dict[str, np.ndarray]:
    """O (and with do: dQ, dK, dV; with gq, gk, gv too: GQ, GK, GV, GdO) of
    the chunked loop, over [..., T, D] arrays."""
    q, k, v = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
    t = q.shape[-2]
    out = {"o": np.zeros_like(q)}
    names = []
    if do is not None:
        names = ["dq", "dk", "dv"]
        if gq is not None:
            names += ["gq", "gk", "gv", "gdo"]
    for n in names:
        out[n] = np.zeros_like(q)
    for start, end, kv in chunks(t, window):
        bias = local_chunk_bias(start, end, kv, end, window)
        qs, ks, vs = q[..., start:end, :], k[..., kv:end, :], v[..., kv:end, :]
        if gq is not None:
            r = closed_form.double_backward(qs, ks, vs, do[..., start:end, :], gq[..., start:end, :],
                                            gk[..., kv:end, :], gv[..., kv:end, :], False, scale, bias)
        elif do is not None:
            r = closed_form.backward(qs, ks, vs, do[..., start:end, :], False, scale, bias)
        else:
            r = closed_form.forward(qs, ks, vs, False, scale, bias)
        out["o"][..., start:end, :] = r["o"]
        for n in names:
            rows = slice(start, end) if n in ("dq", "gq", "gdo") else slice(kv, end)
            out[n][..., rows, :] += r[n]
    return out
