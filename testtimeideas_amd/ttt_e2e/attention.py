"""Attention of the reference's TTT model on the HIP kernels.

Reference module: ``cloud_ttt_e2e/ttt_e2e/attention.py``.

``GradGradAttentionFn.apply(q, k, v, attn_mask)`` (reference :21-53) computes
``softmax(q k^T / sqrt(d) + attn_mask) v`` (the reference's ``_attention``,
:9-18) for q ``[B,H,Lq,D]``, k and v ``[B,H,Lk,D]`` and an additive mask
broadcastable to ``[B,H,Lq,Lk]`` (or None).  Its backward is differentiable
whenever grad mode is on, as ``create_graph=True`` makes it, so
``torch.autograd.grad(..., create_graph=True)`` through it yields the exact
second derivative.  The reference decides with
``need_higher = grad_out.requires_grad`` (:34), which drops the second-order
terms when the incoming gradient is a constant even under
``create_graph=True``; grad mode does not.  The mask is a constant: it gets
no gradient (the reference returns None for it, :53).

``WindowedSelfAttention`` (reference :72-131) runs its window as one problem
with a structured mask (``windowed_attention``): for T > window the
reference's loop over query chunks of ``window`` rows, each attending
causally to the ``window`` keys that end with the chunk, becomes one launch
whose tiles outside each chunk's key range are skipped; for T <= window it is
causal attention, as the reference's ``make_window_mask`` is then.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn.functional as F
from torch import nn

from .. import _lib
from ..ttt_kernels.triton_attention import Layout, attn_backward, attn_forward


def _check(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    _lib.check_inputs(k, v)
    if q.device.type != "cuda":
        _lib.check_inputs(q)
    if q.dim() != 4 or q.shape[:2] != k.shape[:2] or q.size(-1) != k.size(-1):
        raise ValueError(f"q {tuple(q.shape)} does not match k {tuple(k.shape)} in B, H or D")
    if q.dtype != k.dtype or q.device != k.device:
        raise ValueError("all operands must share dtype and device")


def _kernel_bias(attn_mask: Optional[torch.Tensor], q: torch.Tensor, lq: int, lk: int) -> Optional[torch.Tensor]:
    """The mask as the kernels' [B,H,T,T] bias, T = max(Lq, Lk): with Lq < Lk
    the Lk - Lq padded query rows in front get zeros (any finite values do:
    those rows contribute nothing), with Lq > Lk the padded key columns at
    the end get -inf."""
    b, h = q.shape[:2]
    t = max(lq, lk)
    if attn_mask is None:
        if lq <= lk:
            return None
        m = torch.zeros((1, 1, 1, lk), dtype=q.dtype, device=q.device)
    else:
        m = attn_mask.detach()
        if m.dim() > 4:
            raise ValueError(f"attn_mask of shape {tuple(attn_mask.shape)} does not broadcast to [B, H, Lq, Lk]")
        while m.dim() < 4:
            m = m.unsqueeze(0)
        if m.size(2) not in (1, lq) or m.size(3) not in (1, lk) or m.size(0) not in (1, b) or m.size(1) not in (1, h):
            raise ValueError(f"attn_mask of shape {tuple(attn_mask.shape)} does not broadcast to {(b, h, lq, lk)}")
    if lq < lk and m.size(2) != 1:
        m = F.pad(m, (0, 0, lk - lq, 0))
    if lq > lk:
        m = F.pad(m.expand(m.size(0), m.size(1), m.size(2), lk), (0, lq - lk), value=float("-inf"))
    return _lib.prep_bias(m, b, h, t, q.dtype, q.device)


class GradGradAttentionFn(torch.autograd.Function):
    """softmax(q k^T / sqrt(d) + attn_mask) v with a differentiable backward
    (reference: cloud_ttt_e2e/ttt_e2e/attention.py:21-53).  The optional
    `bwd_mode` takes the strings of ``triton_attention``; the default keeps
    only the row LSE and recomputes P in the backward passes, as the
    reference's recomputing backward does."""

    @staticmethod
    def forward(ctx, q, k, v, attn_mask, bwd_mode: str = "recompute"):
        _check(q, k, v)
        lq, lk = q.size(-2), k.size(-2)
        lay = Layout(q.size(-1), qpad=max(0, lk - lq), kpad=max(0, lq - lk))
        mask = _lib.Mask(causal=False, bias=_kernel_bias(attn_mask, q, lq, lk))
        return attn_forward(ctx, q, k, v, mask, 1.0 / math.sqrt(q.size(-1)), bwd_mode, lay)

    @staticmethod
    def backward(ctx, grad_out):
        dq, dk, dv = attn_backward(ctx, grad_out)
        return dq, dk, dv, None, None


class _WindowAttentionFn(torch.autograd.Function):
    """Square attention under a structured mask (causal, optionally a key
    window), with the same differentiable backward."""

    @staticmethod
    def forward(ctx, q, k, v, mask, scale, bwd_mode):
        _lib.check_inputs(q, k, v)
        return attn_forward(ctx, q, k, v, mask, scale, bwd_mode, Layout(q.size(-1)))

    @staticmethod
    def backward(ctx, grad_out):
        dq, dk, dv = attn_backward(ctx, grad_out)
        return dq, dk, dv, None, None, None


def gradgrad_attention(q, k, v, attn_mask=None, *, bwd_mode: str = "recompute"):
    """``GradGradAttentionFn.apply`` with keyword arguments."""
    return GradGradAttentionFn.apply(q, k, v, attn_mask, bwd_mode)


def windowed_attention(q, k, v, window: Optional[int], *, local: bool = True, scale: Optional[float] = None,
                       bwd_mode: str = "recompute"):
    """Causal attention of [B,H,T,D] tensors with a key window and no mask
    tensor.  local=True: the chunked window of ``WindowedSelfAttention``
    (query chunks of `window` rows; a chunk sees the `window` keys that end
    with it, causally), reference attention.py:111-128.  local=False: the
    sliding window of ``make_window_mask`` (query i sees keys i-window+1..i),
    reference utils.py:40-54.  window None, or >= T: plain causal."""
    t = q.size(-2)
    if scale is None:
        scale = 1.0 / math.sqrt(q.size(-1))
    w = 0 if window is None or window >= t else int(window)
    if window is not None and window < 1:
        raise ValueError(f"window must be >= 1, got {window}")
    kind = _lib.WINDOW_LOCAL if local else _lib.WINDOW_SLIDING
    return _WindowAttentionFn.apply(q, k, v, _lib.Mask(causal=True, window=w, window_kind=kind), scale, bwd_mode)


class WindowedSelfAttention(nn.Module):
    """Multi-head self-attention with the reference's chunked window
    (cloud_ttt_e2e/ttt_e2e/attention.py:72-131): same constructor, parameters
    and forward.  Both settings of `use_gradgrad` run the HIP kernels (the
    reference's False branch calls torch SDPA on the same masks, :106-107 and
    :124-126); the double backward is exact either way."""

    def __init__(self, d_model: int, n_heads: int, window_size: Optional[int], use_gradgrad: bool = True):
        super().__init__()
        self.d_model = d_model
        self.n_heads = n_heads
        self.head_dim = d_model // n_heads
        self.window_size = window_size
        self.use_gradgrad = use_gradgrad
        self.q_proj = nn.Linear(d_model, d_model)
        self.k_proj = nn.Linear(d_model, d_model)
        self.v_proj = nn.Linear(d_model, d_model)
        self.out_proj = nn.Linear(d_model, d_model)

    def _split_heads(self, x: torch.Tensor) -> torch.Tensor:
        b, t, _ = x.shape
        return x.view(b, t, self.n_heads, self.head_dim).transpose(1, 2)

    def _merge_heads(self, x: torch.Tensor) -> torch.Tensor:
        b, h, t, d = x.shape
        return x.transpose(1, 2).contiguous().view(b, t, h * d)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        q = self._split_heads(self.q_proj(x))
        k = self._split_heads(self.k_proj(x))
        v = self._split_heads(self.v_proj(x))
        out = windowed_attention(q, k, v, self.window_size, local=True)
        return self.out_proj(self._merge_heads(out))
