"""Torch restatement of the reference's math path — TEST INFRASTRUCTURE ONLY.

Follows ttt_kernels/triton_attention.py:18-25 operation for operation: the
scale multiplies the score matmul, the causal mask is ``triu(ones, 1)`` filled
with -inf, softmax over the last dim, then the value matmul.  The grad-grad
steps follow the two harness forms the reference and its baseline use.
"""
from __future__ import annotations

import math
from typing import Dict, Optional

import torch


def attention_math(q, k, v, causal: bool, scale: float):
    """O = softmax(scale * q k^T, causal-masked) v  (triton_attention.py:18-25)."""
    scores = torch.matmul(q, k.transpose(-2, -1)) * scale
    if causal:
        t = scores.size(-1)
        upper = torch.ones((t, t), dtype=torch.bool, device=scores.device).triu(1)
        scores = scores.masked_fill(upper, float("-inf"))
    return torch.matmul(torch.softmax(scores, dim=-1), v)


def attention_with_probs(q, k, v, causal: bool, scale: float):
    """(O, P) with P in the input dtype  (triton_attention.py:51-59)."""
    scores = torch.matmul(q, k.transpose(-2, -1)) * scale
    if causal:
        t = scores.size(-1)
        upper = torch.ones((t, t), dtype=torch.bool, device=scores.device).triu(1)
        scores = scores.masked_fill(upper, float("-inf"))
    p = torch.softmax(scores, dim=-1)
    return torch.matmul(p, v), p


def lse_math(q, k, causal: bool, scale: float):
    """Row log-sum-exp of the scaled, masked scores (float64 internally)."""
    scores = torch.matmul(q.double(), k.double().transpose(-2, -1)) * scale
    if causal:
        t = scores.size(-1)
        upper = torch.ones((t, t), dtype=torch.bool, device=scores.device).triu(1)
        scores = scores.masked_fill(upper, float("-inf"))
    return torch.logsumexp(scores, dim=-1)


def attention_masked(q, k, v, attn_mask):
    """softmax(q k^T / sqrt(d) + attn_mask) v, the reference TTT model's
    ``_attention`` (cloud_ttt_e2e/ttt_e2e/attention.py:9-18); q [..,Lq,D],
    k, v [..,Lk,D], attn_mask broadcastable to [..,Lq,Lk] or None."""
    scores = torch.matmul(q, k.transpose(-2, -1)) * (1.0 / math.sqrt(q.size(-1)))
    if attn_mask is not None:
        scores = scores + attn_mask
    return torch.matmul(torch.softmax(scores, dim=-1), v)


def gradgrad_step(q, k, v, do, rq, rk, rv, causal: bool, scale: float,
                  do_requires_grad: bool = False, attn_mask=None) -> Dict[str, Optional[torch.Tensor]]:
    """The BASELINE cotangent form of one step on the math path:

        O = attn(q, k, v)
        dQ, dK, dV = grad(O, (q, k, v), dO, create_graph=True)
        GQ, GK, GV (, GdO) = grad(sum(dQ*rq + dK*rk + dV*rv), (q, k, v (, dO)))

    With attn_mask, attn is ``attention_masked`` (scale 1/sqrt(d)) instead.
    """
    q, k, v = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    do = do.detach().clone().requires_grad_(do_requires_grad)
    o = attention_math(q, k, v, causal, scale) if attn_mask is None else attention_masked(q, k, v, attn_mask)
    dq, dk, dv = torch.autograd.grad(o, (q, k, v), do, create_graph=True)
    s = (dq * rq).sum() + (dk * rk).sum() + (dv * rv).sum()
    wrt = (q, k, v, do) if do_requires_grad else (q, k, v)
    g = torch.autograd.grad(s, wrt)
    out = {"o": o.detach(), "dq": dq.detach(), "dk": dk.detach(), "dv": dv.detach(),
           "gq": g[0], "gk": g[1], "gv": g[2], "gdo": g[3] if do_requires_grad else None}
    return out


def harness_step(q, k, v, causal: bool, scale: float) -> Dict[str, torch.Tensor]:
    """The reference harness form (tests/bench_gradgrad.py:75-80,
    tests/test_gradgrad_compare.py:33-51): loss = out.float().mean(), then the
    grad of sum(g.pow(2).mean()) over the first-order grads."""
    q, k, v = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o = attention_math(q, k, v, causal, scale)
    loss = o.float().mean()
    grads = torch.autograd.grad(loss, (q, k, v), create_graph=True)
    s = sum(g.pow(2).mean() for g in grads)
    gg = torch.autograd.grad(s, (q, k, v))
    return {"o": o.detach(), "dq": grads[0].detach(), "dk": grads[1].detach(), "dv": grads[2].detach(),
            "gq": gg[0], "gk": gg[1], "gv": gg[2]}


def window_chunks_attention(q, k, v, window: int):
    """The attention of WindowedSelfAttention.forward for T > window, as the
    reference computes it (cloud_ttt_e2e/ttt_e2e/attention.py:111-128): query
    chunks [s, e) of `window` rows against keys [max(0, e - window), e), each
    with the local mask of :56-69 through ``attention_masked``, outputs
    concatenated.  Differentiable (torch autograd); T <= window is causal."""
    t = q.size(-2)
    if t <= window:
        i = torch.arange(t)
        mask = torch.zeros((t, t), dtype=q.dtype).masked_fill(i[None, :] > i[:, None], float("-inf"))
        return attention_masked(q, k, v, mask)
    outs = []
    for start in range(0, t, window):
        end = min(t, start + window)
        kv = max(0, end - window)
        qi = torch.arange(start, end)[:, None]
        kj = torch.arange(kv, end)[None, :]
        mask = torch.zeros((end - start, end - kv), dtype=q.dtype)
        mask = mask.masked_fill((kj > qi) | (qi - kj >= window), float("-inf"))
        outs.append(attention_masked(q[..., start:end, :], k[..., kv:end, :], v[..., kv:end, :], mask))
    return torch.cat(outs, dim=-2)


def window_gradgrad_step(q, k, v, do, rq, rk, rv, window: int) -> Dict[str, torch.Tensor]:
    """``gradgrad_step``'s BASELINE form over ``window_chunks_attention``."""
    q, k, v = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o = window_chunks_attention(q, k, v, window)
    dq, dk, dv = torch.autograd.grad(o, (q, k, v), do, create_graph=True)
    s = (dq * rq).sum() + (dk * rk).sum() + (dv * rv).sum()
    g = torch.autograd.grad(s, (q, k, v))
    return {"o": o.detach(), "dq": dq.detach(), "dk": dk.detach(), "dv": dv.detach(),
            "gq": g[0], "gk": g[1], "gv": g[2]}
