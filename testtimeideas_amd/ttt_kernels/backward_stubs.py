"""Backward and double-backward launchers of the grad-grad attention, on HIP.

Same names, arguments and return values as the reference module
``ttt_kernels/backward_stubs.py``; every launcher runs hand-written gfx950
kernels through ``libttt_attn.so``.  The reference's not-implemented stubs
(``triton_attn_bwd_dq``/``_dk``, ``triton_attn_bwd2_*``) are implemented.

Differences from the reference, deliberate:
  * ``TritonDqDkFn.backward`` uses the correct term ``Q @ grad_dk^T`` in
    ``grad_ds`` (the reference has ``grad_dk @ Q^T``, backward_stubs.py:491-492).
  * Inputs must live on a ROCm device (there is no CPU path), and head dims
    other than 64 and 128 (up to 128) are zero-padded to the next of the two.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
from torch.autograd import Function

from .. import _lib


def _scale_or_default(scale: Optional[float], d: int) -> float:
    return 1.0 / math.sqrt(d) if scale is None else float(scale)


def _padded(*ts: torch.Tensor):
    d = ts[0].size(-1)
    dp = _lib.padded_head_dim(d)
    return d, [None if t is None else _lib.prep(t, dp) for t in ts]


def _rowsum_f32(rowsum: torch.Tensor) -> torch.Tensor:
    return rowsum.to(torch.float32).contiguous()


def triton_attn_bwd_dv(q, k, v, do, *, causal: bool, scale: float):
    """dV with P recomputed from the row statistics (reference: _attn_bwd_dv_kernel +
    triton_attn_bwd_dv, backward_stubs.py:22-121).  Not differentiable."""
    _lib.check_inputs(q, k, v, do)
    d, (qp, kp, vp, dop) = _padded(q, k, v, do)
    with torch.no_grad():
        _, lse, _ = _lib.fwd(qp, kp, vp, causal, scale, False)
        _, dv = _lib.bwd_dkdv(qp, kp, None, dop, None, lse, None, causal, scale, want_dk=False)
    return dv[..., :d]


def triton_attn_bwd_dv_from_p(p, do):
    """dV = P^T dO from a saved P (reference: backward_stubs.py:124-181)."""
    _lib.check_inputs(do)
    if p.shape != do.shape[:3] + (do.shape[2],) or p.dtype != do.dtype or p.device != do.device:
        raise ValueError(f"p must be [B,H,T,T] in do's dtype; got {tuple(p.shape)} {p.dtype}")
    d, (dop,) = _padded(do)
    pp = _lib.prep_p(p)
    _, dv = _lib.bwd_dkdv(None, None, None, dop, pp, None, None, False, 1.0, want_dk=False)
    return dv[..., :d]


def triton_attn_rowsum_from_p(p, do, v, *, causal: bool):
    """rowsum[m] = sum_n (dO V^T)[m,n] P[m,n], fp32 [B,H,T] (reference:
    backward_stubs.py:184-255)."""
    _lib.check_inputs(do, v)
    _, (dop, vp) = _padded(do, v)
    return _lib.rowsum_from_p(_lib.prep_p(p), dop, vp, causal)


def triton_attn_bwd_dqdk_from_p(q, k, v, do, p, rowsum, *, causal: bool, scale: float):
    """(dQ, dK) from a saved P and row statistic (reference: backward_stubs.py:259-425)."""
    _lib.check_inputs(q, k, v, do)
    d, (qp, kp, vp, dop) = _padded(q, k, v, do)
    pp = _lib.prep_p(p)
    rs = _rowsum_f32(rowsum)
    dq = _lib.bwd_dq(qp, kp, vp, dop, pp, None, rs, causal, scale)
    dk, _ = _lib.bwd_dkdv(qp, kp, vp, dop, pp, None, rs, causal, scale, want_dk=True)
    return dq[..., :d], dk[..., :d]


class TritonDvFn(Function):
    """dV = P^T dO as a differentiable function of (P, dO) (reference:
    backward_stubs.py:428-439)."""

    @staticmethod
    def forward(ctx, p, do):
        ctx.save_for_backward(p, do)
        return triton_attn_bwd_dv_from_p(p, do)

    @staticmethod
    def backward(ctx, grad_dv):
        p, do = ctx.saved_tensors
        grad_p = torch.matmul(do, grad_dv.transpose(-2, -1).contiguous())
        grad_do = torch.matmul(p, grad_dv)
        return grad_p, grad_do


class TritonRowSumFn(Function):
    """rowsum = sum_n P o (dO V^T) as a differentiable function of (P, dO, V)
    (reference: backward_stubs.py:442-459)."""

    @staticmethod
    def forward(ctx, p, do, v, causal: bool):
        ctx.save_for_backward(p, do, v)
        ctx.causal = causal
        return triton_attn_rowsum_from_p(p, do, v, causal=causal)

    @staticmethod
    def backward(ctx, grad_rs):
        p, do, v = ctx.saved_tensors
        g = grad_rs.to(p.dtype).unsqueeze(-1)
        dp = torch.matmul(do, v.transpose(-2, -1).contiguous())
        grad_p = g * dp
        grad_do = g * torch.matmul(p, v)
        grad_v = torch.matmul(p.transpose(-2, -1).contiguous(), g * do)
        return grad_p, grad_do, grad_v, None


class TritonDqDkFn(Function):
    """(dQ, dK) as a differentiable function of (q, k, v, dO, P, rowsum), with P
    and rowsum treated as independent inputs (reference: backward_stubs.py:462-514)."""

    @staticmethod
    def forward(ctx, q, k, v, do, p, rowsum, scale: float, causal: bool):
        ctx.save_for_backward(q, k, v, do, p, rowsum)
        ctx.scale = scale
        ctx.causal = causal
        return triton_attn_bwd_dqdk_from_p(q, k, v, do, p, rowsum, causal=causal, scale=scale)

    @staticmethod
    def backward(ctx, grad_dq, grad_dk):
        q, k, v, do, p, rowsum = ctx.saved_tensors
        s = ctx.scale
        dt = q.dtype
        rs = rowsum.to(dt).unsqueeze(-1)
        gdq = torch.zeros_like(q) if grad_dq is None else grad_dq.to(dt)
        gdk = torch.zeros_like(k) if grad_dk is None else grad_dk.to(dt)
        dp = torch.matmul(do, v.transpose(-2, -1).contiguous())
        ds = (dp - rs) * p
        grad_ds = (torch.matmul(gdq, k.transpose(-2, -1).contiguous())
                   + torch.matmul(q, gdk.transpose(-2, -1).contiguous())) * s
        grad_q = torch.matmul(ds, gdk) * s
        grad_k = torch.matmul(ds.transpose(-2, -1).contiguous(), gdq) * s
        grad_dp = grad_ds * p
        grad_p = grad_ds * (dp - rs)
        grad_rowsum = -(grad_ds * p).sum(dim=-1)
        grad_do = torch.matmul(grad_dp, v)
        grad_v = torch.matmul(grad_dp.transpose(-2, -1).contiguous(), do)
        return (grad_q, grad_k, grad_v, grad_do, grad_p, grad_rowsum.to(rowsum.dtype), None, None)


# ---------------------------------------------------------------------------
# Recompute-mode first backward (the reference's stubs, backward_stubs.py:529-534).
# ---------------------------------------------------------------------------
def _recompute_bwd(q, k, v, do, causal: bool, scale: float):
    _lib.check_inputs(q, k, v, do)
    d, (qp, kp, vp, dop) = _padded(q, k, v, do)
    with torch.no_grad():
        o, lse, _ = _lib.fwd(qp, kp, vp, causal, scale, False)
        dq, dk, dv, _ = _lib.bwd(qp, kp, vp, o, dop, lse, None, causal, scale)
    return dq[..., :d], dk[..., :d], dv[..., :d]


def triton_attn_bwd_dq(q, k, v, do, *, causal: bool, scale: float):
    """dQ with P recomputed from the row statistics.  Not differentiable."""
    return _recompute_bwd(q, k, v, do, causal, scale)[0]


def triton_attn_bwd_dk(q, k, v, do, *, causal: bool, scale: float):
    """dK with P recomputed from the row statistics.  Not differentiable."""
    return _recompute_bwd(q, k, v, do, causal, scale)[1]


# ---------------------------------------------------------------------------
# Double backward (the reference's stubs, backward_stubs.py:537-548).
# ---------------------------------------------------------------------------
def triton_attn_bwd2(q, k, v, do, grad_dq, grad_dk, grad_dv, *, causal: bool = False,
                     scale: Optional[float] = None, want_gdo: bool = True
                     ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """Exact second derivative: gradients of sum(dQ*grad_dq + dK*grad_dk + dV*grad_dv)
    with respect to (q, k, v, dO).  Recomputes P from the row statistics."""
    _lib.check_inputs(q, k, v, do, grad_dq, grad_dk, grad_dv)
    scale = _scale_or_default(scale, q.size(-1))
    d, (qp, kp, vp, dop, g1, g2, g3) = _padded(q, k, v, do, grad_dq, grad_dk, grad_dv)
    with torch.no_grad():
        o, lse, _ = _lib.fwd(qp, kp, vp, causal, scale, False)
        _, _, _, rowsum = _lib.bwd(qp, kp, vp, o, dop, lse, None, causal, scale)
        gq, gk, gv, gdo = _lib.gg(qp, kp, vp, dop, lse, None, rowsum, g1, g2, g3, causal, scale, want_gdo)
    return gq[..., :d], gk[..., :d], gv[..., :d], (None if gdo is None else gdo[..., :d])


def triton_attn_bwd2_dq(q, k, v, do, grad_dq, grad_dk, grad_dv, *, causal: bool = False,
                        scale: Optional[float] = None):
    """Second-order gradient with respect to q."""
    return triton_attn_bwd2(q, k, v, do, grad_dq, grad_dk, grad_dv, causal=causal, scale=scale,
                            want_gdo=False)[0]


def triton_attn_bwd2_dk(q, k, v, do, grad_dq, grad_dk, grad_dv, *, causal: bool = False,
                        scale: Optional[float] = None):
    """Second-order gradient with respect to k."""
    return triton_attn_bwd2(q, k, v, do, grad_dq, grad_dk, grad_dv, causal=causal, scale=scale,
                            want_gdo=False)[1]


def triton_attn_bwd2_dv(q, k, v, do, grad_dq, grad_dk, grad_dv, *, causal: bool = False,
                        scale: Optional[float] = None):
    """Second-order gradient with respect to v."""
    return triton_attn_bwd2(q, k, v, do, grad_dq, grad_dk, grad_dv, causal=causal, scale=scale,
                            want_gdo=False)[2]
