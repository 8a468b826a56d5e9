"""Grad-grad-safe attention entry point and autograd wiring, on HIP.

Same public surface as the reference module ``ttt_kernels/triton_attention.py``:
``triton_attention(q, k, v, *, causal=False, scale=None, bwd_mode='recompute')``
and ``TritonAttentionFn.apply(q, k, v, causal, scale, bwd_mode)`` with the
reference's ``bwd_mode`` strings.  All modes run hand-written gfx950 kernels:

  * ``save_p`` family (``save_p``, ``save_p_triton``, ``save_p_triton_bwd``,
    ``save_p_triton_full``): the forward writes P [B,H,T,T] in the input dtype
    (``ctx.saved_probs``, as at triton_attention.py:268-272) and the backward
    and double backward read it.
  * ``recompute`` family (``recompute``, ``recompute_manual``, ``recompute_sdp``,
    ``recompute_sdp_mem``, ``recompute_sdp_auto``, ``recompute_compiled``,
    ``dv_only``) and any unknown string (the reference's default branch,
    :416-420): the forward keeps only the row LSE and later passes recompute P
    tile by tile.
  * ``custom``: first-order gradients from the recompute kernels, returned
    without a graph (the reference routes this mode to its stubs, :345-349).

With ``create_graph=True`` the backward returns the outputs of a second
autograd Function whose backward is the exact closed-form double backward
(GQ, GK, GV and, when dO requires grad, GdO), so second-order gradients match
the math path's ATen double backward (:416-420), including the
softmax-Jacobian terms that the reference's ``save_p*`` modes drop.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
from torch.autograd.function import once_differentiable

from .. import _lib
from . import backward_stubs

SAVE_P_MODES = ("save_p", "save_p_triton", "save_p_triton_bwd", "save_p_triton_full")
RECOMPUTE_MODES = ("recompute", "recompute_manual", "recompute_sdp", "recompute_sdp_mem",
                   "recompute_sdp_auto", "recompute_compiled", "dv_only")
BWD_MODES = RECOMPUTE_MODES + SAVE_P_MODES + ("custom",)


def _unpad(t: Optional[torch.Tensor], d: int) -> Optional[torch.Tensor]:
    return t if t is None or t.size(-1) == d else t[..., :d]


def mode_kind(bwd_mode: str) -> str:
    """'save_p', 'custom' or 'recompute' (unknown strings take the recompute
    backward, as the reference's fall-through does)."""
    if bwd_mode in SAVE_P_MODES:
        return "save_p"
    if bwd_mode == "custom":
        return "custom"
    return "recompute"


class _AttnBwdFn(torch.autograd.Function):
    """First backward as a function of (q, k, v, dO); its backward is the
    double backward."""

    @staticmethod
    def forward(ctx, q, k, v, do, qp, kp, vp, op, lse, p, causal, scale):
        d = q.size(-1)
        dop = _lib.prep(do, qp.size(-1))
        dq, dk, dv, rowsum = _lib.bwd(qp, kp, vp, op, dop, lse, p, causal, scale)
        ctx.save_for_backward(qp, kp, vp, dop, lse, p, rowsum)
        ctx.causal = causal
        ctx.scale = scale
        ctx.d = d
        return _unpad(dq, d), _unpad(dk, d), _unpad(dv, d)

    @staticmethod
    @once_differentiable
    def backward(ctx, gdq, gdk, gdv):
        qp, kp, vp, dop, lse, p, rowsum = ctx.saved_tensors
        d, dpad = ctx.d, qp.size(-1)
        g1, g2, g3 = (_lib.prep(g.to(qp.dtype), dpad) for g in (gdq, gdk, gdv))
        want_gdo = ctx.needs_input_grad[3]
        gq, gk, gv, gdo = _lib.gg(qp, kp, vp, dop, lse, p, rowsum, g1, g2, g3, ctx.causal, ctx.scale,
                                  want_gdo)
        need = ctx.needs_input_grad
        return (_unpad(gq, d) if need[0] else None,
                _unpad(gk, d) if need[1] else None,
                _unpad(gv, d) if need[2] else None,
                _unpad(gdo, d) if want_gdo else None,
                None, None, None, None, None, None, None, None)


class TritonAttentionFn(torch.autograd.Function):
    """Attention whose backward stays differentiable (reference:
    ttt_kernels/triton_attention.py:259-420)."""

    @staticmethod
    def forward(ctx, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
                scale: Optional[float] = None, bwd_mode: str = "recompute"):
        _lib.check_inputs(q, k, v)
        if scale is None:
            scale = 1.0 / math.sqrt(q.size(-1))
        ctx.causal = causal
        ctx.scale = scale
        ctx.bwd_mode = bwd_mode
        kind = mode_kind(bwd_mode)
        d = q.size(-1)
        dpad = _lib.padded_head_dim(d)
        qp, kp, vp = (_lib.prep(t, dpad) for t in (q, k, v))
        op, lse, p = _lib.fwd(qp, kp, vp, causal, scale, want_p=(kind == "save_p"))
        ctx.save_for_backward(q, k, v, qp, kp, vp, op, lse, p)
        ctx.saved_probs = () if p is None else (p,)
        return _unpad(op, d)

    @staticmethod
    def backward(ctx, grad_out: torch.Tensor):
        q, k, v, qp, kp, vp, op, lse, p = ctx.saved_tensors
        causal, scale = ctx.causal, ctx.scale
        if ctx.bwd_mode == "custom":
            dq = backward_stubs.triton_attn_bwd_dq(q, k, v, grad_out, causal=causal, scale=scale)
            dk = backward_stubs.triton_attn_bwd_dk(q, k, v, grad_out, causal=causal, scale=scale)
            dv = backward_stubs.triton_attn_bwd_dv(q, k, v, grad_out, causal=causal, scale=scale)
            return dq, dk, dv, None, None, None
        if torch.is_grad_enabled():
            # The kernel operands go in detached: the closed-form double backward
            # already covers every dependence on q, k, v, so no gradient may flow
            # into O (an output of this node) or into the saved inputs a second time.
            dq, dk, dv = _AttnBwdFn.apply(q, k, v, grad_out, qp.detach(), kp.detach(), vp.detach(),
                                          op.detach(), lse, p, causal, scale)
        else:
            d = q.size(-1)
            dop = _lib.prep(grad_out, qp.size(-1))
            dq, dk, dv, _ = _lib.bwd(qp, kp, vp, op, dop, lse, p, causal, scale)
            dq, dk, dv = _unpad(dq, d), _unpad(dk, d), _unpad(dv, d)
        return dq, dk, dv, None, None, None


def triton_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, causal: bool = False,
                     scale: Optional[float] = None, bwd_mode: str = "recompute") -> torch.Tensor:
    """softmax(scale * q k^T [causal mask]) v over [B, H, T, D] tensors, with a
    backward that supports ``create_graph=True`` (reference:
    ttt_kernels/triton_attention.py:423-424)."""
    return TritonAttentionFn.apply(q, k, v, causal, scale, bwd_mode)
