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
  * ``custom``: the reference routes this mode to its not-implemented stubs
    (:345-349).  Here it runs the recompute-mode kernels: the same
    gradients, differentiable under ``create_graph=True`` like every mode.

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


class Layout:
    """How a problem's operands map onto the kernels' square [B, H, T, Dp]
    operands: the head dim is zero-padded to Dp (64 or 128); with fewer
    queries than keys, query-side tensors (q, O, dO and their gradients) get
    `qpad` zero rows in front; with more queries than keys, key-side tensors
    (k, v and their gradients) get `kpad` zero rows at the end.  Zero query
    rows (q = dO = 0, cotangent 0) contribute nothing to any gradient, and
    padded keys are masked by the bias, so the results on the real rows are
    those of the rectangular problem."""

    def __init__(self, d: int, qpad: int = 0, kpad: int = 0):
        self.d = d
        self.dpad = _lib.padded_head_dim(d)
        self.qpad = qpad
        self.kpad = kpad
        # operands go to the kernels as they are (when their strides allow)
        self.plain = self.dpad == d and qpad == 0 and kpad == 0

    # A plain layout hands operands over as they are: the binding copies one
    # whose strides the kernels do not take.
    def q(self, t: torch.Tensor) -> torch.Tensor:
        if self.plain:
            return t
        return _lib.prep_rows(t, self.dpad, self.qpad, 0)

    def k(self, t: torch.Tensor) -> torch.Tensor:
        if self.plain:
            return t
        return _lib.prep_rows(t, self.dpad, 0, self.kpad)

    def uq(self, t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
        if t is None or self.plain or (self.qpad == 0 and t.size(-1) == self.d):
            return t
        return t[..., self.qpad:, :self.d]

    def uk(self, t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
        if t is None or self.plain or (self.kpad == 0 and t.size(-1) == self.d):
            return t
        return t[..., :t.size(-2) - self.kpad, :self.d]


# Layouts without padding rows, one per head dim (immutable), and the two
# plain causal masks: shared by every call instead of built per call.
_PLAIN_LAYOUTS: dict = {}
_CAUSAL_MASKS = (_lib.Mask(causal=False), _lib.Mask(causal=True))


def plain_layout(d: int) -> Layout:
    lay = _PLAIN_LAYOUTS.get(d)
    if lay is None:
        lay = _PLAIN_LAYOUTS[d] = Layout(d)
    return lay


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
    double backward.  The kernel-layout dQ is kept for it: the row pass of the
    double backward reads dQ = s*(dS*K) instead of forming that product.

    `fwd` = (qp, kp, vp, op, lse, p, mask, scale, lay), the saved forward in
    kernel layout, goes in as one plain object: autograd does not look inside
    it, so no gradient flows into those tensors (the closed-form double
    backward already covers every dependence on q, k, v, and O is an output
    of the forward node)."""

    @staticmethod
    def forward(ctx, q, k, v, do, fwd):
        qp, kp, vp, op, lse, p, mask, scale, lay = fwd
        dop = lay.q(do)
        dq, dk, dv, rowsum = _lib.bwd(qp, kp, vp, op, dop, lse, p, mask, scale)
        ctx.save_for_backward(qp, kp, vp, dop, lse, p, rowsum, dq)
        ctx.mask = mask
        ctx.scale = scale
        ctx.lay = lay
        return lay.uq(dq), lay.uk(dk), lay.uk(dv)

    @staticmethod
    @once_differentiable
    def backward(ctx, gdq, gdk, gdv):
        qp, kp, vp, dop, lse, p, rowsum, dq = ctx.saved_tensors
        lay = ctx.lay
        dt = qp.dtype
        g1 = lay.q(gdq if gdq.dtype == dt else gdq.to(dt))
        g2 = lay.k(gdk if gdk.dtype == dt else gdk.to(dt))
        g3 = lay.k(gdv if gdv.dtype == dt else gdv.to(dt))
        want_gdo = ctx.needs_input_grad[3]
        gq, gk, gv, gdo = _lib.gg(qp, kp, vp, dop, lse, p, rowsum, g1, g2, g3, ctx.mask, ctx.scale, want_gdo,
                                  dq=dq)
        need = ctx.needs_input_grad
        return (lay.uq(gq) if need[0] else None,
                lay.uk(gk) if need[1] else None,
                lay.uk(gv) if need[2] else None,
                lay.uq(gdo) if want_gdo else None,
                None)


class SavedProbs(tuple):
    """``ctx.saved_probs``: the one-tuple ``(P,)`` of a save_p forward.  The
    forward writes only the tiles of P that some row sees; the first time P
    is taken out of this tuple, the other tiles are filled with zeros
    (``_lib.fill_masked_p``) on the current stream, so a caller that reads
    ``ctx.saved_probs[0]`` (as the reference's backward does,
    triton_attention.py:354-378) gets the whole softmax matrix.  The kernels'
    own backward reads P from the saved tensors and never pays for the fill."""

    def __new__(cls, p: torch.Tensor, mask: "_lib.Mask"):
        obj = super().__new__(cls, (p,))
        obj._mask = mask
        obj._filled = False
        return obj

    def _complete(self) -> None:
        if not self._filled:
            _lib.fill_masked_p(tuple.__getitem__(self, 0), self._mask)
            self._filled = True

    def __getitem__(self, i):
        self._complete()
        return tuple.__getitem__(self, i)

    def __iter__(self):
        self._complete()
        return tuple.__iter__(self)


def attn_forward(ctx, q, k, v, mask: "_lib.Mask", scale: float, bwd_mode: str, lay: Layout) -> torch.Tensor:
    """Forward of an attention Function: runs the kernels on the laid-out
    operands and keeps what the backward needs on ctx."""
    ctx.mask = mask
    ctx.scale = scale
    ctx.bwd_mode = bwd_mode
    ctx.lay = lay
    kind = mode_kind(bwd_mode)
    qp = lay.q(q)
    kp, vp = lay.k(k), lay.k(v)
    op, lse, p = _lib.fwd(qp, kp, vp, mask, scale, want_p=(kind == "save_p"))
    ctx.save_for_backward(q, k, v, qp, kp, vp, op, lse, p)
    ctx.saved_probs = () if p is None else SavedProbs(p, mask)
    return lay.uq(op)


def attn_backward(ctx, grad_out: torch.Tensor):
    """(dq, dk, dv) of an attention Function.  Under create_graph=True
    (grad mode on in the backward) they come from _AttnBwdFn, whose backward
    is the exact double backward; otherwise straight from the kernels."""
    q, k, v, qp, kp, vp, op, lse, p = ctx.saved_tensors
    mask, scale, lay = ctx.mask, ctx.scale, ctx.lay
    if torch.is_grad_enabled():
        # O detached: the saved node holds no edge into the forward's graph
        return _AttnBwdFn.apply(q, k, v, grad_out, (qp, kp, vp, op.detach(), lse, p, mask, scale, lay))
    dq, dk, dv, _ = _lib.bwd(qp, kp, vp, op, lay.q(grad_out), lse, p, mask, scale)
    return lay.uq(dq), lay.uk(dk), lay.uk(dv)


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
        return attn_forward(ctx, q, k, v, _CAUSAL_MASKS[bool(causal)], scale, bwd_mode, plain_layout(q.size(-1)))

    @staticmethod
    def backward(ctx, grad_out: torch.Tensor):
        # Every mode, `custom` included, takes the kernels' backward from the
        # saved forward (O, LSE and, for save_p, P); under create_graph=True it
        # stays differentiable.
        dq, dk, dv = attn_backward(ctx, grad_out)
        return dq, dk, dv, None, None, None


def triton_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, causal: bool = False,
                     scale: Optional[float] = None, bwd_mode: str = "recompute") -> torch.Tensor:
    """softmax(scale * q k^T [causal mask]) v over [B, H, T, D] tensors, with a
    backward that supports ``create_graph=True`` (reference:
    ttt_kernels/triton_attention.py:423-424)."""
    return TritonAttentionFn.apply(q, k, v, causal, scale, bwd_mode)
