"""Row-block closed forms of attention, its backward and its full double
backward, for sequences too long for the dense closed forms — TEST
INFRASTRUCTURE ONLY.

The quantities and formulas are those of ``oracle.closed_form`` (forward
S = s Q K^T, P = softmax(S), O = P V, first backward, and the double
backward for cotangents gQ, gK, gV), evaluated one block of query rows at a
time:

  * everything indexed by query rows (O, LSE, D, E, F, dQ, GQ, GdO) depends
    only on that block's rows of S, so it is computed within the block;
  * everything indexed by key rows (dK, dV, GK, GV) is a sum over query rows,
    so each block adds its share (dK += s dS^T Q_blk, dV += P^T dO_blk,
    GK += s (dS^T gQ_blk + gS^T Q_blk), GV += gdP^T dO_blk);
  * causal blocks stop at their last row's key, the keys after it being
    masked for every row of the block; with a key window they also start at
    their first row's first key (the reference TTT model's local window,
    cloud_ttt_e2e/ttt_e2e/attention.py:111-131, or make_window_mask,
    utils.py:40-54).

Memory is O(block * T) instead of O(T^2), so T = 16384 runs in float64 on the
CPU.  The functions work on any torch device and dtype; the parity tests use
float64 on the CPU (the oracle) and, as a second check over many (b, h)
slices, float32 on the GPU.  Agreement with ``closed_form.double_backward``
(pinned by loops, finite differences and autograd) is tested in
tests/test_oracle_blocked.py.

Reference semantics: ttt_kernels/triton_attention.py:18-25 (math path) and
its ATen double backward (:416-420), as in ``closed_form``.
"""
from __future__ import annotations

from typing import Callable, Dict, Optional

import torch


def window_lo(m: torch.Tensor, t: int, window: int, local: bool) -> torch.Tensor:
    """First key query rows m see under a key window (0 without one): the
    local layout of oracle.masks.local_bias (rows in chunks of W; a chunk's
    keys start at min(T, (m // W + 1) W) - W) or the sliding window of
    oracle.masks.window_bias (m - W + 1)."""
    if window <= 0 or window >= t:
        return torch.zeros_like(m)
    if local:
        return torch.clamp(torch.clamp((m // window + 1) * window, max=t) - window, min=0)
    return torch.clamp(m - window + 1, min=0)


def double_backward_blocked(q, k, v, do, gq, gk, gv, causal: bool, scale: float, block: int = 512,
                            on_p: Optional[Callable[[int, int, torch.Tensor], None]] = None,
                            gradgrad: bool = True, window: int = 0, local: bool = True) -> Dict[str, torch.Tensor]:
    """One (b, h) slice: q, k, v, do, gq, gk, gv are [T, D] tensors (gq, gk,
    gv may be None when gradgrad is False).  Returns o, lse (natural log),
    rowsum (D), dq, dk, dv and, with gradgrad, e, f, gq, gk, gv, gdo, all in
    the inputs' dtype and device.  on_p(r0, r1, p) receives each block's rows
    r0:r1 of P over keys 0:c1 (c1 = r1 when causal, else T); the rest of
    those rows is zero.  A key window (window > 0, with causal; see
    window_lo) also hides the keys before each row's first one: a block then
    works on keys c0:c1 with c0 its first row's first key (on_p still
    receives keys 0:c1, zeros before c0)."""
    t, d = q.shape
    dev, dt = q.device, q.dtype
    z = lambda *s: torch.zeros(*s, dtype=dt, device=dev)  # noqa: E731
    out = {"o": z(t, d), "lse": z(t), "rowsum": z(t), "dq": z(t, d), "dk": z(t, d), "dv": z(t, d)}
    if gradgrad:
        out.update({"e": z(t), "f": z(t), "gq": z(t, d), "gk": z(t, d), "gv": z(t, d), "gdo": z(t, d)})
    if window > 0 and not causal:
        raise ValueError("a key window needs causal")
    for r0 in range(0, t, block):
        r1 = min(t, r0 + block)
        c1 = r1 if causal else t
        rows = torch.arange(r0, r1, device=dev)[:, None]
        lo = window_lo(rows, t, window, local)
        c0 = int(lo[0, 0])
        qb, dob = q[r0:r1], do[r0:r1]
        kc, vc = k[c0:c1], v[c0:c1]
        s = scale * (qb @ kc.T)
        if causal:
            cols = torch.arange(c0, c1, device=dev)[None, :]
            s = s.masked_fill((cols > rows) | (cols < lo), float("-inf"))
        mx = s.amax(dim=1, keepdim=True)
        ex = torch.exp(s - mx)
        den = ex.sum(dim=1, keepdim=True)
        p = ex / den
        del s, ex
        if on_p is not None:
            on_p(r0, r1, p if c0 == 0 else torch.cat([torch.zeros(r1 - r0, c0, dtype=dt, device=dev), p], 1))
        out["lse"][r0:r1] = (mx + torch.log(den))[:, 0]
        out["o"][r0:r1] = p @ vc
        dp = dob @ vc.T
        dd = (p * dp).sum(dim=1, keepdim=True)
        ds = p * (dp - dd)
        out["rowsum"][r0:r1] = dd[:, 0]
        out["dq"][r0:r1] = scale * (ds @ kc)
        out["dk"][c0:c1] += scale * (ds.T @ qb)
        out["dv"][c0:c1] += p.T @ dob
        if not gradgrad:
            continue
        gqb = gq[r0:r1]
        gkc, gvc = gk[c0:c1], gv[c0:c1]
        gds = scale * (gqb @ kc.T + qb @ gkc.T)
        e = (gds * p).sum(dim=1, keepdim=True)
        gdp = p * (gds - e)
        gp = dob @ gvc.T + gds * (dp - dd) - e * dp
        del gds
        f = (gp * p).sum(dim=1, keepdim=True)
        gs = p * (gp - f)
        del gp
        out["e"][r0:r1] = e[:, 0]
        out["f"][r0:r1] = f[:, 0]
        out["gq"][r0:r1] = scale * (ds @ gkc + gs @ kc)
        out["gk"][c0:c1] += scale * (ds.T @ gqb + gs.T @ qb)
        out["gv"][c0:c1] += gdp.T @ dob
        out["gdo"][r0:r1] = p @ gvc + gdp @ vc
    return out
