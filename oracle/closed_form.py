"""Float64 numpy closed forms of attention, its backward and its full double
backward — TEST INFRASTRUCTURE ONLY.

Arrays are [..., T, D] (any leading batch dims).  Per slice, with s = scale:

  S = s Q K^T (masked entries -inf), P = softmax(S), O = P V
  dV = P^T dO, dP = dO V^T, D = rowsum(P o dP), dS = P o (dP - D),
  dQ = s dS K, dK = s dS^T Q

Double backward for cotangents (gQ, gK, gV) on (dQ, dK, dV), derived by the
chain rule through dQ, dK (directly and through dS), dS (through dP, P and D),
dV (through P and dO), dP (through dO and V) and P (through S):

  gdS = s (gQ K^T + Q gK^T)            E = rowsum(gdS o P)
  gdP = P o (gdS - E)                  gP = dO gV^T + gdS o (dP - D) - E o dP
  F   = rowsum(gP o P)                 gS = P o (gP - F)
  GQ  = s (dS gK + gS K)               GK = s (dS^T gQ + gS^T Q)
  GV  = gdP^T dO                       GdO = P gV + gdP V

An additive score bias (a constant) enters only through P, so the same
formulas hold with one.

This is the reference's recompute-mode second derivative
(ttt_kernels/triton_attention.py:416-420), i.e. ATen's double backward of the
math path (:18-25), written out.
"""
from __future__ import annotations

from typing import Dict

import numpy as np


def _t(x):
    return np.swapaxes(x, -1, -2)


def _mask(t: int) -> np.ndarray:
    return np.triu(np.ones((t, t), dtype=bool), 1)


def forward(q, k, v, causal: bool, scale: float, bias=None, p_store=None) -> Dict[str, np.ndarray]:
    """bias: an additive score bias broadcastable to [..., Tq, Tk] (entries
    may be -inf), added before the causal mask and the softmax, as the
    reference TTT model's ``_attention`` does
    (cloud_ttt_e2e/ttt_e2e/attention.py:9-18).  p_store: None, or a map of P
    to P as stored (a rounding to a storage format); O and every later use
    of P then see the stored values, as in the save_p modes, whose forward
    returns O from the cached probabilities (triton_attention.py:51-59)."""
    q, k, v = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
    s = scale * (q @ _t(k))
    if bias is not None:
        s = s + np.asarray(bias, dtype=np.float64)
    if causal:
        s = np.where(_mask(s.shape[-1]), -np.inf, s)
    mx = s.max(axis=-1, keepdims=True)
    e = np.exp(s - mx)
    l = e.sum(axis=-1, keepdims=True)
    p = e / l
    if p_store is not None:
        p = np.asarray(p_store(p), dtype=np.float64)
    return {"o": p @ v, "p": p, "lse": (mx + np.log(l))[..., 0]}


def backward(q, k, v, do, causal: bool, scale: float, bias=None, p_store=None) -> Dict[str, np.ndarray]:
    q, k, v, do = (np.asarray(x, dtype=np.float64) for x in (q, k, v, do))
    f = forward(q, k, v, causal, scale, bias, p_store)
    p, o = f["p"], f["o"]
    dp = do @ _t(v)
    dd = (p * dp).sum(axis=-1, keepdims=True)
    ds = p * (dp - dd)
    return {"o": o, "p": p, "lse": f["lse"], "dq": scale * (ds @ k), "dk": scale * (_t(ds) @ q),
            "dv": _t(p) @ do, "rowsum": dd[..., 0], "ds": ds, "dp": dp}


def double_backward(q, k, v, do, gq, gk, gv, causal: bool, scale: float, bias=None,
                    p_store=None) -> Dict[str, np.ndarray]:
    q, k, v, do, gq, gk, gv = (np.asarray(x, dtype=np.float64) for x in (q, k, v, do, gq, gk, gv))
    b = backward(q, k, v, do, causal, scale, bias, p_store)
    p, dp, ds = b["p"], b["dp"], b["ds"]
    dd = b["rowsum"][..., None]
    gds = scale * (gq @ _t(k) + q @ _t(gk))
    e = (gds * p).sum(axis=-1, keepdims=True)
    gdp = p * (gds - e)
    gp = do @ _t(gv) + gds * (dp - dd) - e * dp
    f = (gp * p).sum(axis=-1, keepdims=True)
    gs = p * (gp - f)
    out = dict(b)
    out.update({
        "gq": scale * (ds @ gk + gs @ k),
        "gk": scale * (_t(ds) @ gq + _t(gs) @ q),
        "gv": _t(gdp) @ do,
        "gdo": p @ gv + gdp @ v,
        "e": e[..., 0],
        "f": f[..., 0],
    })
    return out
