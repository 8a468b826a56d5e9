"""Pure-Python loop restatement for tiny sizes — TEST INFRASTRUCTURE ONLY.

Independent of numpy/torch linear algebra: every sum is an explicit loop over
a single (T, D) slice given as nested lists.  ``gradgrad_fd`` differentiates
the looped first backward by central finite differences, which pins the
closed-form double backward without any autograd.
"""
from __future__ import annotations

import math
from typing import List, Tuple

Mat = List[List[float]]


def _zeros(r: int, c: int) -> Mat:
    return [[0.0] * c for _ in range(r)]


def forward(q: Mat, k: Mat, v: Mat, causal: bool, scale: float, bias: Mat = None) -> Tuple[Mat, Mat]:
    """(O, P); bias: an additive [Tq][Tk] score bias (entries may be -inf)."""
    t, tk, d = len(q), len(k), len(q[0])
    p = _zeros(t, tk)
    o = _zeros(t, d)
    for m in range(t):
        row = []
        for n in range(tk):
            if causal and n > m:
                row.append(-math.inf)
            else:
                x = scale * sum(q[m][x] * k[n][x] for x in range(d))
                row.append(x + bias[m][n] if bias is not None else x)
        mx = max(row)
        ex = [0.0 if r == -math.inf else math.exp(r - mx) for r in row]
        z = sum(ex)
        for n in range(tk):
            p[m][n] = ex[n] / z
        for x in range(d):
            o[m][x] = sum(p[m][n] * v[n][x] for n in range(tk))
    return o, p


def backward(q: Mat, k: Mat, v: Mat, do: Mat, causal: bool, scale: float) -> Tuple[Mat, Mat, Mat]:
    """(dQ, dK, dV) by loops over the definitions of the attention backward."""
    t, d = len(q), len(q[0])
    _, p = forward(q, k, v, causal, scale)
    dp = [[sum(do[m][x] * v[n][x] for x in range(d)) for n in range(t)] for m in range(t)]
    ds = _zeros(t, t)
    for m in range(t):
        dd = sum(p[m][n] * dp[m][n] for n in range(t))
        for n in range(t):
            ds[m][n] = p[m][n] * (dp[m][n] - dd)
    dq = [[scale * sum(ds[m][n] * k[n][x] for n in range(t)) for x in range(d)] for m in range(t)]
    dk = [[scale * sum(ds[m][n] * q[m][x] for m in range(t)) for x in range(d)] for n in range(t)]
    dv = [[sum(p[m][n] * do[m][x] for m in range(t)) for x in range(d)] for n in range(t)]
    return dq, dk, dv


def _objective(q, k, v, do, gq, gk, gv, causal, scale) -> float:
    dq, dk, dv = backward(q, k, v, do, causal, scale)
    tot = 0.0
    for a, g in ((dq, gq), (dk, gk), (dv, gv)):
        for i in range(len(a)):
            for j in range(len(a[0])):
                tot += a[i][j] * g[i][j]
    return tot


def gradgrad_fd(q, k, v, do, gq, gk, gv, causal: bool, scale: float, eps: float = 1e-5):
    """Gradients of sum(dQ*gQ + dK*gK + dV*gV) w.r.t. (q, k, v, dO) by central
    differences of the looped backward."""
    ins = [q, k, v, do]
    grads = []
    for which in range(4):
        base = ins[which]
        g = _zeros(len(base), len(base[0]))
        for i in range(len(base)):
            for j in range(len(base[0])):
                vals = []
                for sgn in (1.0, -1.0):
                    pert = [row[:] for row in base]
                    pert[i][j] += sgn * eps
                    args = list(ins)
                    args[which] = pert
                    vals.append(_objective(*args, gq, gk, gv, causal, scale))
                g[i][j] = (vals[0] - vals[1]) / (2 * eps)
        grads.append(g)
    return tuple(grads)
