"""The backward of the helper autograd Functions in backward_stubs
(TritonDvFn, TritonRowSumFn, TritonDqDkFn; reference backward_stubs.py:428-514)
on the CPU: each is a torch-op vector-Jacobian product with P and rowsum
treated as independent inputs, and must equal float64 autograd of the
function its forward computes:

  TritonDvFn      dV = P^T dO
  TritonRowSumFn  rowsum = sum_n P o (dO V^T)
  TritonDqDkFn    dS = P o (dO V^T - rowsum), dQ = s dS K, dK = s dS^T Q

The backward methods are called directly with a stand-in ctx (no kernel
runs).  The reference's own TritonDqDkFn backward has K^T-shaped term
``grad_dk @ Q^T`` where autograd gives ``Q @ grad_dk^T`` (BS:491-492); a
planted copy of that term fails the same check.
"""
from types import SimpleNamespace

import torch

from testtimeideas_amd.ttt_kernels.backward_stubs import TritonDqDkFn, TritonDvFn, TritonRowSumFn

TOL = 1e-12


def _mt(x):
    return x.transpose(-2, -1)


def _rand(*shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float64)


def _softmax_p(b, h, t, causal, seed):
    s = _rand(b, h, t, t, seed=seed)
    if causal:
        s = s.masked_fill(torch.triu(torch.ones(t, t, dtype=torch.bool), 1), float("-inf"))
    return torch.softmax(s, dim=-1)


def _vjp(fn, inputs, cotangents):
    xs = [x.clone().requires_grad_(True) for x in inputs]
    outs = fn(*xs)
    outs = outs if isinstance(outs, tuple) else (outs,)
    gs = torch.autograd.grad(outs, xs, cotangents, allow_unused=True)
    return [torch.zeros_like(x) if g is None else g for x, g in zip(xs, gs)]


def _close(a, b, name):
    err = float((a - b).abs().max())
    scale = float(b.abs().max())
    assert err <= TOL * max(scale, 1.0), f"{name}: max-abs {err:.3e} (scale {scale:.3e})"


def test_dv_fn_backward():
    b, h, t, d = 1, 2, 40, 16
    p, do, g = _softmax_p(b, h, t, True, 1), _rand(b, h, t, d, seed=2), _rand(b, h, t, d, seed=3)
    ctx = SimpleNamespace(saved_tensors=(p, do))
    got = TritonDvFn.backward(ctx, g)
    ref = _vjp(lambda p_, do_: _mt(p_) @ do_, (p, do), (g,))
    for name, a, r in zip(("grad_p", "grad_do"), got, ref):
        _close(a, r, name)


def test_rowsum_fn_backward():
    b, h, t, d = 2, 1, 33, 16
    p = _softmax_p(b, h, t, False, 4)
    do, v, g = _rand(b, h, t, d, seed=5), _rand(b, h, t, d, seed=6), _rand(b, h, t, seed=7)
    ctx = SimpleNamespace(saved_tensors=(p, do, v), causal=False)
    got = TritonRowSumFn.backward(ctx, g)
    assert got[3] is None
    ref = _vjp(lambda p_, do_, v_: (p_ * (do_ @ _mt(v_))).sum(-1), (p, do, v), (g,))
    for name, a, r in zip(("grad_p", "grad_do", "grad_v"), got[:3], ref):
        _close(a, r, name)


def _dqdk(q, k, v, do, p, rowsum, s):
    ds = p * (do @ _mt(v) - rowsum.unsqueeze(-1))
    return s * (ds @ k), s * (_mt(ds) @ q)


def _dqdk_case(seed, causal):
    b, h, t, d = 1, 2, 37, 16
    q, k, v, do = (_rand(b, h, t, d, seed=seed + i) for i in range(4))
    p = _softmax_p(b, h, t, causal, seed + 4)
    rowsum = _rand(b, h, t, seed=seed + 5)
    gdq, gdk = _rand(b, h, t, d, seed=seed + 6), _rand(b, h, t, d, seed=seed + 7)
    return (q, k, v, do, p, rowsum), (gdq, gdk)


def test_dqdk_fn_backward_matches_autograd():
    for causal in (False, True):
        inputs, (gdq, gdk) = _dqdk_case(10, causal)
        s = 0.3
        ctx = SimpleNamespace(saved_tensors=inputs, scale=s, causal=causal)
        got = TritonDqDkFn.backward(ctx, gdq, gdk)
        assert got[6] is None and got[7] is None
        ref = _vjp(lambda *xs: _dqdk(*xs, s), inputs, (gdq, gdk))
        for name, a, r in zip(("grad_q", "grad_k", "grad_v", "grad_do", "grad_p", "grad_rowsum"), got[:6], ref):
            _close(a, r, name)


def test_dqdk_fn_backward_with_one_cotangent():
    inputs, (gdq, _) = _dqdk_case(20, True)
    ctx = SimpleNamespace(saved_tensors=inputs, scale=0.5, causal=True)
    got = TritonDqDkFn.backward(ctx, gdq, None)
    ref = _vjp(lambda *xs: _dqdk(*xs, 0.5)[0], inputs, (gdq,))
    for name, a, r in zip(("grad_q", "grad_k", "grad_v", "grad_do", "grad_p", "grad_rowsum"), got[:6], ref):
        _close(a, r, name)


def test_planted_transposed_gdk_term_fails():
    """The check above catches the reference's transposed term: the same VJP
    with ``grad_dk @ Q^T`` in place of ``Q @ grad_dk^T`` misses autograd on
    grad_v, grad_do, grad_p and grad_rowsum."""
    inputs, (gdq, gdk) = _dqdk_case(30, False)
    q, k, v, do, p, rowsum = inputs
    s = 0.3
    dp = do @ _mt(v)
    grad_ds = (gdq @ _mt(k) + gdk @ _mt(q)) * s  # the planted (transposed) term
    planted = {
        "grad_v": _mt(grad_ds * p) @ do,
        "grad_do": (grad_ds * p) @ v,
        "grad_p": grad_ds * (dp - rowsum.unsqueeze(-1)),
        "grad_rowsum": -(grad_ds * p).sum(-1),
    }
    ref = dict(zip(("grad_q", "grad_k", "grad_v", "grad_do", "grad_p", "grad_rowsum"),
                   _vjp(lambda *xs: _dqdk(*xs, s), inputs, (gdq, gdk))))
    for name, a in planted.items():
        assert float((a - ref[name]).abs().max()) > 1e-3 * float(ref[name].abs().max()), name
