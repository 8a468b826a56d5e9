"""Pins the CPU oracle (CPU only).

Each oracle function is checked against something that does not restate its
own formula: independent pure-Python loops, central finite differences,
torch's float64 gradcheck/gradgradcheck, closed-form special cases, and
identities.  Planted mistakes in a copy of the closed form must fail.
"""
import math

import numpy as np
import pytest
import torch

from oracle import brute, closed_form as cf, math_path


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(shape, generator=g, dtype=torch.float64) * scale for _ in range(7)]


def _lists(x: torch.Tensor):
    return x.tolist()


# ----------------------------------------------------------------------------- forward
@pytest.mark.parametrize("causal", [False, True])
def test_math_forward_matches_loops(causal):
    q, k, v = _rand((5, 3), 1)[:3]
    o_loop, p_loop = brute.forward(_lists(q), _lists(k), _lists(v), causal, 0.7)
    o, p = math_path.attention_with_probs(q, k, v, causal, 0.7)
    assert np.allclose(o.numpy(), o_loop, atol=1e-13)
    assert np.allclose(p.numpy(), p_loop, atol=1e-13)
    f = cf.forward(q.numpy(), k.numpy(), v.numpy(), causal, 0.7)
    assert np.allclose(f["o"], o_loop, atol=1e-13)
    assert np.allclose(math_path.attention_math(q, k, v, causal, 0.7).numpy(), o_loop, atol=1e-13)


def test_special_cases():
    q, k, v = _rand((1, 2, 9, 4), 2)[:3]
    # T = 1: the only key gets weight 1, so O = V.
    o1 = math_path.attention_math(q[..., :1, :], k[..., :1, :], v[..., :1, :], False, 0.5)
    assert torch.allclose(o1, v[..., :1, :])
    # q = 0: uniform weights; O is the column mean of V, or the prefix mean when causal.
    z = torch.zeros_like(q)
    assert torch.allclose(math_path.attention_math(z, k, v, False, 0.5),
                          v.mean(dim=-2, keepdim=True).expand_as(v))
    prefix = torch.cumsum(v, dim=-2) / torch.arange(1, 10, dtype=torch.float64)[:, None]
    assert torch.allclose(math_path.attention_math(z, k, v, True, 0.5), prefix)
    # causal row 0 attends only to key 0.
    assert torch.allclose(math_path.attention_math(q, k, v, True, 0.5)[..., 0, :], v[..., 0, :])
    # LSE: log(T) when q = 0 (non-causal).
    assert torch.allclose(math_path.lse_math(z, k, False, 0.5), torch.full((1, 2, 9), math.log(9.0),
                                                                           dtype=torch.float64))


# ----------------------------------------------------------------------------- backward
@pytest.mark.parametrize("causal", [False, True])
def test_closed_form_backward_vs_loops_and_autograd(causal):
    q, k, v, do = _rand((6, 4), 3)[:4]
    dq_l, dk_l, dv_l = brute.backward(_lists(q), _lists(k), _lists(v), _lists(do), causal, 0.6)
    b = cf.backward(q.numpy(), k.numpy(), v.numpy(), do.numpy(), causal, 0.6)
    assert np.allclose(b["dq"], dq_l, atol=1e-12)
    assert np.allclose(b["dk"], dk_l, atol=1e-12)
    assert np.allclose(b["dv"], dv_l, atol=1e-12)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    o = math_path.attention_math(qq, kk, vv, causal, 0.6)
    g = torch.autograd.grad(o, (qq, kk, vv), do)
    for name, x in zip(("dq", "dk", "dv"), g):
        assert np.allclose(b[name], x.numpy(), atol=1e-12), name


def test_rowsum_identity():
    """rowsum(P o dP) == rowsum(dO o O): the O(T d) form of D used by the kernels."""
    q, k, v, do = (x.numpy() for x in _rand((2, 3, 17, 8), 4)[:4])
    for causal in (False, True):
        b = cf.backward(q, k, v, do, causal, 0.4)
        assert np.allclose(b["rowsum"], (do * b["o"]).sum(-1), atol=1e-12)


def test_gradcheck_math_path():
    q, k, v = (t.requires_grad_(True) for t in _rand((1, 1, 5, 3), 5)[:3])
    for causal in (False, True):
        f = lambda a, b_, c: math_path.attention_math(a, b_, c, causal, 0.9)  # noqa: E731
        assert torch.autograd.gradcheck(f, (q, k, v))
        assert torch.autograd.gradgradcheck(f, (q, k, v))


# ----------------------------------------------------------------------------- double backward
@pytest.mark.parametrize("causal", [False, True])
def test_double_backward_vs_finite_differences(causal):
    q, k, v, do, gq, gk, gv = (_lists(x) for x in _rand((4, 3), 6))
    fd = brute.gradgrad_fd(q, k, v, do, gq, gk, gv, causal, 0.8)
    a = [np.asarray(x) for x in (q, k, v, do, gq, gk, gv)]
    cfo = cf.double_backward(*a, causal, 0.8)
    for name, ref in zip(("gq", "gk", "gv", "gdo"), fd):
        assert np.allclose(cfo[name], ref, atol=1e-7), (name, np.abs(cfo[name] - ref).max())


@pytest.mark.parametrize("causal", [False, True])
def test_double_backward_vs_autograd(causal):
    xs = _rand((2, 2, 24, 8), 7)
    ref = math_path.gradgrad_step(*xs, causal, 0.35, do_requires_grad=True)
    cfo = cf.double_backward(*(x.numpy() for x in xs), causal, 0.35)
    for name in ("o", "dq", "dk", "dv", "gq", "gk", "gv", "gdo"):
        assert np.allclose(cfo[name], ref[name].numpy(), atol=1e-11), name


def test_f_single_pass_identity():
    """F = rowsum(P o gP1) + rowsum(gdS o dS) - E*D equals rowsum(gP o P)."""
    q, k, v, do, gq, gk, gv = (x.numpy() for x in _rand((1, 2, 20, 8), 8))
    c = cf.double_backward(q, k, v, do, gq, gk, gv, True, 0.5)
    p, ds = c["p"], c["ds"]
    gds = 0.5 * (gq @ np.swapaxes(k, -1, -2) + q @ np.swapaxes(gk, -1, -2))
    gp1 = do @ np.swapaxes(gv, -1, -2)
    f1 = (p * gp1).sum(-1) + (gds * ds).sum(-1) - c["e"] * c["rowsum"]
    assert np.allclose(f1, c["f"], atol=1e-12)


def test_mean_loss_gradgrad_underflows_in_fp16():
    """Why the tests use N(0,1) cotangents: with the reference's mean-loss harness
    the true grad-grad magnitudes are ~1e-10, below fp16's smallest subnormal."""
    xs = _rand((1, 1, 64, 64), 0)
    r = math_path.harness_step(*xs[:3], True, 0.125)
    mags = [r[n].abs().max().item() for n in ("gq", "gk", "gv")]
    assert max(mags) < 6e-8, mags


# ----------------------------------------------------------------------------- planted mistakes
def _gg_variant(q, k, v, do, gq, gk, gv, causal, scale, bug):
    """Copy of the closed form with one plausible mistake switched on."""
    T = lambda x: np.swapaxes(x, -1, -2)  # noqa: E731
    b = cf.backward(q, k, v, do, causal, scale)
    p, dp, ds = b["p"], b["dp"], b["ds"]
    dd = b["rowsum"][..., None]
    if bug == "transposed_gk":  # the reference's grad_ds term, backward_stubs.py:491-492
        gds = scale * (gq @ T(k) + gk @ T(q))
    else:
        gds = scale * (gq @ T(k) + q @ T(gk))
    e = (gds * p).sum(-1, keepdims=True)
    gdp = p * (gds - (0 if bug == "drop_e" else e))
    gp = do @ T(gv) + gds * (dp - dd) - (-e if bug == "sign_e" else e) * dp
    if bug == "p_constant":  # the reference's save_p* grad-grad: no softmax Jacobian term
        gs = np.zeros_like(p)
    else:
        f = (gp * p).sum(-1, keepdims=True)
        gs = p * (gp - f)
    return {"gq": scale * (ds @ gk + gs @ k), "gk": scale * (T(ds) @ gq + T(gs) @ q), "gv": T(gdp) @ do}


@pytest.mark.parametrize("bug", ["transposed_gk", "drop_e", "sign_e", "p_constant"])
def test_planted_mistakes_are_caught(bug):
    xs = [x.numpy() for x in _rand((1, 1, 4, 3), 9)]
    ok = _gg_variant(*xs, True, 0.8, None)
    fd = brute.gradgrad_fd(*[x[0, 0].tolist() for x in xs], True, 0.8)
    for name, ref in zip(("gq", "gk", "gv"), fd[:3]):
        assert np.allclose(ok[name][0, 0], ref, atol=1e-7)
    bad = _gg_variant(*xs, True, 0.8, bug)
    worst = max(np.abs(bad[n][0, 0] - np.asarray(r)).max() for n, r in zip(("gq", "gk", "gv"), fd[:3]))
    assert worst > 1e-3, (bug, worst)
