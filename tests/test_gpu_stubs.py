"""GPU parity of the reference-named launchers and helper Functions of
``ttt_kernels.backward_stubs`` (reference backward_stubs.py:22-548), each
called as the reference's callers call it, against the float64 closed forms
on the same dtype-rounded inputs:

  triton_attn_bwd_dv_from_p(p, dO)          dV = P^T dO   (P from a causal or
                                            full save_p forward, read whole)
  triton_attn_rowsum_from_p(p, dO, v)       rowsum = sum_n P o (dO V^T)
  triton_attn_bwd_dqdk_from_p(..., rowsum)  dQ, dK with the row statistic given
  triton_attn_bwd_dv / _dq / _dk            recompute-mode first backward
  triton_attn_bwd2 / 2_dq / 2_dk / 2_dv     the exact double backward
  TritonDvFn, TritonRowSumFn, TritonDqDkFn  forward on the kernels; backward
                                            against float64 autograd of the
                                            function the forward computes

Tolerances: fp16/bf16 relative Frobenius <= 2e-2 (tests/_util.py); fp32
max-abs <= 1e-5, for the helper Functions' VJPs times the reference's largest
magnitude where that exceeds 1 (tests/_util.py: check_f32_scaled).
"""
import math

import pytest
import torch

from oracle import closed_form as cf
from tests._util import check, check_f32_scaled
from ttt_kernels import backward_stubs as bs
from ttt_kernels import triton_attention

pytestmark = pytest.mark.gpu

DT = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}


def _inputs(b, h, t, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(b, h, t, d, generator=g).to(dtype) for _ in range(7)]


def _ref(xs, causal, scale):
    return cf.double_backward(*(x.double().numpy() for x in xs), causal, scale)


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("causal", [False, True])
def test_launchers_from_saved_p(dtype, causal):
    """The save_p flow of the reference's backward (triton_attention.py:354-378):
    P from ctx.saved_probs, then dv_from_p (no causal flag: it reads all of
    P), rowsum_from_p and dqdk_from_p.  The caching allocator is first handed
    NaN-filled blocks of P's size, so tiles the forward left unwritten would
    show up as NaN."""
    dt = DT[dtype]
    b, h, t, d = 1, 2, 200, 64
    xs = _inputs(b, h, t, d, dt, seed=31)
    scale = 1.0 / math.sqrt(d)
    print(f"[case] launchers from P dtype={dtype} causal={causal}", flush=True)
    junk = [torch.full((b, h, t, t), float("nan"), dtype=dt, device="cuda") for _ in range(4)]
    del junk
    q, k, v, do = (x.cuda() for x in xs[:4])
    leaves = [x.detach().requires_grad_(True) for x in (q, k, v)]
    o = triton_attention(*leaves, causal=causal, scale=scale, bwd_mode="save_p_triton_full")
    p = o.grad_fn.saved_probs[0]
    torch.cuda.synchronize()
    ref = _ref(xs, causal, scale)
    assert bool(torch.isfinite(p).all()), "P holds non-finite values"
    check("p", p, ref["p"], dt)
    if causal:
        upper = torch.triu(torch.ones(t, t, dtype=torch.bool, device="cuda"), 1)
        assert int((p[..., upper] != 0).sum()) == 0, "masked entries of P are not zero"
    dv = bs.triton_attn_bwd_dv_from_p(p, do)
    rs = bs.triton_attn_rowsum_from_p(p, do, v, causal=causal)
    dq, dk = bs.triton_attn_bwd_dqdk_from_p(q, k, v, do, p, rs, causal=causal, scale=scale)
    rs_ref = torch.from_numpy(ref["rowsum"]).float().cuda()
    dq2, dk2 = bs.triton_attn_bwd_dqdk_from_p(q, k, v, do, p, rs_ref, causal=causal, scale=scale)
    torch.cuda.synchronize()
    assert rs.dtype == torch.float32 and rs.shape == (b, h, t)
    check("dv", dv, ref["dv"], dt)
    check("rowsum", rs, ref["rowsum"], dt)
    for name, got in (("dq", dq), ("dk", dk), ("dq (oracle rowsum)", dq2), ("dk (oracle rowsum)", dk2)):
        check(name, got, ref[name.split()[0]], dt)


@pytest.mark.parametrize("causal", [False, True])
def test_recompute_launchers(causal):
    dt = torch.float16
    xs = _inputs(2, 1, 150, 64, dt, seed=32)
    print(f"[case] recompute launchers causal={causal}", flush=True)
    q, k, v, do = (x.cuda() for x in xs[:4])
    dv = bs.triton_attn_bwd_dv(q, k, v, do, causal=causal, scale=0.125)
    dq = bs.triton_attn_bwd_dq(q, k, v, do, causal=causal, scale=0.125)
    dk = bs.triton_attn_bwd_dk(q, k, v, do, causal=causal, scale=0.125)
    torch.cuda.synchronize()
    ref = _ref(xs, causal, 0.125)
    for n, x in (("dv", dv), ("dq", dq), ("dk", dk)):
        check(n, x, ref[n], dt)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("causal", [False, True])
def test_bwd2_launchers(dtype, causal):
    dt = DT[dtype]
    xs = _inputs(1, 2, 130, 64, dt, seed=33)
    print(f"[case] bwd2 dtype={dtype} causal={causal}", flush=True)
    q, k, v, do, rq, rk, rv = (x.cuda() for x in xs)
    gq, gk, gv, gdo = bs.triton_attn_bwd2(q, k, v, do, rq, rk, rv, causal=causal)
    one = [bs.triton_attn_bwd2_dq(q, k, v, do, rq, rk, rv, causal=causal),
           bs.triton_attn_bwd2_dk(q, k, v, do, rq, rk, rv, causal=causal),
           bs.triton_attn_bwd2_dv(q, k, v, do, rq, rk, rv, causal=causal)]
    torch.cuda.synchronize()
    ref = _ref(xs, causal, 0.125)
    for n, x in (("gq", gq), ("gk", gk), ("gv", gv), ("gdo", gdo)):
        check(n, x, ref[n], dt)
    # the single-output launchers run the double backward without GdO (other
    # kernel variants: equal to rounding, not bitwise)
    for n, x in zip(("gq", "gk", "gv"), one):
        check(n + " alone", x, ref[n], dt)


def _f64_vjp(fn, inputs, cotangents):
    xs = [x.detach().double().cpu().requires_grad_(True) for x in inputs]
    outs = fn(*xs)
    outs = outs if isinstance(outs, tuple) else (outs,)
    gs = torch.autograd.grad(outs, xs, [c.double().cpu() for c in cotangents], allow_unused=True)
    return [torch.zeros_like(x) if g is None else g for x, g in zip(xs, gs)], [o.detach() for o in outs]


def _mt(x):
    return x.transpose(-2, -1)


@pytest.mark.parametrize("causal", [False, True])
def test_helper_functions(causal):
    """TritonDvFn, TritonRowSumFn and TritonDqDkFn in fp32: forward on the
    kernels, backward through autograd on the GPU, both against float64."""
    dt = torch.float32
    b, h, t, d = 1, 2, 96, 64
    s = 0.125
    xs = _inputs(b, h, t, d, dt, seed=34)
    print(f"[case] helper Functions causal={causal}", flush=True)
    q, k, v, do = (x.cuda() for x in xs[:4])
    leaves = [x.detach().requires_grad_(True) for x in (q, k, v)]
    o = triton_attention(*leaves, causal=causal, scale=s, bwd_mode="save_p")
    p = o.grad_fn.saved_probs[0].detach().clone()
    g = torch.Generator().manual_seed(35)
    cot = [torch.randn(b, h, t, d, generator=g).cuda(), torch.randn(b, h, t, generator=g).cuda(),
           torch.randn(b, h, t, d, generator=g).cuda(), torch.randn(b, h, t, d, generator=g).cuda()]

    def leaf(x):
        return x.detach().clone().requires_grad_(True)

    # TritonDvFn
    pl, dol = leaf(p), leaf(do)
    dv = bs.TritonDvFn.apply(pl, dol)
    got = torch.autograd.grad(dv, (pl, dol), cot[0])
    ref, (dv_ref,) = _f64_vjp(lambda p_, do_: _mt(p_) @ do_, (p, do), (cot[0],))
    check_f32_scaled("dv", dv, dv_ref)
    for n, a, r in zip(("grad_p", "grad_do"), got, ref):
        check_f32_scaled(n, a, r)
    # TritonRowSumFn
    pl, dol, vl = leaf(p), leaf(do), leaf(v)
    rs = bs.TritonRowSumFn.apply(pl, dol, vl, causal)
    got = torch.autograd.grad(rs, (pl, dol, vl), cot[1])
    ref, (rs_ref,) = _f64_vjp(lambda p_, do_, v_: (p_ * (do_ @ _mt(v_))).sum(-1), (p, do, v), (cot[1],))
    check_f32_scaled("rowsum", rs, rs_ref)
    for n, a, r in zip(("grad_p", "grad_do", "grad_v"), got, ref):
        check_f32_scaled(n, a, r)
    # TritonDqDkFn with P and rowsum as independent inputs
    rs0 = rs.detach()
    ins = [leaf(x) for x in (q, k, v, do, p, rs0)]
    dq, dk = bs.TritonDqDkFn.apply(*ins, s, causal)
    got = torch.autograd.grad((dq, dk), ins, (cot[2], cot[3]))

    def dqdk(q_, k_, v_, do_, p_, r_):
        ds = p_ * (do_ @ _mt(v_) - r_.unsqueeze(-1))
        return s * (ds @ k_), s * (_mt(ds) @ q_)

    ref, (dq_ref, dk_ref) = _f64_vjp(dqdk, (q, k, v, do, p, rs0), (cot[2], cot[3]))
    check_f32_scaled("dq", dq, dq_ref)
    check_f32_scaled("dk", dk, dk_ref)
    for n, a, r in zip(("grad_q", "grad_k", "grad_v", "grad_do", "grad_p", "grad_rowsum"), got, ref):
        check_f32_scaled(n, a, r)
