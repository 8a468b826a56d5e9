"""GPU parity of key windows and additive score biases, through the C ABI and
through the reference-shaped drop-ins (``GradGradAttentionFn``,
``WindowedSelfAttention``), against the float64 oracle on the same
(dtype-rounded) inputs: the closed forms with the reference's masks as an
additive bias (oracle.masks), and the reference's chunked window loop.

Tolerances: fp16/bf16 relative Frobenius <= 2e-2; fp32 max-abs <= 1e-5.
"""
import math

import numpy as np
import pytest
import torch

from oracle import closed_form as cf, masks, math_path
from tests._util import check
from testtimeideas_amd import _lib
from testtimeideas_amd.ttt_e2e import (GradGradAttentionFn, WindowedSelfAttention, make_window_mask,
                                       local_window_mask, windowed_attention)

pytestmark = pytest.mark.gpu

DT = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}
NAMES = ("o", "dq", "dk", "dv", "gq", "gk", "gv", "gdo")


def _inputs(b, h, t, d, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(b, h, t, d, generator=g).to(dtype) for _ in range(7)]


def _run(xs, mask, scale, save_p):
    q, k, v, do, gq, gk, gv = (x.cuda() for x in xs)
    o, lse, p = _lib.fwd(q, k, v, mask, scale, save_p)
    dq, dk, dv, rowsum = _lib.bwd(q, k, v, o, do, lse, p, mask, scale)
    GQ, GK, GV, GdO = _lib.gg(q, k, v, do, lse, p, rowsum, gq, gk, gv, mask, scale, True)
    if p is not None:  # the tiles the forward leaves unwritten, zeroed for the comparison
        _lib.fill_masked_p(p, mask)
    torch.cuda.synchronize()
    return dict(o=o, lse=lse, p=p, dq=dq, dk=dk, dv=dv, rowsum=rowsum, gq=GQ, gk=GK, gv=GV, gdo=GdO)


def _tiles_written(bias_np):
    """Elements of P the kernels write: the 64x64 tiles that hold a visible pair."""
    t = bias_np.shape[-1]
    vis = np.isfinite(bias_np)
    nb = -(-t // 64)
    out = np.zeros((t, t), bool)
    for i in range(nb):
        for j in range(nb):
            if vis[i * 64:(i + 1) * 64, j * 64:(j + 1) * 64].any():
                out[i * 64:(i + 1) * 64, j * 64:(j + 1) * 64] = True
    return out


def _compare(out, ref, dtype, p_mask=None):
    for n in NAMES:
        check(n, out[n], ref[n], dtype)
    check("lse", out["lse"], ref["lse"], torch.float32, abs_tol=2e-5 if dtype == torch.float32 else 2e-3)
    check("rowsum", out["rowsum"], ref["rowsum"], dtype)
    if out["p"] is not None and p_mask is not None:
        got = out["p"].double().cpu().numpy()
        check("p", got[..., p_mask], ref["p"][..., p_mask], dtype)
        # after fill_masked_p, the tiles no row of their block sees hold zeros
        assert not np.any(got[..., ~p_mask]), "P outside the visible tiles is not zero"


def _window_case(dtype, d, t, w, kind, save_p, b=1, h=2, seed=0):
    dt = DT[dtype]
    xs = _inputs(b, h, t, d, dt, seed=seed)
    scale = 1.0 / math.sqrt(d)
    bias = masks.window_bias(t, w) if kind == _lib.WINDOW_SLIDING else masks.local_bias(t, w)
    print(f"[case] window dtype={dtype} d={d} t={t} w={w} kind={kind} save_p={save_p}", flush=True)
    out = _run(xs, _lib.Mask(causal=True, window=w, window_kind=kind), scale, save_p)
    ref = cf.double_backward(*(x.double().numpy() for x in xs), False, scale, bias)
    _compare(out, ref, dt, _tiles_written(bias))


@pytest.mark.parametrize("kind", [_lib.WINDOW_SLIDING, _lib.WINDOW_LOCAL])
@pytest.mark.parametrize("t,w", [(100, 2), (333, 64), (333, 100), (700, 200), (700, 512), (512, 128)])
@pytest.mark.parametrize("save_p", [True, False])
def test_window_fp16(kind, t, w, save_p):
    _window_case("fp16", 64, t, w, kind, save_p)


@pytest.mark.parametrize("dtype,d", [("bf16", 64), ("fp32", 64), ("fp16", 128), ("bf16", 128), ("fp32", 128)])
@pytest.mark.parametrize("kind", [_lib.WINDOW_SLIDING, _lib.WINDOW_LOCAL])
@pytest.mark.parametrize("save_p", [True, False])
def test_window_dtypes(dtype, d, kind, save_p):
    _window_case(dtype, d, 300, 130, kind, save_p)


@pytest.mark.parametrize("chunk", [1, 2, 3])
@pytest.mark.parametrize("kind", [_lib.WINDOW_SLIDING, _lib.WINDOW_LOCAL])
@pytest.mark.parametrize("save_p", [True, False])
def test_window_split_chunks(chunk, kind, save_p):
    """Forced splits: chunks of a tile or two, where some rows see no key of a
    chunk (their partial max is -inf and sum 0)."""
    with _lib.split_chunk(chunk):
        _window_case("fp16", 64, 700, 100, kind, save_p, seed=chunk)


@pytest.mark.parametrize("kind", [_lib.WINDOW_SLIDING, _lib.WINDOW_LOCAL])
@pytest.mark.parametrize("save_p", [True, False])
def test_window_one_is_identity(kind, save_p):
    """W = 1: every query sees only its own key, P = I.  Then O = V,
    dQ = dK = 0, dV = dO, and in the double backward GQ = GK = GV = 0 and
    GdO = gV (fp32; in 16-bit types GQ is a difference of rounded terms of
    size |dO gV^T| that cancel exactly, so only fp32 pins it)."""
    xs = _inputs(1, 2, 200, 64, torch.float32, seed=21)
    print(f"[case] window W=1 kind={kind} save_p={save_p}", flush=True)
    out = _run(xs, _lib.Mask(causal=True, window=1, window_kind=kind), 0.125, save_p)
    q, k, v, do, gq, gk, gv = xs
    z = torch.zeros_like(q)
    want = dict(o=v, dq=z, dk=z, dv=do, gq=z, gk=z, gv=z, gdo=gv)
    for n in NAMES:
        check(n, out[n], want[n].double(), torch.float32, abs_tol=2e-5)


def test_window_at_least_t_is_causal():
    xs = _inputs(1, 2, 200, 64, torch.float16, seed=4)
    a = _run(xs, _lib.Mask(causal=True, window=200), 0.125, False)
    b = _run(xs, True, 0.125, False)
    for n in NAMES:
        assert torch.equal(a[n], b[n]), n


def _bias_case(bias, t, causal, save_p, dtype=torch.float16, b=2, h=2, seed=0, split=0):
    xs = _inputs(b, h, t, 64, dtype, seed=seed)
    q = xs[0]
    kb = _lib.prep_bias(bias, b, h, t, dtype, "cuda")
    out = _run(xs, _lib.Mask(causal=causal, bias=kb), 0.125, save_p) if not split else None
    if split:
        with _lib.split_chunk(split):
            out = _run(xs, _lib.Mask(causal=causal, bias=kb), 0.125, save_p)
    bn = bias.to(dtype).double().numpy()
    ref = cf.double_backward(*(x.double().numpy() for x in xs), causal, 0.125, bn)
    # P: every tile is written without causality, the lower block triangle with it
    written = _tiles_written(np.where(np.tri(t, dtype=bool), 0.0, -np.inf)) if causal else np.ones((t, t), bool)
    _compare(out, ref, dtype, written)
    return out


@pytest.mark.parametrize("t", [100, 256])
@pytest.mark.parametrize("save_p", [True, False])
@pytest.mark.parametrize("causal", [False, True])
def test_bias_random_full(t, save_p, causal):
    print(f"[case] bias full t={t} save_p={save_p} causal={causal}", flush=True)
    g = torch.Generator().manual_seed(t)
    _bias_case(torch.randn(2, 2, t, t, generator=g), t, causal, save_p)


@pytest.mark.parametrize("save_p", [True, False])
def test_bias_broadcast_shapes(save_p):
    print(f"[case] bias broadcast save_p={save_p}", flush=True)
    t = 192
    g = torch.Generator().manual_seed(7)
    _bias_case(torch.randn(t, t, generator=g), t, False, save_p)          # [T, T] over B, H
    _bias_case(torch.randn(1, 2, 1, t, generator=g), t, False, save_p)    # per-head key bias over rows
    kp = torch.zeros(2, 1, 1, t)
    kp[0, ..., 150:] = float("-inf")                                      # key padding of batch 0
    _bias_case(kp, t, False, save_p)


@pytest.mark.parametrize("save_p", [True, False])
def test_bias_split_and_bf16(save_p):
    print(f"[case] bias split/bf16 save_p={save_p}", flush=True)
    g = torch.Generator().manual_seed(8)
    _bias_case(torch.randn(1, 1, 600, 600, generator=g), 600, True, save_p, split=2)
    _bias_case(torch.randn(1, 1, 300, 300, generator=g), 300, False, save_p, dtype=torch.bfloat16)
    _bias_case(torch.randn(1, 1, 300, 300, generator=g), 300, False, save_p, dtype=torch.float32)


def test_triangle_bias_equals_causal_flag():
    """A -inf upper triangle as a bias gives the causal results."""
    t = 256
    tri = torch.zeros(t, t).masked_fill(torch.ones(t, t, dtype=torch.bool).triu(1), float("-inf"))
    xs = _inputs(1, 2, t, 64, torch.float16, seed=9)
    a = _run(xs, _lib.Mask(bias=_lib.prep_bias(tri, 1, 2, t, torch.float16, "cuda")), 0.125, False)
    b = _run(xs, True, 0.125, False)
    for n in NAMES:
        check(n, a[n], b[n].double().cpu(), torch.float16, rel_tol=2e-3)


# ----------------------------------------------------------------------------- drop-ins
def _grads_math(q, k, v, do, rq, rk, rv, mask):
    ref = math_path.gradgrad_step(*(x.double().cpu() for x in (q, k, v, do, rq, rk, rv)), False,
                                  1.0 / math.sqrt(q.size(-1)), do_requires_grad=True,
                                  attn_mask=None if mask is None else mask.double().cpu())
    return ref


def _grads_ours(q, k, v, do, rq, rk, rv, mask, fn):
    q, k, v = (x.cuda().requires_grad_(True) for x in (q, k, v))
    do = do.cuda().requires_grad_(True)
    o = fn(q, k, v, None if mask is None else mask.cuda())
    dq, dk, dv = torch.autograd.grad(o, (q, k, v), do, create_graph=True)
    s = (dq.float() * rq.cuda()).sum() + (dk.float() * rk.cuda()).sum() + (dv.float() * rv.cuda()).sum()
    g = torch.autograd.grad(s, (q, k, v, do))
    return dict(o=o, dq=dq, dk=dk, dv=dv, gq=g[0], gk=g[1], gv=g[2], gdo=g[3])


@pytest.mark.parametrize("case", ["window_mask", "local_rect", "wide_rect", "none_rect", "none"])
@pytest.mark.parametrize("dtype", ["fp16", "fp32"])
def test_gradgrad_attention_fn(case, dtype):
    """GradGradAttentionFn.apply with the masks the reference's TTT model
    builds (make_window_mask; _local_window_mask for a last partial chunk,
    fewer queries than keys), a random mask with more queries than keys, and
    no mask; full grad-grad step against autograd of the reference's math."""
    dt = DT[dtype]
    b, h, d = 2, 2, 64
    lq, lk = {"window_mask": (300, 300), "local_rect": (76, 200), "wide_rect": (150, 90), "none_rect": (100, 60),
              "none": (128, 128)}[case]
    g = torch.Generator().manual_seed({"window_mask": 1, "local_rect": 2, "wide_rect": 3, "none_rect": 4,
                                       "none": 5}[case])
    q, do, rq = (torch.randn(b, h, lq, d, generator=g).to(dt) for _ in range(3))
    k, v, rk, rv = (torch.randn(b, h, lk, d, generator=g).to(dt) for _ in range(4))
    if case == "window_mask":
        mask = make_window_mask(lq, 128, "cpu", dt).view(1, 1, lq, lq)
    elif case == "local_rect":
        # last partial chunk of T = 1100 with W = 200: queries 1024..1099, keys 900..1099
        mask = local_window_mask(1100 - lq, 1100, 1100 - lk, 1100, 200, "cpu", dt).view(1, 1, lq, lk)
    elif case == "wide_rect":
        mask = torch.randn(1, h, lq, lk, generator=g).to(dt)
    else:
        mask = None
    print(f"[case] GradGradAttentionFn {case} dtype={dtype} lq={lq} lk={lk}", flush=True)
    ours = _grads_ours(q, k, v, do, rq.float(), rk.float(), rv.float(), mask,
                       lambda a, b_, c, m: GradGradAttentionFn.apply(a, b_, c, m))
    ref = _grads_math(q, k, v, do, rq, rk, rv, mask)
    for n in NAMES:
        check(n, ours[n], ref[n], dt)


def test_gradgrad_attention_fn_constant_grad_out():
    """Second-order terms survive a grad_out that does not require grad (the
    reference's need_higher = grad_out.requires_grad drops them)."""
    t, d = 128, 64
    g = torch.Generator().manual_seed(11)
    q, k, v = (torch.randn(1, 2, t, d, generator=g, dtype=torch.float32) for _ in range(3))
    mask = make_window_mask(t, 64, "cpu", torch.float32).view(1, 1, t, t)
    qc, kc, vc = (x.cuda().requires_grad_(True) for x in (q, k, v))
    o = GradGradAttentionFn.apply(qc, kc, vc, mask.cuda())
    w = torch.randn(o.shape, generator=g).cuda()  # constant: loss = sum(o * w)
    dq, dk, dv = torch.autograd.grad((o * w).sum(), (qc, kc, vc), create_graph=True)
    gg = torch.autograd.grad((dq * dq).sum() + (dk * dk).sum() + (dv * dv).sum(), (qc, kc, vc))
    q64, k64, v64 = (x.double().requires_grad_(True) for x in (q, k, v))
    o64 = math_path.attention_masked(q64, k64, v64, mask.double())
    d64 = torch.autograd.grad((o64 * w.double().cpu()).sum(), (q64, k64, v64), create_graph=True)
    g64 = torch.autograd.grad(sum((x * x).sum() for x in d64), (q64, k64, v64))
    for n, a, r in zip(("gq", "gk", "gv"), gg, g64):
        check(n, a, r, torch.float32, abs_tol=1e-5 * max(1.0, float(r.abs().max())))
    assert float(gg[0].abs().max()) > 0


@pytest.mark.parametrize("t,w", [(1100, 512), (1024, 512), (300, 512), (640, 128)])
@pytest.mark.parametrize("save_p", [False, True])
def test_windowed_attention_matches_chunked_loop(t, w, save_p):
    """One launch with the local window equals the reference's loop over
    chunks (restated in oracle.masks.chunked_loop), double backward included."""
    xs = _inputs(1, 2, t, 64, torch.float16, seed=t + w)
    scale = 0.125
    print(f"[case] windowed_attention t={t} w={w} save_p={save_p}", flush=True)
    q, k, v, do, gq, gk, gv = (x.cuda() for x in xs)
    q, k, v = (x.requires_grad_(True) for x in (q, k, v))
    do.requires_grad_(True)
    o = windowed_attention(q, k, v, w, scale=scale, bwd_mode="save_p" if save_p else "recompute")
    dq, dk, dv = torch.autograd.grad(o, (q, k, v), do, create_graph=True)
    s = (dq.float() * gq.float()).sum() + (dk.float() * gk.float()).sum() + (dv.float() * gv.float()).sum()
    GQ, GK, GV, GdO = torch.autograd.grad(s, (q, k, v, do))
    ref = masks.chunked_loop(*(x.double().numpy() for x in xs[:3]), w, scale,
                             *(x.double().numpy() for x in xs[3:]))
    ours = dict(o=o, dq=dq, dk=dk, dv=dv, gq=GQ, gk=GK, gv=GV, gdo=GdO)
    for n in NAMES:
        check(n, ours[n], ref[n], torch.float16)


def test_windowed_self_attention_module():
    """WindowedSelfAttention (same constructor and parameters as the
    reference's) against the reference's loop on the same weights, and a
    meta-gradient (grad of a function of parameter gradients) through it."""
    torch.manual_seed(0)
    d_model, heads, w, t = 256, 4, 128, 300
    mod = WindowedSelfAttention(d_model, heads, w).cuda()
    x = torch.randn(2, t, d_model, device="cuda")
    out = mod(x)
    ref = {n: p.detach().double().cpu() for n, p in mod.named_parameters()}
    xd = x.double().cpu()

    def proj(name):
        y = xd @ ref[name + ".weight"].T + ref[name + ".bias"]
        return y.view(2, t, heads, d_model // heads).transpose(1, 2).numpy()

    o = masks.chunked_loop(proj("q_proj"), proj("k_proj"), proj("v_proj"), w, 1.0 / math.sqrt(d_model // heads))["o"]
    o = torch.from_numpy(o).transpose(1, 2).reshape(2, t, d_model)
    want = o @ ref["out_proj.weight"].T + ref["out_proj.bias"]
    assert float((out.detach().double().cpu() - want).abs().max()) < 1e-4
    # meta-gradient: d/dW of |dL/dW_q|^2, through the attention's double backward
    wq = mod.q_proj.weight
    loss = mod(x).square().mean()
    (gw,) = torch.autograd.grad(loss, (wq,), create_graph=True)
    (meta,) = torch.autograd.grad(gw.square().sum(), (mod.k_proj.weight,))
    assert torch.isfinite(meta).all() and float(meta.abs().max()) > 0
