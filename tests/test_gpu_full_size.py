"""GPU parity at the benchmark configurations, at full size, through the
public API (``triton_attention`` + ``autograd.grad``) with the library
choosing its own split of every streamed loop:

  C4  b1 h1 d64 fp16, T in {512, ..., 16384} x {non-causal, causal}, both
      save_p_triton_full and recompute (C3 is the T = 8192 causal point);
  C2  b2 h4 T2048 d128 fp16 non-causal, save_p forward + first backward;
  C5  b4 h16 T8192 d128 bf16 causal (q, k, v scaled by 0.5), full grad-grad;
  and beyond the reference's sweep, b1 h1 d64 fp16 causal at T = 32768 and
  65536 in recompute mode (the LSE-only mode such lengths need);
  TTT_W512 and TTT_W512_8K, the reference TTT model's windowed attention at
  the sizes the benchmark runs (b8 h6 d64, local window of 512; T1024 fp32
  and T8192 bf16), through ``windowed_attention``.

Reference values: float64 closed forms on the CPU, one block of query rows at
a time (oracle/blocked.py), on the same dtype-rounded inputs.  C5 compares two
(b, h) slices with them (the first, and the last, whose P lies past 2^31
elements) and every one of its 64 slices with the same closed forms in
float32 on the GPU.  P is compared over whole rows: the masked tiles must hold
exact zeros.

Tolerances (tests/_util.py): fp16/bf16 relative Frobenius <= 2e-2 per (b, h)
slice and tensor; LSE max-abs <= 2e-3.
"""
import math
import time

import pytest
import torch

from oracle import blocked
from tests._util import REL_FRO_16, check
from testtimeideas_amd import _lib, workloads
from testtimeideas_amd.ttt_e2e import windowed_attention
from ttt_kernels import triton_attention

pytestmark = pytest.mark.gpu

SWEEP_T = (512, 1024, 2048, 4096, 8192, 16384)
LSE_ABS_16 = 2e-3
GG_NAMES = ("o", "dq", "dk", "dv", "gq", "gk", "gv")
FB_NAMES = ("o", "dq", "dk", "dv")


def _log(msg):
    print(msg, flush=True)


def _gpu_step(xs, causal, scale, mode, gradgrad=True):
    """O, (dQ, dK, dV) and, with gradgrad, the VJP of (dQ, dK, dV) with
    cotangents (rq, rk, rv); plus P (save_p modes) and the forward's LSE."""
    q, k, v, do, rq, rk, rv = (x.cuda() for x in xs)
    q, k, v = (t.requires_grad_(True) for t in (q, k, v))
    o = triton_attention(q, k, v, causal=causal, scale=scale, bwd_mode=mode)
    probs = o.grad_fn.saved_probs
    dq, dk, dv = torch.autograd.grad(o, (q, k, v), do, create_graph=gradgrad)
    out = dict(o=o.detach(), dq=dq.detach(), dk=dk.detach(), dv=dv.detach(), p=probs[0] if probs else None)
    if gradgrad:
        out["gq"], out["gk"], out["gv"] = torch.autograd.grad((dq, dk, dv), (q, k, v), (rq, rk, rv))
    with torch.no_grad():
        out["lse"] = _lib.fwd(q.detach(), k.detach(), v.detach(), causal, scale, out["p"] is not None)[1]
    torch.cuda.synchronize()
    return out


class _PErr:
    """Relative Frobenius error of the GPU's P against the oracle's, summed
    over row blocks; also checks that the keys past each block's last visible
    key hold exact zeros."""

    def __init__(self, p_gpu, causal):
        self.p = p_gpu
        self.causal = causal
        self.num = 0.0
        self.den = 0.0
        self.nonzero_masked = 0

    def __call__(self, r0, r1, p_ref):
        c1 = p_ref.shape[1]
        got = self.p[r0:r1].to(device=p_ref.device, dtype=p_ref.dtype)
        self.num += float(((got[:, :c1] - p_ref) ** 2).sum())
        self.den += float((p_ref ** 2).sum())
        self.nonzero_masked += int((got[:, c1:] != 0).sum())
        if self.causal:  # the entries above the diagonal inside the block's columns
            rows = torch.arange(r0, r1, device=p_ref.device)[:, None]
            cols = torch.arange(c1, device=p_ref.device)[None, :]
            self.nonzero_masked += int(((got[:, :c1] != 0) & (cols > rows)).sum())

    def err(self):
        return math.sqrt(self.num / max(self.den, 1e-300))


def _oracle_slice(xs, bi, hi, causal, scale, gradgrad, p_gpu=None, device="cpu", dtype=torch.float64,
                  block=512):
    args = [x[bi, hi].to(device=device, dtype=dtype) for x in xs]
    if not gradgrad:
        args[4:] = [None, None, None]
    perr = None if p_gpu is None else _PErr(p_gpu[bi, hi], causal)
    ref = blocked.double_backward_blocked(*args, causal, scale, block=block, on_p=perr, gradgrad=gradgrad)
    return ref, perr


def _compare_slice(tag, got, ref, perr, bi, hi, dtype, names):
    errs = {}
    for n in names:
        errs[n] = check(f"{tag} ({bi},{hi}) {n}", got[n][bi, hi], ref[n], dtype)
    lse_err = float((got["lse"][bi, hi].double().cpu() - ref["lse"].double().cpu()).abs().max())
    assert lse_err <= LSE_ABS_16, f"{tag} ({bi},{hi}) lse max-abs {lse_err:.3e} > {LSE_ABS_16}"
    errs["lse"] = lse_err
    if perr is not None:
        errs["p"] = perr.err()
        assert perr.nonzero_masked == 0, f"{tag} ({bi},{hi}): {perr.nonzero_masked} masked P entries not zero"
        assert errs["p"] <= REL_FRO_16, f"{tag} ({bi},{hi}) p rel-Frobenius {errs['p']:.3e} > {REL_FRO_16}"
    return errs


def _split_note(cfg, xs):
    pr = _lib._problem(xs[0], cfg.causal, cfg.scale)
    notes = []
    for name, entry, lp in (("fwd", _lib.ENTRY_FWD_P, True), ("gg_row", _lib.ENTRY_GG_ROW, True),
                            ("gg_col", _lib.ENTRY_GG_COL, True)):
        c, n, sl = _lib.split_info(pr, entry, lp)
        notes.append(f"{name}: chunk {c} x{n} (slots {sl})")
    return "; ".join(notes)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("t", SWEEP_T)
def test_c4_sweep_point(t, causal):
    """One point of the C4 sweep (C3 at T = 8192 causal): save_p_triton_full
    and recompute against the float64 row-block oracle; P over whole rows."""
    cfg = workloads.sweep_config(t, causal)
    xs = list(workloads.make_inputs(cfg, seed=0).values())
    _log(f"[case] C4 T={t} causal={causal}: {_split_note(cfg, xs)}")
    t0 = time.time()
    runs = {mode: _gpu_step(xs, causal, cfg.scale, mode) for mode in ("save_p_triton_full", "recompute")}
    _log(f"  gpu steps done ({time.time() - t0:.1f} s)")
    t0 = time.time()
    ref, perr = _oracle_slice(xs, 0, 0, causal, cfg.scale, True, p_gpu=runs["save_p_triton_full"]["p"])
    _log(f"  float64 oracle done ({time.time() - t0:.1f} s)")
    for mode, got in runs.items():
        errs = _compare_slice(f"C4 T={t} causal={causal} {mode}", got, ref,
                              perr if mode == "save_p_triton_full" else None, 0, 0, torch.float16, GG_NAMES)
        _log(f"  {mode}: " + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()))


def test_c2_full():
    """C2: b2 h4 T2048 d128 fp16 non-causal, save_p forward + first backward;
    every (b, h) slice against the float64 oracle."""
    cfg = workloads.CONFIGS["C2"]
    xs = list(workloads.make_inputs(cfg, seed=0).values())
    _log(f"[case] C2: {_split_note(cfg, xs)}")
    got = _gpu_step(xs, cfg.causal, cfg.scale, cfg.bwd_mode, gradgrad=False)
    assert got["p"] is not None and got["p"].shape == (2, 4, 2048, 2048)
    for bi in range(cfg.b):
        for hi in range(cfg.h):
            ref, perr = _oracle_slice(xs, bi, hi, cfg.causal, cfg.scale, False, p_gpu=got["p"])
            errs = _compare_slice("C2", got, ref, perr, bi, hi, torch.float16, FB_NAMES)
            _log(f"  ({bi},{hi}): " + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()))


def test_c5_full_launch():
    """C5: b4 h16 T8192 d128 bf16 causal, full grad-grad in one launch of each
    kernel over all 64 slices (XCD-remapped grid, P of 2^32 elements).  Slices
    (0, 0) and (3, 15) against the float64 oracle; every slice against the
    same closed forms in float32 on the GPU; every output finite."""
    cfg = workloads.CONFIGS["C5"]
    xs = list(workloads.make_inputs(cfg, seed=0).values())
    _log(f"[case] C5: {_split_note(cfg, xs)}")
    got = _gpu_step(xs, cfg.causal, cfg.scale, cfg.bwd_mode)
    assert got["p"].shape == (4, 16, 8192, 8192)
    for n in GG_NAMES + ("lse",):
        assert bool(torch.isfinite(got[n]).all()), f"C5 {n}: non-finite values"
    for bi, hi in ((0, 0), (3, 15)):
        t0 = time.time()
        ref, perr = _oracle_slice(xs, bi, hi, cfg.causal, cfg.scale, True, p_gpu=got["p"])
        errs = _compare_slice("C5 float64", got, ref, perr, bi, hi, torch.bfloat16, GG_NAMES)
        _log(f"  float64 ({bi},{hi}) [{time.time() - t0:.1f} s]: " + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()))
    xg = [x.cuda() for x in xs]
    worst = {}
    for bi in range(cfg.b):
        for hi in range(cfg.h):
            ref, perr = _oracle_slice(xg, bi, hi, cfg.causal, cfg.scale, True, p_gpu=got["p"], device="cuda",
                                      dtype=torch.float32, block=2048)
            errs = _compare_slice("C5 float32", got, ref, perr, bi, hi, torch.bfloat16, GG_NAMES)
            for k, v in errs.items():
                worst[k] = max(worst.get(k, 0.0), v)
    _log("  float32, worst over 64 slices: " + ", ".join(f"{k} {v:.2e}" for k, v in worst.items()))


@pytest.mark.parametrize("t", [32768, 65536])
def test_long_sequence_recompute(t):
    """T = 32768 and 65536, b1 h1 d64 fp16 causal, recompute mode: every
    output against the row-block closed forms in float32 on the GPU (the
    float64 CPU oracle would take minutes at these lengths)."""
    cfg = workloads.sweep_config(t, True)
    xs = list(workloads.make_inputs(cfg, seed=0).values())
    _log(f"[case] long T={t} recompute: {_split_note(cfg, xs)}")
    t0 = time.time()
    got = _gpu_step(xs, True, cfg.scale, "recompute")
    _log(f"  gpu step done ({time.time() - t0:.1f} s)")
    for n in GG_NAMES + ("lse",):
        assert bool(torch.isfinite(got[n]).all()), f"T={t} {n}: non-finite values"
    xg = [x.cuda() for x in xs]
    ref, _ = _oracle_slice(xg, 0, 0, True, cfg.scale, True, device="cuda", dtype=torch.float32, block=2048)
    errs = _compare_slice(f"long T={t}", got, ref, None, 0, 0, torch.float16, GG_NAMES)
    _log("  " + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()))


def _gpu_window_step(xs, window, local, mode):
    """O, (dQ, dK, dV) and the VJP of (dQ, dK, dV) with (rq, rk, rv) through
    windowed_attention, as the TTT benchmark runs it."""
    q, k, v, do, rq, rk, rv = (x.cuda() for x in xs)
    q, k, v = (t.requires_grad_(True) for t in (q, k, v))
    o = windowed_attention(q, k, v, window, local=local, bwd_mode=mode)
    dq, dk, dv = torch.autograd.grad(o, (q, k, v), do, create_graph=True)
    gq, gk, gv = torch.autograd.grad((dq, dk, dv), (q, k, v), (rq, rk, rv))
    torch.cuda.synchronize()
    return dict(o=o.detach(), dq=dq.detach(), dk=dk.detach(), dv=dv.detach(), gq=gq, gk=gk, gv=gv)


@pytest.mark.parametrize("name", ["TTT_W512", "TTT_W512_8K"])
def test_ttt_window_full(name):
    """The benchmark's TTT workloads at full size (b8 h6 d64, local window
    512): three (b, h) slices against the float64 row-block closed forms with
    the same window (oracle/blocked.py, pinned to the dense closed forms with
    the window as a bias); fp32 max-abs <= 1e-5, bf16 relative Frobenius <=
    2e-2; bf16 also every one of the 48 slices against the same closed forms
    in float32 on the GPU."""
    cfg = workloads.CONFIGS[name]
    local = cfg.window_kind == "local"
    xs = list(workloads.make_inputs(cfg, seed=0).values())
    _log(f"[case] {name}: b{cfg.b} h{cfg.h} T{cfg.t} {cfg.dtype} window {cfg.window} ({cfg.window_kind})")
    got = _gpu_window_step(xs, cfg.window, local, cfg.bwd_mode)
    for n in GG_NAMES:
        assert bool(torch.isfinite(got[n]).all()), f"{name} {n}: non-finite values"
    dt = cfg.torch_dtype
    for bi, hi in ((0, 0), (3, 2), (cfg.b - 1, cfg.h - 1)):
        args = [x[bi, hi].double() for x in xs]
        ref = blocked.double_backward_blocked(*args, True, cfg.scale, block=512, window=cfg.window, local=local)
        errs = {n: check(f"{name} ({bi},{hi}) {n}", got[n][bi, hi], ref[n], dt) for n in GG_NAMES}
        _log(f"  float64 ({bi},{hi}): " + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()))
    if dt != torch.float32:
        xg = [x.cuda() for x in xs]
        worst = {}
        for bi in range(cfg.b):
            for hi in range(cfg.h):
                args = [x[bi, hi].float() for x in xg]
                ref = blocked.double_backward_blocked(*args, True, cfg.scale, block=1024, window=cfg.window,
                                                      local=local)
                for n in GG_NAMES:
                    worst[n] = max(worst.get(n, 0.0), check(f"{name} f32 ({bi},{hi}) {n}", got[n][bi, hi],
                                                            ref[n], dt))
        _log("  float32, worst over 48 slices: " + ", ".join(f"{k} {v:.2e}" for k, v in worst.items()))
