"""GPU parity of every kernel entry point, called through the C ABI, against the
float64 closed-form oracle on the same (dtype-rounded) inputs.

Tolerances: fp16/bf16 relative Frobenius <= 2e-2; fp32 max-abs <= 1e-5.
"""
import math

import numpy as np
import pytest
import torch

from oracle import closed_form as cf
from tests._util import check, rel_fro, max_abs
from testtimeideas_amd import _lib

pytestmark = pytest.mark.gpu

DT = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}


def _inputs(b, h, t, d, dtype, seed=0, qkv_scale=1.0):
    g = torch.Generator().manual_seed(seed)
    xs = [torch.randn(b, h, t, d, generator=g) for _ in range(7)]
    for i in range(3):
        xs[i] = xs[i] * qkv_scale
    return [x.to(dtype) for x in xs]


def _ref(xs, causal, scale):
    return cf.double_backward(*(x.double().numpy() for x in xs), causal, scale)


def _run(xs, causal, scale, save_p, want_gdo=True):
    """Every entry point once; the double backward twice: as asked (the row
    pass forms all its products) and in the dQ form (no GdO; the row pass
    reads the first backward's dQ), whose results are the *_dq entries."""
    q, k, v, do, gq, gk, gv = (x.cuda() for x in xs)
    o, lse, p = _lib.fwd(q, k, v, causal, scale, save_p)
    dq, dk, dv, rowsum = _lib.bwd(q, k, v, o, do, lse, p, causal, scale)
    GQ, GK, GV, GdO = _lib.gg(q, k, v, do, lse, p, rowsum, gq, gk, gv, causal, scale, want_gdo)
    GQ2, GK2, GV2, _ = _lib.gg(q, k, v, do, lse, p, rowsum, gq, gk, gv, causal, scale, False, dq=dq)
    if p is not None:  # the tiles the forward leaves unwritten, zeroed for the comparison
        _lib.fill_masked_p(p, causal)
    torch.cuda.synchronize()
    return dict(o=o, lse=lse, p=p, dq=dq, dk=dk, dv=dv, rowsum=rowsum, gq=GQ, gk=GK, gv=GV, gdo=GdO,
                gq_dq=GQ2, gk_dq=GK2, gv_dq=GV2)


def _compare(out, ref, dtype, causal, t, names=("o", "dq", "dk", "dv", "gq", "gk", "gv", "gdo")):
    errs = {}
    for n in names:
        if out.get(n) is None:
            continue
        errs[n] = check(n, out[n], ref[n], dtype)
        if out.get(n + "_dq") is not None:
            errs[n + "_dq"] = check(n + "_dq", out[n + "_dq"], ref[n], dtype)
    # row statistics: LSE (natural log) and D
    errs["lse"] = check("lse", out["lse"], ref["lse"], torch.float32, abs_tol=2e-5 if dtype == torch.float32 else 2e-3)
    errs["rowsum"] = check("rowsum", out["rowsum"], ref["rowsum"], dtype)
    if out["p"] is not None:
        # masked entries are zeros (inside active tiles from the forward,
        # elsewhere from fill_masked_p)
        got = out["p"].double().cpu().numpy()
        errs["p"] = check("p", got, ref["p"], dtype)
        if causal:
            assert not np.any(got[..., np.triu(np.ones((t, t), dtype=bool), 1)]), "masked P entries not zero"
    return errs


@pytest.mark.parametrize("dtype", ["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("save_p", [True, False])
def test_all_kernels_small(dtype, d, causal, save_p):
    t = 128
    dt = DT[dtype]
    xs = _inputs(1, 2, t, d, dt, seed=1)
    scale = 1.0 / math.sqrt(d)
    print(f"[case] small dtype={dtype} d={d} causal={causal} save_p={save_p} t={t}", flush=True)
    out = _run(xs, causal, scale, save_p)
    _compare(out, _ref(xs, causal, scale), dt, causal, t)


@pytest.mark.parametrize("t", [1, 37, 64, 100, 191, 257])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("save_p", [True, False])
def test_ragged_lengths(t, causal, save_p):
    dt = torch.float16
    xs = _inputs(2, 1, t, 64, dt, seed=t)
    scale = 0.125
    print(f"[case] ragged t={t} causal={causal} save_p={save_p}", flush=True)
    out = _run(xs, causal, scale, save_p)
    _compare(out, _ref(xs, causal, scale), dt, causal, t)


@pytest.mark.parametrize("t", [37, 191, 257])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("save_p", [True, False])
def test_ragged_lengths_d128(t, causal, save_p):
    """Head dim 128 (16-bit direct-load kernels: two buffer sets, P staged in
    dK/dV) over ragged lengths, unsplit: paired steps, an odd last step and a
    ragged last tile."""
    dt = torch.bfloat16
    xs = _inputs(1, 2, t, 128, dt, seed=t + 1)
    scale = 1.0 / math.sqrt(128)
    print(f"[case] ragged d128 t={t} causal={causal} save_p={save_p}", flush=True)
    out = _run(xs, causal, scale, save_p)
    _compare(out, _ref(xs, causal, scale), dt, causal, t)


@pytest.mark.parametrize("scale", [-0.125, 0.0, 0.37])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("save_p", [True, False])
def test_scale_signs(scale, causal, save_p):
    """Negative and zero scales take the statistics pass's scaled-score path
    (its fused raw-score form needs a positive scale), and in the online pass
    a negated q (negative scale) and masked entries selected after the
    exponential (zero scale, where -inf * 0 is NaN); a positive non-power of
    two takes the fused forms.  Ragged T covers the clamped tiles."""
    dt = torch.float16
    t = 100
    xs = _inputs(1, 2, t, 64, dt, seed=11)
    print(f"[case] scale={scale} causal={causal} save_p={save_p}", flush=True)
    out = _run(xs, causal, scale, save_p)
    _compare(out, _ref(xs, causal, scale), dt, causal, t)


@pytest.mark.parametrize("dtype", ["fp32", "fp16"])
def test_c1_shape_fp32_parity(dtype):
    """C1 shape (b1 h1 T64 d64, non-causal) on the GPU kernels."""
    dt = DT[dtype]
    xs = _inputs(1, 1, 64, 64, dt, seed=0)
    print(f"[case] c1 dtype={dtype}", flush=True)
    for save_p in (True, False):
        out = _run(xs, False, 0.125, save_p)
        _compare(out, _ref(xs, False, 0.125), dt, False, 64)


def test_per_kernel_entry_points_match_fused():
    """The per-kernel entry points (used under timing) give the fused results."""
    xs = _inputs(1, 2, 192, 64, torch.float16, seed=3)
    print("[case] per-kernel vs fused", flush=True)
    a = _run(xs, True, 0.125, True)
    with _lib.kernel_timing() as rec:
        b = _run(xs, True, 0.125, True)
    for n in ("o", "dq", "dk", "dv", "gq", "gk", "gv", "gdo", "rowsum", "lse", "gq_dq", "gk_dq", "gv_dq"):
        assert torch.equal(a[n], b[n]), n
    assert set(rec) >= {"ttt_attn_fwd", "ttt_attn_bwd_dq", "ttt_attn_bwd_dkdv", "ttt_attn_gg_row",
                        "ttt_attn_gg_col"}


def _mask(win):
    """Causal, or a (kind, W) key window."""
    if win is None:
        return True
    return _lib.Mask(causal=True, window=win[1], window_kind=win[0])


@pytest.mark.parametrize("b,h,t,d,dtype,save_p,chunk,win", [
    (1, 2, 192, 64, "fp16", True, 1, None),
    (1, 1, 300, 64, "bf16", True, 2, None),
    (2, 4, 200, 64, "fp16", True, 2, None),
    (2, 4, 200, 64, "fp16", False, 3, None),
    (1, 3, 257, 128, "bf16", True, 2, None),
    (1, 2, 130, 64, "fp32", True, 2, None),
    (1, 1, 1024, 64, "fp16", True, 0, None),
    (1, 2, 700, 64, "fp16", True, 2, (_lib.WINDOW_SLIDING, 200)),
    (1, 1, 640, 64, "bf16", False, 3, (_lib.WINDOW_LOCAL, 128)),
])
def test_fused_backward_entry(b, h, t, d, dtype, save_p, chunk, win):
    """ttt_attn_bwd, whose dK/dV launch also finishes dQ's split blocks, gives
    bitwise the results of ttt_attn_bwd_dq + ttt_attn_bwd_dkdv."""
    import ctypes
    dt = DT[dtype]
    m = _mask(win)
    q, k, v, do = (x.cuda() for x in _inputs(b, h, t, d, dt, seed=t + d)[:4])
    print(f"[case] fused bwd b={b} h={h} t={t} d={d} {dtype} save_p={save_p} chunk={chunk} win={win}", flush=True)
    o, lse, p = _lib.fwd(q, k, v, m, 0.125, save_p)
    with _lib.split_chunk(chunk), _lib.kernel_timing():  # timing: the two per-family entry points
        dq0, dk0, dv0, rs0 = _lib.bwd(q, k, v, o, do, lse, p, m, 0.125)
    pr = _lib._problem(q, m, 0.125, chunk)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    rs = torch.empty(b, h, t, dtype=torch.float32, device=q.device)
    wp, wn, _buf = _lib._workspace(pr, _lib.ENTRY_BWD, q.device)
    _lib._call("ttt_attn_bwd", ctypes.byref(pr), _lib._view(q), _lib._view(k), _lib._view(v), _lib._view(o),
               _lib._view(do), _lib._fptr(lse), _lib._view(p), rs.data_ptr(), _lib._view(dq), _lib._view(dk),
               _lib._view(dv), wp, wn, _lib._stream())
    torch.cuda.synchronize()
    for n, x, y in (("dq", dq, dq0), ("dk", dk, dk0), ("dv", dv, dv0), ("rowsum", rs, rs0)):
        assert torch.equal(x, y), n


@pytest.mark.parametrize("b,h,t,d,dtype,save_p,gdo,chunk,win", [
    (1, 2, 192, 64, "fp16", True, False, 1, None),
    (1, 1, 300, 64, "bf16", True, True, 2, None),
    (2, 4, 200, 64, "fp16", False, False, 2, None),
    (2, 4, 200, 64, "bf16", True, True, 3, None),
    (1, 3, 257, 128, "bf16", True, False, 2, None),
    (1, 2, 190, 128, "fp16", True, True, 2, None),
    (1, 2, 130, 128, "fp32", False, True, 2, None),
    (1, 1, 1024, 64, "fp16", True, False, 0, None),
    (1, 2, 700, 64, "fp16", True, True, 2, (_lib.WINDOW_SLIDING, 200)),
    (1, 1, 640, 64, "bf16", False, False, 3, (_lib.WINDOW_LOCAL, 128)),
])
@pytest.mark.parametrize("use_dq", [False, True])
def test_fused_double_backward_entry(b, h, t, d, dtype, save_p, gdo, chunk, win, use_dq):
    """ttt_attn_gg, whose column launch also finishes the row pass's split
    blocks, gives bitwise the results of ttt_attn_gg_row + ttt_attn_gg_col,
    with and without the first backward's dQ (ignored with GdO)."""
    import ctypes
    dt = DT[dtype]
    m = _mask(win)
    q, k, v, do, gq, gk, gv = (x.cuda() for x in _inputs(b, h, t, d, dt, seed=t + d + 1))
    print(f"[case] fused gg b={b} h={h} t={t} d={d} {dtype} save_p={save_p} gdo={gdo} chunk={chunk} win={win} "
          f"dq={use_dq}", flush=True)
    o, lse, p = _lib.fwd(q, k, v, m, 0.125, save_p)
    dq, _, _, rs = _lib.bwd(q, k, v, o, do, lse, p, m, 0.125)
    if not use_dq:
        dq = None
    with _lib.split_chunk(chunk), _lib.kernel_timing():  # timing: the row and column entry points
        ref = _lib.gg(q, k, v, do, lse, p, rs, gq, gk, gv, m, 0.125, gdo, dq=dq)
    pr = _lib._problem(q, m, 0.125, chunk)
    out = [torch.empty_like(x) for x in (q, k, v)] + [torch.empty_like(do) if gdo else None]
    e = torch.empty(b, h, t, dtype=torch.float32, device=q.device)
    f = torch.empty_like(e)
    wp, wn, _buf = _lib._workspace(pr, _lib.ENTRY_GG, q.device, gdo)
    _lib._call("ttt_attn_gg", ctypes.byref(pr), _lib._view(q), _lib._view(k), _lib._view(v), _lib._view(do),
               _lib._fptr(lse), _lib._view(p), rs.data_ptr(), _lib._view(dq), _lib._view(gq), _lib._view(gk),
               _lib._view(gv), _lib._view(out[0]), _lib._view(out[1]), _lib._view(out[2]), _lib._view(out[3]),
               e.data_ptr(), f.data_ptr(), wp, wn, _lib._stream())
    torch.cuda.synchronize()
    for n, x, y in zip(("gq", "gk", "gv", "gdo"), out, ref):
        if y is not None:
            assert torch.equal(x, y), n


def test_deterministic():
    """Two runs give bitwise identical outputs (no atomics anywhere)."""
    xs = _inputs(1, 1, 320, 64, torch.bfloat16, seed=4)
    print("[case] determinism", flush=True)
    a = _run(xs, True, 0.125, True)
    b = _run(xs, True, 0.125, True)
    for n in ("o", "dq", "dk", "dv", "gq", "gk", "gv", "gdo", "lse", "rowsum", "gq_dq", "gk_dq", "gv_dq"):
        assert torch.equal(a[n], b[n]), n
    assert torch.equal(a["p"], b["p"])


def test_rowsum_from_p_and_dv_from_p():
    """Reference-definition launchers: rowsum = sum P o (dO V^T); dV = P^T dO."""
    xs = _inputs(2, 2, 130, 64, torch.float16, seed=5)
    q, k, v, do = (x.cuda() for x in xs[:4])
    print("[case] rowsum/dv from P", flush=True)
    ref = _ref(xs, False, 0.125)
    _, _, p = _lib.fwd(q, k, v, False, 0.125, True)
    rs = _lib.rowsum_from_p(p, do, v, False)
    _, dv = _lib.bwd_dkdv(None, None, None, do, p, None, None, False, 1.0, want_dk=False)
    torch.cuda.synchronize()
    check("rowsum", rs, ref["rowsum"], torch.float16)
    check("dv", dv, ref["dv"], torch.float16)


def test_strided_inputs():
    """Operands that are transposed views of [B,T,H,D] storage run without copies."""
    g = torch.Generator().manual_seed(6)
    b, h, t, d = 2, 3, 96, 64
    base = [torch.randn(b, t, h, d, generator=g).to(torch.float16) for _ in range(7)]
    xs = [x.transpose(1, 2) for x in base]  # [B,H,T,D] views, stride_t = H*D
    print("[case] strided", flush=True)
    dev = [y.cuda().transpose(1, 2) for y in base]
    assert not dev[0].is_contiguous()
    q, k, v, do, gq, gk, gv = dev
    o, lse, p = _lib.fwd(q, k, v, True, 0.125, True)
    dq, dk, dv, rowsum = _lib.bwd(q, k, v, o, do, lse, p, True, 0.125)
    GQ, GK, GV, GdO = _lib.gg(q, k, v, do, lse, p, rowsum, gq, gk, gv, True, 0.125, True)
    torch.cuda.synchronize()
    ref = _ref([x.contiguous() for x in xs], True, 0.125)
    for n, x in dict(o=o, dq=dq, dk=dk, dv=dv, gq=GQ, gk=GK, gv=GV, gdo=GdO).items():
        check(n, x, ref[n], torch.float16)


@pytest.mark.parametrize("dtype", ["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("save_p", [True, False])
@pytest.mark.parametrize("chunk", [1, 2])
def test_split_chunks(dtype, d, causal, save_p, chunk):
    """Streamed loops split into chunks of 1 or 2 tiles (partials + combine
    kernels) on a ragged 5-block sequence give the oracle's results."""
    dt = DT[dtype]
    t = 300
    xs = _inputs(1, 2, t, d, dt, seed=21)
    scale = 1.0 / math.sqrt(d)
    print(f"[case] split dtype={dtype} d={d} causal={causal} save_p={save_p} chunk={chunk}", flush=True)
    with _lib.split_chunk(chunk):
        out = _run(xs, causal, scale, save_p)
    _compare(out, _ref(xs, causal, scale), dt, causal, t)


@pytest.mark.parametrize("chunk", [5, 7])
@pytest.mark.parametrize("save_p", [True, False])
def test_longest_first_order_many_chunks(chunk, save_p):
    """A split causal launch whose longest-first order has several full-chunk
    indices and last chunks of every length below the chunk (24 blocks, three
    slices, ragged T) gives the oracle's results in fp32 (max-abs 1e-5)."""
    t = 1500
    xs = _inputs(1, 3, t, 64, torch.float32, seed=23)
    print(f"[case] longest-first chunk={chunk} save_p={save_p}", flush=True)
    with _lib.split_chunk(chunk):
        out = _run(xs, True, 0.125, save_p)
    _compare(out, _ref(xs, True, 0.125), torch.float32, True, t)


def test_split_matches_unsplit():
    """Split and unsplit runs agree to fp32 summation-order noise."""
    xs = _inputs(2, 1, 512, 64, torch.float32, seed=22)
    print("[case] split vs unsplit", flush=True)
    a = _run(xs, True, 0.125, True)
    with _lib.split_chunk(3):
        b = _run(xs, True, 0.125, True)
    for n in ("o", "dq", "dk", "dv", "gq", "gk", "gv", "gdo", "lse", "rowsum"):
        assert (a[n] - b[n]).abs().max().item() < 1e-5, n


@pytest.mark.parametrize("b,h", [(2, 4), (1, 16)])
@pytest.mark.parametrize("save_p", [True, False])
@pytest.mark.parametrize("chunk", [0, 2])
def test_slices_divisible_by_eight(b, h, save_p, chunk):
    """B*H a multiple of 8: each slice's workgroups run on one XCD (the
    kernels remap the grid); results must be the same as per-slice math."""
    dt = torch.float16
    t = 200
    xs = _inputs(b, h, t, 64, dt, seed=b * 10 + h)
    print(f"[case] slices b={b} h={h} save_p={save_p} chunk={chunk}", flush=True)
    with _lib.split_chunk(chunk):
        out = _run(xs, True, 0.125, save_p)
    _compare(out, _ref(xs, True, 0.125), dt, True, t)


@pytest.mark.parametrize("save_p", [True, False])
def test_launch_timing_counts_and_leaves_results_unchanged(save_p):
    """Per-kernel timing (ttt_kernel_timing) brackets every main-kernel
    launch of the fused step with events: one launch per family per step
    (the double backward's two per step: _run takes it in both forms),
    positive durations, each shorter than the steps' wall time, and results
    bitwise those of an untimed step."""
    import time
    xs = _inputs(1, 2, 1100, 64, torch.float16, seed=5)
    causal, scale = True, 0.125
    ref = _run(xs, causal, scale, save_p)
    steps = 3
    with _lib.launch_timing() as read:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            out = _run(xs, causal, scale, save_p)
        wall_ms = (time.perf_counter() - t0) * 1e3 / steps
        times = read()
    fams = ("fwd_stats", "fwd_p") if save_p else ("fwd_online",)
    for name in fams + ("bwd_dq", "bwd_dkdv", "gg_row", "gg_col"):
        ms, n = times[name]
        assert n == (2 if name.startswith("gg") else 1) * steps and 0.0 < ms < wall_ms, (name, ms, n, wall_ms)
    assert set(times) == set(fams + ("bwd_dq", "bwd_dkdv", "gg_row", "gg_col"))
    for key in ("o", "lse", "dq", "dk", "dv", "gq", "gk", "gv", "gdo", "gq_dq", "gk_dq", "gv_dq"):
        assert torch.equal(out[key], ref[key]), key
    with _lib.launch_timing() as read:  # a new record each time, nothing timed yet
        assert read() == {}


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("rows", [64, 128])
@pytest.mark.parametrize("chunk", [0, 2, 5])
def test_fwd_block_rows(dtype, d, causal, rows, chunk):
    """The O + LSE forward in 64-row blocks (k_fwd_online) and in 128-row
    blocks (k_fwd_lse, pairs of row blocks), unsplit and split into chunks
    (a causal row-pair launch rounds 5 up to 6 tiles), on a ragged sequence
    of an odd block count (the last pair has one block): O and LSE against
    the float64 oracle, and the first backward and grad-grad from that
    forward."""
    dt = DT[dtype]
    t = 300
    xs = _inputs(1, 3, t, d, dt, seed=60 + d + rows)
    scale = 1.0 / math.sqrt(d)
    print(f"[case] fwd block_rows={rows} dtype={dtype} d={d} causal={causal} chunk={chunk}", flush=True)
    with _lib.block_rows(rows), _lib.split_chunk(chunk):
        out = _run(xs, causal, scale, False)
    _compare(out, _ref(xs, causal, scale), dt, causal, t)


def test_fwd_block_rows_edge_cases():
    """Rows past T in a pair's second block, T = 1, one pair whose second
    block is absent, and a negative and a zero scale (q negated; every visible
    key equally likely) in 128-row blocks."""
    dt = torch.float16
    for t, causal, scale in ((65, True, 0.125), (1, False, 0.125), (64, True, 0.125), (200, True, -0.125),
                             (130, False, 0.0), (130, True, 0.0)):
        xs = _inputs(2, 1, t, 64, dt, seed=t)
        print(f"[case] fwd block_rows=128 t={t} causal={causal} scale={scale}", flush=True)
        with _lib.block_rows(128):
            q, k, v = (x.cuda() for x in xs[:3])
            o, lse, _ = _lib.fwd(q, k, v, causal, scale, False)
            torch.cuda.synchronize()
        ref = cf.forward(*(x.double().numpy() for x in xs[:3]), causal, scale)
        check(f"t={t} o", o, ref["o"], dt)
        check(f"t={t} lse", lse, ref["lse"], torch.float32, abs_tol=2e-3)
