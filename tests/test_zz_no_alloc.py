"""ttt_attn_gg_noalloc (the double backward with its scratch in the library's
static device array) against ttt_attn_gg (caller workspace and E/F
buffers), called through the C ABI, on calls in a row whose sizes shrink.

Where the library's own split fits in the scratch the two run the same
kernels on the same split and must agree bitwise; where it does not (the
no-allocation entry then takes fewer chunks per block), they must agree to
the parity bar: fp16/bf16 relative Frobenius <= 2e-2, fp32 max-abs <= 1e-5
(tests/_util.py), here also against the float64 oracle.
"""
import math

import pytest
import torch

from oracle import blocked
from tests._util import check
from testtimeideas_amd import _lib

pytestmark = pytest.mark.gpu


def _inputs(b, h, t, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(b, h, t, d, generator=g).to(dtype).cuda() for _ in range(7)]


def _both(xs, causal, scale, save_p, want_gdo):
    """Without GdO both take the first backward's dQ (the row pass's dQ form)."""
    q, k, v, do, rq, rk, rv = xs
    o, lse, p = _lib.fwd(q, k, v, causal, scale, save_p)
    dq, _, _, rowsum = _lib.bwd(q, k, v, o, do, lse, p, causal, scale)
    dq = None if want_gdo else dq
    ref = _lib.gg(q, k, v, do, lse, p, rowsum, rq, rk, rv, causal, scale, want_gdo, dq=dq)
    got = _lib.gg_noalloc(q, k, v, do, lse, p, rowsum, rq, rk, rv, causal, scale, want_gdo, dq=dq)
    torch.cuda.synchronize()
    return ref, got


# (b, h, t, d, dtype, causal, save_p, want_gdo): the second call of each pair is smaller.
CALLS = [
    (1, 2, 1024, 64, torch.float16, True, True, True),
    (1, 1, 300, 64, torch.float16, True, True, True),
    (2, 1, 700, 128, torch.bfloat16, False, False, False),
    (1, 1, 100, 128, torch.float32, True, False, True),
]


def test_noalloc_matches_gg_bitwise_in_a_row():
    for i, (b, h, t, d, dt, causal, save_p, gdo) in enumerate(CALLS):
        print(f"[case] noalloc call {i}: b{b} h{h} t{t} d{d} {dt} causal={causal} save_p={save_p} gdo={gdo}",
              flush=True)
        xs = _inputs(b, h, t, d, dt, seed=40 + i)
        ref, got = _both(xs, causal, 1.0 / math.sqrt(d), save_p, gdo)
        for name, a, r in zip(("gq", "gk", "gv", "gdo"), got, ref):
            if r is None:
                assert a is None
                continue
            assert torch.equal(a, r), f"call {i}: {name} differs from ttt_attn_gg"


def test_noalloc_with_a_capped_split():
    """T = 16384 with GdO: the library's split needs more partials than the
    scratch holds, so the no-allocation entry takes fewer chunks; then a
    smaller call reuses the scratch."""
    for t in (16384, 2048):
        print(f"[case] noalloc capped t={t}", flush=True)
        xs = _inputs(1, 1, t, 64, torch.float16, seed=t)
        ref, got = _both(xs, True, 0.125, True, True)
        for name, a, r in zip(("gq", "gk", "gv", "gdo"), got, ref):
            check(f"t={t} {name} vs ttt_attn_gg", a, r, torch.float16)
        o = blocked.double_backward_blocked(*(x[0, 0].double().cpu() for x in xs), True, 0.125, block=1024)
        for name, a in zip(("gq", "gk", "gv", "gdo"), got):
            check(f"t={t} {name} vs oracle", a[0, 0], o[name], torch.float16)


def test_noalloc_captured_in_a_graph():
    """One eager call first (the device's scratch lookup), then the entry
    captured into a HIP graph and replayed three times, each replay followed
    by an eager call of another size that overwrites the scratch: every
    replay equals the eager result bitwise."""
    print("[case] noalloc graph capture", flush=True)
    xs = _inputs(1, 2, 1024, 64, torch.float16, seed=77)
    q, k, v, do, rq, rk, rv = xs
    o, lse, p = _lib.fwd(q, k, v, True, 0.125, True)
    _, _, _, rowsum = _lib.bwd(q, k, v, o, do, lse, p, True, 0.125)
    ref = _lib.gg_noalloc(q, k, v, do, lse, p, rowsum, rq, rk, rv, True, 0.125, True)
    ref = [r.clone() for r in ref]
    other = _inputs(1, 1, 300, 64, torch.float16, seed=78)
    oq, ok, ov, odo, orq, ork, orv = other
    oo, olse, op = _lib.fwd(oq, ok, ov, True, 0.125, True)
    _, _, _, orow = _lib.bwd(oq, ok, ov, oo, odo, olse, op, True, 0.125)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = _lib.gg_noalloc(q, k, v, do, lse, p, rowsum, rq, rk, rv, True, 0.125, True)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for name, a, r in zip(("gq", "gk", "gv", "gdo"), out, ref):
            assert torch.equal(a, r), f"replay {i}: {name} differs from the eager call"
        _lib.gg_noalloc(oq, ok, ov, odo, olse, op, orow, orq, ork, orv, True, 0.125, True)
        torch.cuda.synchronize()
    del graph


def test_noalloc_rejects_too_many_rows():
    """E and F must fit in their part of the scratch: B*H*T <= 2^21."""
    q = torch.empty(64, 1, 32769, 64, dtype=torch.float16, device="cuda")
    st = torch.empty(64, 1, 32769, dtype=torch.float32, device="cuda")
    with pytest.raises(RuntimeError, match="B\\*H\\*T"):
        _lib.gg_noalloc(q, q, q, q, st, None, st, q, q, q, True, 0.125, False)
