"""The autotuned splits on the GPU: with tuning on, the first step of a shape
times the candidate splits of each kernel family on its own operands; the
step's results match the float64 math path (fp16: relative Frobenius <= 2e-2)
and every later step of the shape reuses the choices, bitwise repeatable.

b1 h2 T1024 d64 causal: 32 row blocks against hundreds of workgroup slots,
so every family's walk is split and has several candidate splits."""
import pytest
import torch

from oracle import math_path
from testtimeideas_amd import autotune
from tests._util import check
from ttt_kernels.triton_attention import triton_attention

pytestmark = pytest.mark.gpu

FAMILIES = {"save_p_triton_full": 5, "recompute": 5}  # fwd, dq, dkdv, gg_row, gg_col


def _step(xs, mode):
    q, k, v, do, rq, rk, rv = (x.cuda() for x in xs)
    q, k, v = (t.requires_grad_(True) for t in (q, k, v))
    o = triton_attention(q, k, v, causal=True, scale=0.125, bwd_mode=mode)
    dq, dk, dv = torch.autograd.grad(o, (q, k, v), do, create_graph=True)
    g = torch.autograd.grad((dq, dk, dv), (q, k, v), (rq, rk, rv))
    torch.cuda.synchronize()
    return dict(o=o, dq=dq, dk=dk, dv=dv, gq=g[0], gk=g[1], gv=g[2])


@pytest.mark.parametrize("mode", ["save_p_triton_full", "recompute"])
def test_autotuned_step(mode):
    prev = autotune.enabled()
    autotune.enable(True)
    autotune.clear()
    try:
        g = torch.Generator().manual_seed(3)
        xs = [torch.randn(1, 2, 1024, 64, generator=g).to(torch.float16) for _ in range(7)]
        print(f"[case] autotune mode={mode}", flush=True)
        first = _step(xs, mode)
        chosen = autotune.choices()
        assert len(chosen) == FAMILIES[mode], chosen
        ref = math_path.gradgrad_step(*(x.double() for x in xs), True, 0.125)
        for n in ("o", "dq", "dk", "dv", "gq", "gk", "gv"):
            check(n, first[n], ref[n], torch.float16)
        second = _step(xs, mode)
        third = _step(xs, mode)
        assert autotune.choices() == chosen
        for n in second:
            assert torch.equal(second[n], third[n]), n
    finally:
        autotune.enable(prev)
        autotune.clear()
