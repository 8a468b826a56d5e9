"""The autotuned kernels on the GPU: with tuning on, the first step of a shape
times the candidate splits of each kernel family, and for the O + LSE
forward also both block heights (64-row blocks, or 128-row pairs of blocks,
which run at one or two waves per SIMD depending on D), on its own operands;
the step's results match the float64 math path (fp16/bf16: relative
Frobenius <= 2e-2) and every later step of the shape reuses the choices,
bitwise repeatable.

b1 h2 T1024 d64 fp16 causal: 32 row blocks against hundreds of workgroup
slots, so every family's walk is split and has several candidate splits.
A C5-shaped slice, b1 h4 T2048 d128 bf16 causal with q, k, v ~ N(0, 0.5^2),
runs the same at C5's head dim and type."""
import pytest
import torch

from oracle import math_path
from testtimeideas_amd import autotune
from tests._util import check
from ttt_kernels.triton_attention import triton_attention

pytestmark = pytest.mark.gpu

FAMILIES = {"save_p_triton_full": 5, "recompute": 5}  # fwd, dq, dkdv, gg_row, gg_col


def _step(xs, mode, scale=0.125):
    q, k, v, do, rq, rk, rv = (x.cuda() for x in xs)
    q, k, v = (t.requires_grad_(True) for t in (q, k, v))
    o = triton_attention(q, k, v, causal=True, scale=scale, bwd_mode=mode)
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


@pytest.mark.parametrize("mode", ["recompute", "save_p_triton_full"])
def test_autotuned_step_c5_slice(mode):
    prev = autotune.enabled()
    autotune.enable(True)
    autotune.clear()
    try:
        g = torch.Generator().manual_seed(5)
        xs = [torch.randn(1, 4, 2048, 128, generator=g) for _ in range(7)]
        xs = [(x * 0.5 if i < 3 else x).to(torch.bfloat16) for i, x in enumerate(xs)]
        scale = 128 ** -0.5
        print(f"[case] autotune C5 slice mode={mode}", flush=True)
        first = _step(xs, mode, scale)
        chosen = autotune.choices()
        if mode == "recompute":
            fwd = [c for key, c in chosen.items() if key[0] == "fwd_rows"]
            assert len(fwd) == 1, chosen
            print(f"  forward (block rows, split): {fwd[0]}", flush=True)
        ref = math_path.gradgrad_step(*(x.double() for x in xs), True, scale)
        for n in ("o", "dq", "dk", "dv", "gq", "gk", "gv"):
            check(n, first[n], ref[n], torch.bfloat16)
        second = _step(xs, mode, scale)
        third = _step(xs, mode, scale)
        assert autotune.choices() == chosen
        for n in second:
            assert torch.equal(second[n], third[n]), n
    finally:
        autotune.enable(prev)
        autotune.clear()
