"""Storage precision of the cached probabilities P (save_p modes): the gate
for storing P in fewer bits.

The double backward reads P in five products (O, dV, dS, gdP, gS), so
P's storage rounding reaches every output.  With P rounded as stored and
everything else exact (float64 closed forms, ``p_store``), the relative
Frobenius error of O, dQ, dK, dV, GQ, GK, GV and GdO against unrounded P is
measured at a C5-like slice (d = 128, q, k, v ~ N(0, 0.5^2) rounded to bf16,
T = 512, causal and not).  P in the input's 16-bit type stays well inside
the 2e-2 tolerance of the 16-bit parity tests; every 8-bit float format
exceeds it, so P is not stored in 8 bits:
  e4m3: P < 2^-9 flushes to zero (rows of T > 512 keys are mostly such);
  e5m2: 2 mantissa bits, about 5e-2;
  e4m3 scaled by the row max: about 2.5e-2, still above the tolerance.
"""
import math

import numpy as np
import pytest
import torch

from oracle import closed_form as cf

TOL = 2e-2  # the 16-bit parity tolerance (tests/_util.py)
T, D = 512, 128
OUTS = ("o", "dq", "dk", "dv", "gq", "gk", "gv", "gdo")


def _store(dt, row_scaled=False):
    def f(p):
        x = torch.from_numpy(p)
        if row_scaled:
            m = x.amax(dim=-1, keepdim=True)
            return ((x / m).to(dt).double() * m).numpy()
        return x.to(dt).double().numpy()
    return f


def _worst(causal, store):
    g = torch.Generator().manual_seed(5)
    xs = [(torch.randn(T, D, generator=g) * (0.5 if i < 3 else 1.0)).to(torch.bfloat16).double().numpy()
          for i in range(7)]
    s = 1.0 / math.sqrt(D)
    ref = cf.double_backward(*xs, causal, s)
    out = cf.double_backward(*xs, causal, s, p_store=store)
    return max(float(np.linalg.norm(out[k] - ref[k]) / np.linalg.norm(ref[k])) for k in OUTS)


@pytest.mark.parametrize("causal", [True, False])
def test_sixteen_bit_p_within_tolerance(causal):
    assert _worst(causal, _store(torch.float16)) < 1e-3
    assert _worst(causal, _store(torch.bfloat16)) < 5e-3


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("fmt", ["e4m3", "e5m2", "e4m3_row_scaled"])
def test_eight_bit_p_exceeds_tolerance(causal, fmt):
    dt = torch.float8_e5m2 if fmt == "e5m2" else torch.float8_e4m3fn
    err = _worst(causal, _store(dt, row_scaled=fmt.endswith("row_scaled")))
    assert err > TOL, f"{fmt}: {err:.2e}"
