"""Writes tests/golden/c1_b1h1_t64_d64_fp32.npz: the C1 configuration (b1 h1
T64 d64 fp32, non-causal, scale 1/8) with inputs drawn as the benchmark draws
them (CPU generator, seed 0, order q k v dO rq rk rv) and the float64 oracle's
O, dQ, dK, dV, GQ, GK, GV, GdO stored as float32.

The reference's tests hold no golden vectors for this path, so this fixture
is produced by the oracle (oracle.math_path, autograd in float64) and pins the
GPU float32 path and any later change to the oracle.

    python tests/golden/make_c1.py
"""
import os
import sys

import numpy as np
import torch

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), "..", ".."))
sys.path.insert(0, ROOT)

from oracle import math_path  # noqa: E402
from testtimeideas_amd import workloads  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c1_b1h1_t64_d64_fp32.npz")


def build():
    cfg = workloads.CONFIGS["C1"]
    x = workloads.make_inputs(cfg, seed=0)
    names = ("q", "k", "v", "do", "rq", "rk", "rv")
    r = math_path.gradgrad_step(*(x[n].double() for n in names), cfg.causal, cfg.scale, do_requires_grad=True)
    arrays = {f"in_{n}": x[n].numpy() for n in names}
    arrays.update({f"out_{n}": r[n].numpy().astype(np.float32)
                   for n in ("o", "dq", "dk", "dv", "gq", "gk", "gv", "gdo")})
    return arrays


if __name__ == "__main__":
    np.savez_compressed(OUT, **build())
    print("wrote", OUT)
