"""The harness TTT model and meta step (ttt_e2e/model.py, ttt_e2e/meta.py)
against the reference's own meta step, through the fixture that
tests/golden/make_meta_fixture.py wrote by running the reference package
(cloud_ttt_e2e/ttt_e2e, meta.py:140-177) in float64 on the CPU.

On the CPU, in float64, with the attention swapped for the oracle's
restatement of the reference's chunked attention
(oracle.math_path.window_chunks_attention): the parameters load by name
(strict), and the losses and every parameter's meta-gradient agree to
rounding (losses 1e-12 relative; gradients 1e-9 of the largest gradient's
norm).  tests/test_gpu_e2e.py runs the same fixture through the HIP
attention.
"""
import os

import numpy as np
import torch

from oracle import math_path
from tests.golden.make_meta_fixture import CFG, STEP
from testtimeideas_amd.ttt_e2e import attention as attn_mod
from ttt_e2e import meta
from ttt_e2e.model import ModelConfig, TTTModel

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "meta_step_small.npz")


def load_fixture():
    f = np.load(FIXTURE)
    params = {n[len("param/"):]: torch.from_numpy(f[n]) for n in f.files if n.startswith("param/")}
    grads = {n[len("grad/"):]: torch.from_numpy(f[n]) for n in f.files if n.startswith("grad/")}
    batch = {n: torch.from_numpy(f[n]) for n in ("input_ids", "targets", "inner_mask", "outer_mask")}
    return params, grads, batch, float(f["inner_loss"]), float(f["outer_loss"])


def oracle_windowed(q, k, v, window, local=True, scale=None, bwd_mode=None):
    assert local and scale is None
    return math_path.window_chunks_attention(q, k, v, window if window is not None else q.size(-2))


def test_meta_step_matches_reference_fixture(monkeypatch):
    params, grads, batch, inner_ref, outer_ref = load_fixture()
    model = TTTModel(ModelConfig(**CFG)).double()
    model.load_state_dict(params, strict=True)
    assert [n for n, _ in model.named_parameters()] == list(params)  # same names, same order
    monkeypatch.setattr(attn_mod, "windowed_attention", oracle_windowed)
    inner, outer = meta.meta_step(model, batch["input_ids"], batch["targets"], batch["inner_mask"],
                                  batch["outer_mask"], **STEP)
    outer.backward()
    assert abs(inner.item() - inner_ref) <= 1e-12 * abs(inner_ref)
    assert abs(outer.item() - outer_ref) <= 1e-12 * abs(outer_ref)
    top = max(float(g.norm()) for g in grads.values())
    for name, p in model.named_parameters():
        err = float((p.grad - grads[name]).norm())
        assert err <= 1e-9 * top, f"{name}: {err:.3e} (largest gradient norm {top:.3e})"


def test_fixture_is_a_real_meta_gradient():
    """The fixture's meta-gradient reaches the parameters the inner loop does
    not update (through the adapted ones) and is not zero anywhere it should
    not be: it pins the second-order path, not just the first."""
    params, grads, _, _, _ = load_fixture()
    assert set(grads) == set(params)
    for name in ("prefix_blocks.0.attn.q_proj.weight", "suffix_blocks.0.attn.k_proj.weight", "embed.weight",
                 "suffix_blocks.1.mlp_slow.0.weight", "suffix_blocks.0.mlp_fast.2.weight"):
        assert float(grads[name].abs().max()) > 0, name
