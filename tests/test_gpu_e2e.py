"""The TTT model's meta-learning step on the GPU (HIP attention, fp32)
against the same model in float64 on the CPU with the reference's chunked
attention restated in the oracle (oracle.math_path.window_chunks_attention),
and against the reference's own meta step (the fixture written by
tests/golden/make_meta_fixture.py): inner and outer losses, and the
meta-gradient of every parameter, which runs the attention's double backward
through the inner updates.

Tolerances: losses relative 1e-5; meta-gradients relative Frobenius 1e-3 per
parameter, against at least 1e-4 of the largest gradient norm (fp32 kernels
against float64 through a few hundred ops).
"""
import copy

import pytest
import torch

from oracle import math_path
from tests.golden.make_meta_fixture import CFG, STEP
from tests.test_e2e_meta_fixture import load_fixture
from testtimeideas_amd.ttt_e2e import attention as attn_mod
from ttt_e2e import data, meta
from ttt_e2e.model import ModelConfig, TTTModel

pytestmark = pytest.mark.gpu


def _oracle_windowed(q, k, v, window, local=True, scale=None, bwd_mode=None):
    assert local and scale is None
    return math_path.window_chunks_attention(q, k, v, window if window is not None else q.size(-2))


@pytest.mark.parametrize("t,window,chunk", [(256, 64, 128), (192, 128, 64)])
def test_meta_step_matches_float64_reference(t, window, chunk, monkeypatch):
    print(f"[case] meta_step t={t} window={window} chunk={chunk}", flush=True)
    torch.manual_seed(0)
    cfg = ModelConfig(vocab_size=64, max_seq_len=t, window_size=window, d_model=64, n_heads=2, n_layers=3, d_ff=128,
                      suffix_layers=2, dual_mlp=True)
    gpu_model = TTTModel(cfg).cuda()
    cpu_model = copy.deepcopy(gpu_model).cpu().double()
    g = torch.Generator().manual_seed(5)
    bt = data.generate_kv_batch(2, (t * 3) // 4, t // 4, cfg.vocab_size, num_keys=16, device="cpu", pad_to=t,
                                far_frac=0.5, generator=g)
    kw = dict(inner_lr=0.1, inner_steps=2, param_filter="mlp_fast", chunk_size=chunk)

    inner_g, outer_g = meta.meta_step(gpu_model, bt.input_ids.cuda(), bt.targets.cuda(), bt.inner_mask.cuda(),
                                      bt.outer_mask.cuda(), **kw)
    outer_g.backward()
    torch.cuda.synchronize()

    monkeypatch.setattr(attn_mod, "windowed_attention", _oracle_windowed)
    inner_c, outer_c = meta.meta_step(cpu_model, bt.input_ids, bt.targets, bt.inner_mask.double(),
                                      bt.outer_mask.double(), **kw)
    outer_c.backward()

    assert abs(inner_g.item() - inner_c.item()) <= 1e-5 * abs(inner_c.item())
    assert abs(outer_g.item() - outer_c.item()) <= 1e-5 * abs(outer_c.item())
    ref = dict(cpu_model.named_parameters())
    # Some gradients are zero in exact arithmetic (a key bias shifts every
    # score of a query equally, so the softmax ignores it): their reference is
    # float64 rounding noise, so errors are taken relative to at least 1e-4 of
    # the largest gradient norm.
    top = max(float(p.grad.norm()) for p in ref.values())
    worst = 0.0
    for name, p in gpu_model.named_parameters():
        r = ref[name].grad
        assert p.grad is not None and r is not None, name
        err = float((p.grad.double().cpu() - r).norm()) / max(float(r.norm()), 1e-4 * top)
        worst = max(worst, err)
        assert err <= 1e-3, f"{name}: relative error {err:.2e}"
    print(f"worst meta-gradient error {worst:.2e}", flush=True)


def test_meta_step_on_gpu_matches_reference_fixture():
    """The reference's meta step (fixture: its package run in float64 on the
    CPU) against the harness model on the GPU, fp32, HIP attention."""
    print("[case] meta_step reference fixture", flush=True)
    params, grads, batch, inner_ref, outer_ref = load_fixture()
    model = TTTModel(ModelConfig(**CFG))
    model.load_state_dict({n: p.float() for n, p in params.items()}, strict=True)
    model = model.cuda()
    b = {n: (x.float() if x.is_floating_point() else x).cuda() for n, x in batch.items()}
    inner, outer = meta.meta_step(model, b["input_ids"], b["targets"], b["inner_mask"], b["outer_mask"], **STEP)
    outer.backward()
    torch.cuda.synchronize()
    assert abs(inner.item() - inner_ref) <= 1e-5 * abs(inner_ref)
    assert abs(outer.item() - outer_ref) <= 1e-5 * abs(outer_ref)
    top = max(float(g.norm()) for g in grads.values())
    for name, p in model.named_parameters():
        r = grads[name]
        err = float((p.grad.double().cpu() - r).norm()) / max(float(r.norm()), 1e-4 * top)
        assert err <= 1e-3, f"{name}: relative error {err:.2e}"
