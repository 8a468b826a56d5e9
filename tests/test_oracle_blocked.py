"""The row-block closed forms (oracle/blocked.py) against the dense float64
closed forms (oracle/closed_form.py, pinned in tests/test_oracle.py by loops,
finite differences and autograd), on the CPU."""
import numpy as np
import pytest
import torch

from oracle import blocked, closed_form, masks

NAMES = ("o", "lse", "rowsum", "dq", "dk", "dv", "e", "f", "gq", "gk", "gv", "gdo")


def _inputs(t, d, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(t, d, generator=g, dtype=torch.float64) for _ in range(7)]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("t,block", [(300, 64), (300, 100), (300, 300), (130, 512), (1, 16)])
def test_blocked_matches_dense(t, block, causal):
    xs = _inputs(t, 64, seed=t + block)
    ref = closed_form.double_backward(*(x.numpy() for x in xs), causal, 0.125)
    rows = {}
    got = blocked.double_backward_blocked(*xs, causal, 0.125, block=block,
                                          on_p=lambda r0, r1, p: rows.__setitem__(r0, (r1, p.clone())))
    for n in NAMES:
        np.testing.assert_allclose(got[n].numpy(), ref[n], rtol=1e-10, atol=1e-12, err_msg=n)
    # P, rebuilt from the row blocks (keys past c1 are zero)
    p = np.zeros((t, t))
    for r0, (r1, pb) in rows.items():
        p[r0:r1, :pb.shape[1]] = pb.numpy()
    assert sorted(rows) == list(range(0, t, block))
    np.testing.assert_allclose(p, ref["p"], rtol=1e-12, atol=1e-15)


def test_first_backward_only():
    xs = _inputs(200, 64, seed=3)
    ref = closed_form.backward(*(x.numpy() for x in xs[:4]), True, 0.2)
    got = blocked.double_backward_blocked(*xs[:4], None, None, None, True, 0.2, block=64, gradgrad=False)
    for n in ("o", "lse", "rowsum", "dq", "dk", "dv"):
        np.testing.assert_allclose(got[n].numpy(), ref[n], rtol=1e-10, atol=1e-12, err_msg=n)
    assert "gq" not in got


def test_float32_agrees_with_float64():
    """The float32 form (used on the GPU as a second check over many slices)
    stays within 1e-5 relative Frobenius of float64 at T = 512."""
    xs = _inputs(512, 128, seed=9)
    a = blocked.double_backward_blocked(*xs, True, 128 ** -0.5, block=256)
    b = blocked.double_backward_blocked(*(x.float() for x in xs), True, 128 ** -0.5, block=256)
    for n in NAMES:
        r = a[n].numpy()
        err = np.linalg.norm(b[n].double().numpy() - r) / np.linalg.norm(r)
        assert err < 1e-5, (n, err)


@pytest.mark.parametrize("local", [True, False])
@pytest.mark.parametrize("t,window,block", [(300, 64, 64), (300, 100, 64), (300, 37, 100), (257, 128, 300),
                                            (300, 300, 64)])
def test_blocked_window_matches_dense_bias(t, window, block, local):
    """The key window of the row-block forms against the dense closed forms
    with the window as an additive -inf bias (oracle.masks, pinned against
    literal masks and the reference's chunk loop in tests/test_oracle_masks.py);
    P is rebuilt from the blocks, zeros before each block's first key."""
    xs = _inputs(t, 64, seed=t + window + block)
    bias = masks.local_bias(t, window) if local else masks.window_bias(t, window)
    ref = closed_form.double_backward(*(x.numpy() for x in xs), True, 0.125, bias=bias)
    rows = {}
    got = blocked.double_backward_blocked(*xs, True, 0.125, block=block, window=window, local=local,
                                          on_p=lambda r0, r1, p: rows.__setitem__(r0, (r1, p.clone())))
    for n in NAMES:
        np.testing.assert_allclose(got[n].numpy(), ref[n], rtol=1e-10, atol=1e-12, err_msg=n)
    p = np.zeros((t, t))
    for r0, (r1, pb) in rows.items():
        p[r0:r1, :pb.shape[1]] = pb.numpy()
    np.testing.assert_allclose(p, ref["p"], rtol=1e-12, atol=1e-15)


def test_blocked_window_planted_mistake_fails():
    """A window one key too wide is caught by the dense reference."""
    t, w = 200, 64
    xs = _inputs(t, 64, seed=5)
    ref = closed_form.double_backward(*(x.numpy() for x in xs), True, 0.125, bias=masks.window_bias(t, w))
    wrong = blocked.double_backward_blocked(*xs, True, 0.125, block=64, window=w + 1, local=False)
    assert not np.allclose(wrong["o"].numpy(), ref["o"], rtol=1e-6, atol=1e-8)
