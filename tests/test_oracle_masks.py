"""Pins the mask part of the CPU oracle (CPU only): the reference TTT model's
window masks, its chunked window loop, and the additive bias in the closed
forms.  The checks do not restate the functions they pin: literal masks
written out from the reference's definitions, two formulations of the
chunked window (a loop of rectangular problems, one square mask), softmax
shift invariance, torch float64 autograd of the reference's masked math, and
pure-Python loops."""
import numpy as np
import pytest
import torch

from oracle import brute, closed_form as cf, masks, math_path

NEG = -np.inf


def test_window_masks_by_hand():
    # make_window_mask(5, 2): query i sees keys i-1 and i (utils.py:40-54)
    want = np.array([[0, NEG, NEG, NEG, NEG],
                     [0, 0, NEG, NEG, NEG],
                     [NEG, 0, 0, NEG, NEG],
                     [NEG, NEG, 0, 0, NEG],
                     [NEG, NEG, NEG, 0, 0]])
    assert np.array_equal(masks.window_bias(5, 2), want)
    # no window, or one of at least T: causal
    causal = np.where(np.triu(np.ones((5, 5), bool), 1), NEG, 0.0)
    assert np.array_equal(masks.window_bias(5, None), causal)
    assert np.array_equal(masks.window_bias(5, 5), causal)
    assert np.array_equal(masks.window_bias(5, 9), causal)
    # W = 1: the diagonal only
    assert np.array_equal(masks.window_bias(4, 1), np.where(np.eye(4, dtype=bool), 0.0, NEG))
    # _local_window_mask(4, 6, 2, 6, 4): queries 4, 5 against keys 2..5
    assert np.array_equal(masks.local_chunk_bias(4, 6, 2, 6, 4), np.array([[0, 0, 0, NEG], [0, 0, 0, 0]]))


def test_local_layout_by_hand():
    # T = 7, W = 3: chunks [0,3) [3,6) [6,7); the last sees keys 4..6
    assert masks.chunks(7, 3) == [(0, 3, 0), (3, 6, 3), (6, 7, 4)]
    vis = masks.local_bias(7, 3) == 0
    want = [[0], [0, 1], [0, 1, 2], [3], [3, 4], [3, 4, 5], [4, 5, 6]]
    assert [list(np.nonzero(r)[0]) for r in vis] == want
    # T a multiple of W: block-diagonal causal
    vis = masks.local_bias(6, 3) == 0
    assert [list(np.nonzero(r)[0]) for r in vis] == [[0], [0, 1], [0, 1, 2], [3], [3, 4], [3, 4, 5]]
    # T <= W: causal, as the reference's unchunked branch (attention.py:100-105)
    assert np.array_equal(masks.local_bias(5, 8), masks.window_bias(5, None))


@pytest.mark.parametrize("t,w", [(300, 128), (256, 64), (130, 64), (65, 64), (20, 7)])
def test_chunked_loop_equals_one_square_mask(t, w):
    rng = np.random.default_rng(t + w)
    q, k, v, do, gq, gk, gv = (rng.standard_normal((2, t, 8)) for _ in range(7))
    loop = masks.chunked_loop(q, k, v, w, 0.3, do, gq, gk, gv)
    one = cf.double_backward(q, k, v, do, gq, gk, gv, False, 0.3, masks.local_bias(t, w))
    for n in ("o", "dq", "dk", "dv", "gq", "gk", "gv", "gdo"):
        assert np.allclose(loop[n], one[n], atol=1e-12), n


def test_bias_enters_before_the_softmax():
    rng = np.random.default_rng(5)
    q, k, v, do, gq, gk, gv = (rng.standard_normal((3, 9, 4)) for _ in range(7))
    bias = rng.standard_normal((3, 9, 9))
    # a per-row constant added to the bias changes nothing (softmax shift)
    shifted = bias + rng.standard_normal((3, 9, 1)) * 5
    a = cf.double_backward(q, k, v, do, gq, gk, gv, False, 0.5, bias)
    b = cf.double_backward(q, k, v, do, gq, gk, gv, False, 0.5, shifted)
    for n in ("o", "p", "dq", "dk", "dv", "gq", "gk", "gv", "gdo"):
        assert np.allclose(a[n], b[n], atol=1e-12), n
    # but a per-column one does (it reweights keys)
    c = cf.forward(q, k, v, False, 0.5, bias + np.arange(9.0))
    assert not np.allclose(c["o"], a["o"], atol=1e-3)
    # a -inf upper triangle is the causal flag
    tri = np.where(np.triu(np.ones((9, 9), bool), 1), NEG, 0.0)
    x = cf.double_backward(q, k, v, do, gq, gk, gv, True, 0.5)
    y = cf.double_backward(q, k, v, do, gq, gk, gv, False, 0.5, tri)
    for n in ("o", "dq", "dk", "dv", "gq", "gk", "gv", "gdo"):
        assert np.allclose(x[n], y[n], atol=1e-13), n


def test_bias_forward_matches_loops():
    rng = np.random.default_rng(6)
    q, k, v = (rng.standard_normal((5, 3)) for _ in range(3))
    bias = rng.standard_normal((5, 5))
    bias[1, 3] = NEG
    o, p = brute.forward(q.tolist(), k.tolist(), v.tolist(), False, 0.7, bias.tolist())
    f = cf.forward(q, k, v, False, 0.7, bias)
    assert np.allclose(f["o"], o, atol=1e-13) and np.allclose(f["p"], p, atol=1e-13)
    assert f["p"][1, 3] == 0.0
    # rectangular (fewer queries than keys)
    o, p = brute.forward(q[:3].tolist(), k.tolist(), v.tolist(), False, 0.7, bias[:3].tolist())
    assert np.allclose(cf.forward(q[:3], k, v, False, 0.7, bias[:3])["o"], o, atol=1e-13)


@pytest.mark.parametrize("lq,lk", [(7, 7), (4, 7), (7, 4)])
def test_masked_double_backward_vs_autograd(lq, lk):
    """The closed forms with a bias against torch float64 autograd of the
    reference's masked math (attention.py:9-18), rectangular included."""
    g = torch.Generator().manual_seed(lq * 10 + lk)
    q, do, rq = (torch.randn((2, lq, 4), generator=g, dtype=torch.float64) for _ in range(3))
    k, v, rk, rv = (torch.randn((2, lk, 4), generator=g, dtype=torch.float64) for _ in range(4))
    bias = torch.randn((lq, lk), generator=g, dtype=torch.float64)
    bias[0, 1:] = float("-inf")
    ref = math_path.gradgrad_step(q, k, v, do, rq, rk, rv, False, 0.5, do_requires_grad=True, attn_mask=bias)
    got = cf.double_backward(q.numpy(), k.numpy(), v.numpy(), do.numpy(), rq.numpy(), rk.numpy(), rv.numpy(),
                             False, 0.5, bias.numpy())
    for n in ("o", "dq", "dk", "dv", "gq", "gk", "gv", "gdo"):
        assert np.allclose(got[n], ref[n].numpy(), atol=1e-12), n


def test_planted_mask_mistakes_fail():
    """A window off by one, or a chunk layout that ignores the last partial
    chunk's overlap, is caught by the checks above."""
    off_by_one = masks.local_chunk_bias(0, 5, 0, 5, 3)  # the right one for W = 3
    assert not np.array_equal(off_by_one, masks.window_bias(5, 2))
    rng = np.random.default_rng(9)
    q, k, v = (rng.standard_normal((1, 7, 4)) for _ in range(3))
    i = np.arange(7)[:, None]
    j = np.arange(7)[None, :]
    no_overlap = np.where((j > i) | (j < (i // 3) * 3), NEG, 0.0)  # last chunk sees only itself
    loop = masks.chunked_loop(q, k, v, 3, 0.5)
    assert not np.allclose(loop["o"], cf.forward(q, k, v, False, 0.5, no_overlap)["o"], atol=1e-6)


@pytest.mark.parametrize("t,w", [(300, 128), (100, 128), (129, 64)])
def test_torch_window_loop_equals_numpy_loop(t, w):
    """math_path.window_gradgrad_step (torch autograd through the reference's
    chunk loop, the CPU baseline's workload) equals the closed forms per chunk."""
    g = torch.Generator().manual_seed(t)
    q, k, v, do, rq, rk, rv = (torch.randn((2, t, 8), generator=g, dtype=torch.float64) for _ in range(7))
    a = math_path.window_gradgrad_step(q, k, v, do, rq, rk, rv, w)
    b = masks.chunked_loop(q.numpy(), k.numpy(), v.numpy(), w, 1.0 / np.sqrt(8), do.numpy(), rq.numpy(),
                           rk.numpy(), rv.numpy())
    for n in ("o", "dq", "dk", "dv", "gq", "gk", "gv"):
        assert np.allclose(a[n].numpy(), b[n], atol=1e-12), n
