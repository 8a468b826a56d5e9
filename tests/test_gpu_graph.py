"""HIP-graph capture of the whole grad-grad step: every replay, with eager
steps and synchronisations between replays, must equal the eager result
bitwise (the kernels are deterministic and issue no memsets; the loss uses a
two-stage sum, whose reduction launches no memset either)."""
import pytest
import torch

from ttt_kernels import triton_attention

pytestmark = pytest.mark.gpu


def _two_stage_sum(t):
    return t.reshape(256, -1).sum(1).sum()


@pytest.mark.parametrize("mode", ["save_p_triton_full", "recompute"])
@pytest.mark.parametrize("t_len", [512, 1000])
def test_graph_replay_matches_eager(mode, t_len):
    print(f"graph replay mode={mode} T={t_len}", flush=True)
    g = torch.Generator().manual_seed(3)
    shape = (1, 2, t_len, 64)
    q, k, v, do, rq, rk, rv = (torch.randn(shape, generator=g).half().cuda() for _ in range(7))
    q.requires_grad_(True)
    k.requires_grad_(True)
    v.requires_grad_(True)

    def step():
        o = triton_attention(q, k, v, causal=True, bwd_mode=mode)
        dq, dk, dv = torch.autograd.grad(o, (q, k, v), do, create_graph=True)
        s = _two_stage_sum(dq * rq) + _two_stage_sum(dk * rk) + _two_stage_sum(dv * rv)
        return (o.detach(),) + tuple(torch.autograd.grad(s, (q, k, v)))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    ref = [t.clone() for t in step()]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    for i in range(4):
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("o", "gq", "gk", "gv"), out, ref):
            assert torch.equal(a, b), f"replay {i}: {name} differs from eager"
        step()
        torch.cuda.synchronize()
    del graph
