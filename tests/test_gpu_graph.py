"""A forward + backward step captured in a HIP graph (torch.cuda.CUDAGraph) and replayed.

A finetuning loop whose steps are launch-bound (small heads such as the README shape, where the
three kernels take about 35 us and the autograd step about twice that on the host) can capture the
step once and replay it.  The path allocates its outputs and workspace through PyTorch's caching
allocator and never synchronizes the host or calls hipMemsetAsync, so it can be captured.

Each replay is checked bitwise against an eager call on the same values (the kernels are
deterministic), with the graph's static inputs overwritten between replays and eager work of other
shapes in between, as a captured graph that read stale or wrong memory on a later replay would fail.
"""
import pytest
import torch

from conftest import load_pkg
from test_gpu_parity import BF, FP

pytestmark = pytest.mark.gpu

# (B, Hq, Hkv, L, D, W, S, dtype)
GRAPH_CASES = [
    pytest.param(1, 8, 1, 1024, 64, 128, 4, BF, id="sliding-g8"),
    pytest.param(1, 4, 4, 512, 16, 256, 4, FP, id="readme-d16"),
    pytest.param(2, 4, 2, 300, 128, 512, 16, FP, id="d128-sinks16"),
]


def _step(fa, q, k, v, do, W, S):
    o = fa.flash_swda_with_sink(q, k, v, W, S)
    o.backward(do)
    return o


def _eager(fa, q, k, v, do, W, S):
    qe, ke, ve = (t.detach().clone().requires_grad_() for t in (q, k, v))
    o = _step(fa, qe, ke, ve, do, W, S)
    return o.detach(), qe.grad, ke.grad, ve.grad


@pytest.mark.parametrize("B,Hq,Hkv,L,D,W,S,dtype", GRAPH_CASES)
def test_graph_replay_matches_eager(gpu, B, Hq, Hkv, L, D, W, S, dtype):
    print(f"case graph B={B} Hq={Hq} Hkv={Hkv} L={L} D={D} W={W} S={S} {dtype}", flush=True)
    fa = load_pkg()
    dt = dtype
    dev = torch.device("cuda", 0)
    gen = torch.Generator().manual_seed(11)

    def draw(*shape):
        return torch.randn(*shape, generator=gen).to(dt).to(dev)

    q = draw(B, Hq, L, D).requires_grad_()
    k = draw(B, Hkv, L, D).requires_grad_()
    v = draw(B, Hkv, L, D).requires_grad_()
    do = draw(B, Hq, L, D)

    # warm-up on a side stream (library loading, allocator pools), as graph capture requires
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            q.grad = k.grad = v.grad = None
            _step(fa, q, k, v, do, W, S)
    torch.cuda.current_stream().wait_stream(side)

    q.grad = k.grad = v.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        o_static = _step(fa, q, k, v, do, W, S)
    dq_static, dk_static, dv_static = q.grad, k.grad, v.grad

    other = [draw(1, 2, 200, 64) for _ in range(4)]
    for rep in range(4):
        with torch.no_grad():  # new values in the graph's static inputs
            for t in (q, k, v, do):
                t.copy_(draw(*t.shape))
        graph.replay()
        # eager work of another shape between the replays
        oe = _step(fa, *(t.clone().requires_grad_() for t in other[:3]), other[3], 64, 1)
        torch.cuda.synchronize()
        ref = _eager(fa, q, k, v, do, W, S)
        torch.cuda.synchronize()
        for name, got, want in zip(("O", "dQ", "dK", "dV"), (o_static, dq_static, dk_static, dv_static), ref):
            assert torch.equal(got.detach(), want), f"replay {rep}: {name} differs from the eager call"
        assert torch.isfinite(oe).all()
