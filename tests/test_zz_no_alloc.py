"""GPU test of fa_bwd_scratch, the backward entry point that allocates nothing (its workspace is
the library's static per-GPU buffer): through the C ABI it returns fa_bwd's dq, dk and dv bit for
bit, on two calls in a row, the second on a smaller problem (the buffer keeps the first call's
contents, which the kernels must not depend on)."""
import ctypes
import math

import pytest
import torch

from conftest import load_mod
from test_gpu_parity import make_inputs

pytestmark = pytest.mark.gpu


def _scratch_backward(ops, lib, call):
    """dq, dk, dv of fa_bwd_scratch with the parameter block of a prepared fa_bwd call (the outputs
    are zeroed first, so every value is written by this call)."""
    for t in (call.dq, call.dk, call.dv):
        t.zero_()
    with ops._DeviceGuard(call.device):
        stream = ctypes.c_void_p(torch.cuda.current_stream(call.device).cuda_stream)
        rc = lib.fa_bwd_scratch(ctypes.byref(call.params), stream)
    assert rc == 0, lib.fa_strerror(rc)
    torch.cuda.synchronize()
    return call.dq.clone(), call.dk.clone(), call.dv.clone()


@pytest.mark.parametrize("first,second", [
    pytest.param((1, 64, 8, 4096, 64, 128, 4, torch.bfloat16), (1, 16, 2, 700, 64, 64, 4, torch.bfloat16),
                 id="c2-then-small"),
    pytest.param((2, 8, 1, 1100, 128, 50, 20, torch.float16), (1, 4, 4, 300, 16, 40, 3, torch.float16),
                 id="sink-chunks-then-D16"),
])
def test_scratch_entry_point_matches_fa_bwd(gpu, first, second):
    ops = load_mod("_ops")
    lib = load_mod("_lib").lib()
    for i, (B, Hq, Hkv, L, D, W, S, dt) in enumerate((first, second)):
        print(f"case fa_bwd_scratch call {i}: B={B} Hq={Hq} Hkv={Hkv} L={L} D={D} W={W} S={S} {dt}", flush=True)
        q, k, v, do = make_inputs(B, Hq, Hkv, L, D, dt, seed=40 + i)
        sc = 1.0 / math.sqrt(D)
        o, lse = ops.forward(q, k, v, W, S, sc)
        call = ops.BwdCall(q, k, v, o, lse, do, W, S, sc)
        call.run("all")  # fa_bwd with a caller workspace
        torch.cuda.synchronize()
        ref = (call.dq.clone(), call.dk.clone(), call.dv.clone())
        got = _scratch_backward(ops, lib, call)
        for name, a, b in zip(("dq", "dk", "dv"), got, ref):
            assert torch.equal(a, b), (name, float((a.float() - b.float()).abs().max()))


def test_scratch_entry_point_under_graph_capture(gpu):
    """fa_bwd_scratch captured in a HIP graph (after one call outside the capture, which looks up
    the buffer's address on the device) and replayed: every replay gives fa_bwd's dq, dk, dv bit for
    bit, with new dO values written into the graph's input before each replay and, between replays,
    eager fa_bwd_scratch calls of another shape that overwrite the shared buffer."""
    ops = load_mod("_ops")
    lib = load_mod("_lib").lib()
    B, Hq, Hkv, L, D, W, S, dt = 1, 16, 2, 1024, 64, 128, 4, torch.bfloat16
    print(f"case fa_bwd_scratch graph: B={B} Hq={Hq} Hkv={Hkv} L={L} D={D} W={W} S={S} {dt}", flush=True)
    q, k, v, do = make_inputs(B, Hq, Hkv, L, D, dt, seed=51)
    sc = 1.0 / math.sqrt(D)
    o, lse = ops.forward(q, k, v, W, S, sc)
    call = ops.BwdCall(q, k, v, o, lse, do, W, S, sc)  # outputs written by the graph
    ref_call = ops.BwdCall(q, k, v, o, lse, do, W, S, sc)  # fa_bwd with its own workspace and outputs
    other_in = make_inputs(1, 4, 4, 300, 16, torch.float16, seed=52)
    other_o, other_lse = ops.forward(*other_in[:3], 40, 3, 0.25)
    other = ops.BwdCall(*other_in[:3], other_o, other_lse, other_in[3], 40, 3, 0.25)
    _scratch_backward(ops, lib, call)  # first call on the device: outside any capture

    def launch(c):
        with ops._DeviceGuard(c.device):
            stream = ctypes.c_void_p(torch.cuda.current_stream(c.device).cuda_stream)
            return lib.fa_bwd_scratch(ctypes.byref(c.params), stream)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        assert launch(call) == 0
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    rcs = []
    with torch.cuda.graph(graph):
        rcs.append(launch(call))
    assert rcs == [0], lib.fa_strerror(rcs[0])
    gen = torch.Generator().manual_seed(53)
    for rep in range(4):
        do.copy_(torch.randn(do.shape, generator=gen).to(dt).cuda())
        for t in (call.dq, call.dk, call.dv):
            t.zero_()
        graph.replay()
        assert launch(other) == 0  # eager use of the shared buffer, another shape
        ref_call.run("all")
        torch.cuda.synchronize()
        for name, a, b in zip(("dq", "dk", "dv"), (call.dq, call.dk, call.dv), (ref_call.dq, ref_call.dk, ref_call.dv)):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from fa_bwd"
