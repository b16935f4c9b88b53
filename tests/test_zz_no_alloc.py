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
