"""GPU parity of the float32 path (FA_DTYPE_F32): float32 q, k, v in, float32 o, dq, dk, dv out,
computed in float32 throughout on the fp32 matrix instruction -- the reference's autograd
Function accepts float32 tensors (flash_attention_gpt_oss.py:356-357; benchmark_backward_speed.py
dtype "fp32", :35-36).

Oracle: the naive path evaluated in float64 on the same float32 inputs (oracle/naive.py).
Tolerance, elementwise on O, LSE, dQ, dK, dV:  |ours - ref| <= 1e-4 + 1e-4 |ref|  -- two orders of
magnitude tighter than the 16-bit bar (2e-2), so a path that rounded any operand, P or dS to 16
bits would fail it.
"""
import math

import pytest
import torch

from conftest import load_mod, load_pkg
from oracle import naive

pytestmark = pytest.mark.gpu

ATOL = RTOL = 1e-4


def inputs(B, Hq, Hkv, L, D, seed, do_std=1.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, L, D, generator=g)
    k = torch.randn(B, Hkv, L, D, generator=g)
    v = torch.randn(B, Hkv, L, D, generator=g)
    do = torch.randn(B, Hq, L, D, generator=g) * do_std
    return [t.cuda() for t in (q, k, v, do)]


def close(name, got, ref):
    assert got.dtype == torch.float32, (name, got.dtype)
    got, ref = got.double(), ref.double()
    assert torch.isfinite(got).all(), name
    err = (got - ref).abs()
    bad = err > ATOL + RTOL * ref.abs()
    assert not bool(bad.any()), (f"{name}: {int(bad.sum())} elements out of tolerance, max abs err "
                                 f"{float(err.max()):.3g}")
    return float(err.max())


def run(B, Hq, Hkv, L, D, W, S, seed=0, scale=None, sinks=None):
    ops = load_mod("_ops")
    print(f"case fp32 B={B} Hq={Hq} Hkv={Hkv} L={L} D={D} W={W} S={S} scale={scale} sinks={sinks is not None}",
          flush=True)
    q, k, v, do = inputs(B, Hq, Hkv, L, D, seed)
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    o, lse = ops.forward(q, k, v, W, S, sc, sinks=sinks)
    grads = ops.backward(q, k, v, o, lse, do, W, S, sc, sinks=sinks)
    torch.cuda.synchronize()
    if sinks is None:
        ref = naive.attention_fwd_bwd(q, k, v, do, W, S, scale=sc, compute_dtype=torch.float64, row_chunk=2048)
    else:
        ref = naive.attention_fwd_bwd_sinks(q, k, v, sinks, do, W, S, scale=sc, compute_dtype=torch.float64,
                                            row_chunk=2048)
    for name, got, r in zip(("O", "LSE", "dQ", "dK", "dV"), (o, lse) + tuple(grads[:3]), ref):
        close(name, got, r)
    if sinks is not None:
        err = (grads[3].double() - ref[5]).abs()
        assert bool((err <= 1e-4 * (1.0 + ref[5].abs())).all()), float(err.max())
    return o, lse, grads


@pytest.mark.parametrize("B,Hq,Hkv,L,D,W,S", [
    pytest.param(1, 4, 2, 200, 64, 37, 0, id="no-sink-window"),
    pytest.param(1, 4, 1, 300, 64, 300, 0, id="full-causal"),
    pytest.param(1, 2, 1, 600, 64, 50, 100, id="sinks-beyond-window"),
    pytest.param(1, 2, 2, 1, 64, 4, 2, id="L1"),
    pytest.param(1, 8, 2, 33, 32, 5, 2, id="L33-D32"),
    pytest.param(2, 6, 3, 257, 64, 40, 5, id="L257-B2-G2"),
    pytest.param(1, 4, 2, 150, 64, 1, 3, id="W1-sinks"),
    pytest.param(1, 4, 2, 300, 64, 0, 5, id="sinks-only"),
    pytest.param(1, 16, 1, 256, 64, 32, 4, id="G16"),
    pytest.param(1, 4, 4, 300, 16, 64, 4, id="D16-G1"),
    pytest.param(1, 8, 1, 300, 128, 64, 20, id="D128-G8"),
    pytest.param(1, 8, 2, 1100, 64, 8, 40, id="sink-chunks"),
    pytest.param(1, 4, 1, 2000, 128, 100, 70, id="sink-chunks-D128"),
    pytest.param(2, 8, 2, 777, 32, 129, 0, id="W129-B2"),
])
def test_fp32_parity(gpu, B, Hq, Hkv, L, D, W, S):
    run(B, Hq, Hkv, L, D, W, S, seed=L + D + W)


@pytest.mark.parametrize("scale", [0.05, -0.125, 0.0])
def test_fp32_scales(gpu, scale):
    run(1, 4, 2, 200, 64, 48, 4, seed=3, scale=scale)


def test_fp32_learned_sinks(gpu):
    sinks = torch.randn(8, generator=torch.Generator().manual_seed(5)).cuda() * 2
    run(1, 8, 2, 500, 64, 128, 0, seed=7, sinks=sinks)


def test_fp32_gpt_oss_layer_full_size(gpu):
    """The c2 shape (B=1, Hq=64, Hkv=8, L=4096, D=64, W=128, S=4) in float32, every head."""
    run(1, 64, 8, 4096, 64, 128, 4, seed=0)


def test_fp32_autograd_drop_in_and_determinism(gpu):
    """FlashSWDAWithSink with float32 tensors: float32 outputs and gradients equal to the C-ABI
    path's bit for bit, and reruns bitwise identical."""
    fa = load_pkg()
    ops = load_mod("_ops")
    q, k, v, do = inputs(1, 8, 2, 700, 64, seed=9)
    runs = []
    for _ in range(2):
        qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
        o = fa.flash_swda_with_sink(qg, kg, vg, 128, 4)
        o.backward(do)
        runs.append((o.detach(), qg.grad, kg.grad, vg.grad))
    assert all(t.dtype == torch.float32 for t in runs[0])
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    o2, lse2 = ops.forward(q, k, v, 128, 4, 0.125)
    g2 = ops.backward(q, k, v, o2, lse2, do, 128, 4, 0.125)
    assert torch.equal(runs[0][0], o2)
    for a, b in zip(runs[0][1:], g2):
        assert torch.equal(a, b)


def test_fp32_varlen(gpu):
    """Packed float32 batch: every sequence equals the float64 oracle on it alone."""
    ops = load_mod("_ops")
    cu = [0, 300, 301, 1000, 1000, 1777]
    Hq, Hkv, D, W, S = 8, 2, 64, 128, 4
    g = torch.Generator().manual_seed(11)
    q, k, v, do = (torch.randn(cu[-1], h, D, generator=g).cuda() for h in (Hq, Hkv, Hkv, Hq))
    cu_dev, max_len = ops.cu_seqlens_ready(torch.tensor(cu, dtype=torch.int32), cu[-1], q.device)
    o, lse = ops.forward_varlen(q, k, v, cu_dev, max_len, W, S, 0.125)
    dq, dk, dv = ops.backward_varlen(q, k, v, o, lse, do, cu_dev, max_len, W, S, 0.125)
    torch.cuda.synchronize()
    ref = naive.attention_fwd_bwd_varlen(q, k, v, do, torch.tensor(cu), W, S, 0.125, compute_dtype=torch.float64,
                                         row_chunk=1024)
    for name, got, r in zip(("O", "LSE", "dQ", "dK", "dV"), (o, lse, dq, dk, dv), ref):
        close(name, got, r)


def test_fp32_staged_backward_equals_fa_bwd(gpu):
    ops = load_mod("_ops")
    q, k, v, do = inputs(1, 8, 1, 1100, 64, seed=13)
    o, lse = ops.forward(q, k, v, 8, 40, 0.125)
    call = ops.BwdCall(q, k, v, o, lse, do, 8, 40, 0.125)
    call.run("dq")
    call.run("dkdv")
    staged = (call.dq.clone(), call.dk.clone(), call.dv.clone())
    call.run("all")
    torch.cuda.synchronize()
    for a, b in zip(staged, (call.dq, call.dk, call.dv)):
        assert torch.equal(a, b)
