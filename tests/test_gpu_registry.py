"""GPU parity of the benchmark's calling forms and of the reference's own default cases.

* The registry forms ``func(q, k, v, window_size, sink_size) -> o`` (triton_attention and
  triton_attention_split, benchmark_backward_speed.py:615-643): swa_sink_attention (backward in
  one call, fa_bwd) and swa_sink_attention_split (backward as two C-ABI calls, fa_bwd_dq then
  fa_bwd_dkdv, the path bench.py times per kernel), through autograd, against the float32 oracle.
* The staged entry points fa_bwd_dq -> fa_bwd_dkdv equal fa_bwd bit for bit.
* The reference's default cases (parse_cases, benchmark_backward_speed.py:829-835): B = 1,
  Hq = 16, Hkv in {16, 8, 1}, L = 4096, D = 16, W = 256, S = 4, in fp16 and bf16, at the
  north-star bar |ours - ref| <= 2e-2 + 2e-2 |ref| on O, LSE, dQ, dK, dV against the float32 oracle
  on the same inputs, and at the reference's own check (correctness_check, :682-717: allclose,
  atol = rtol = 5e-2, inputs from torch.manual_seed(0), dO = randn_like(o)) against the same
  oracle.
"""
import math

import pytest
import torch

from conftest import load_mod, load_pkg
from oracle import naive
from test_gpu_parity import assert_close, make_inputs, run_case

pytestmark = pytest.mark.gpu

BF, FP = torch.bfloat16, torch.float16


@pytest.mark.parametrize("form", ["swa_sink_attention", "swa_sink_attention_split"])
@pytest.mark.parametrize("B,Hq,Hkv,L,D,W,S,dtype", [
    pytest.param(1, 16, 2, 1000, 64, 128, 4, BF, id="gpt-oss-like"),
    pytest.param(2, 8, 8, 333, 16, 40, 3, FP, id="D16-G1-B2"),
    pytest.param(1, 8, 1, 700, 128, 64, 20, FP, id="D128-G8-sink-chunks"),
    pytest.param(1, 4, 2, 300, 32, 300, 0, BF, id="D32-full-causal"),
])
def test_registry_forms(gpu, form, B, Hq, Hkv, L, D, W, S, dtype):
    fa = load_pkg()
    print(f"case {form} B={B} Hq={Hq} Hkv={Hkv} L={L} D={D} W={W} S={S} {dtype}", flush=True)
    q, k, v, do = make_inputs(B, Hq, Hkv, L, D, dtype, seed=L + Hq)
    qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
    o = getattr(fa, form)(qg, kg, vg, W, S)
    o.backward(do)
    torch.cuda.synchronize()
    ro, _, rdq, rdk, rdv = naive.attention_fwd_bwd(q, k, v, do, W, S, scale=1 / math.sqrt(D), row_chunk=2048)
    assert_close("O", o.detach(), ro)
    assert_close("dQ", qg.grad, rdq)
    assert_close("dK", kg.grad, rdk)
    assert_close("dV", vg.grad, rdv)


def test_split_form_equals_single_call_bitwise(gpu):
    fa = load_pkg()
    q, k, v, do = make_inputs(1, 16, 2, 1500, 64, BF, seed=8)
    grads = []
    for fn in (fa.swa_sink_attention, fa.swa_sink_attention_split):
        qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
        o = fn(qg, kg, vg, 128, 4)
        o.backward(do)
        grads.append((o.detach(), qg.grad, kg.grad, vg.grad))
    for a, b in zip(*grads):
        assert torch.equal(a, b)


@pytest.mark.parametrize("B,Hq,Hkv,L,D,W,S,dtype", [
    pytest.param(1, 64, 8, 4096, 64, 128, 4, BF, id="c2"),
    pytest.param(1, 8, 1, 1100, 64, 8, 40, FP, id="sink-chunks"),
    pytest.param(1, 4, 4, 700, 16, 40, 3, FP, id="dq-sinks-D16"),
    pytest.param(2, 8, 2, 600, 128, 50, 7, BF, id="D128-dq-sinks"),
])
def test_staged_entry_points_equal_fa_bwd(gpu, B, Hq, Hkv, L, D, W, S, dtype):
    """fa_bwd_dq then fa_bwd_dkdv, as bench.py launches them to time each kernel, give fa_bwd's
    dq, dk, dv bit for bit (and so the oracle's, which fa_bwd is checked against)."""
    ops = load_mod("_ops")
    print(f"case staged B={B} Hq={Hq} Hkv={Hkv} L={L} D={D} W={W} S={S} {dtype}", flush=True)
    q, k, v, do = make_inputs(B, Hq, Hkv, L, D, dtype, seed=31)
    sc = 1 / math.sqrt(D)
    o, lse = ops.forward(q, k, v, W, S, sc)
    call = ops.BwdCall(q, k, v, o, lse, do, W, S, sc)
    call.run("dq")
    call.run("dkdv")
    staged = (call.dq.clone(), call.dk.clone(), call.dv.clone())
    call.run("all")
    torch.cuda.synchronize()
    for a, b in zip(staged, (call.dq, call.dk, call.dv)):
        assert torch.equal(a, b)
    if B * Hq * L * L <= 1 << 28:
        _, _, rdq, rdk, rdv = naive.attention_fwd_bwd(q, k, v, do, W, S, scale=sc, row_chunk=2048)
        assert_close("dQ", staged[0], rdq)
        assert_close("dK", staged[1], rdk)
        assert_close("dV", staged[2], rdv)


@pytest.mark.parametrize("dtype", [FP, BF], ids=["fp16", "bf16"])
@pytest.mark.parametrize("Hkv", [16, 8, 1])
def test_reference_default_cases(gpu, Hkv, dtype):
    """parse_cases' three cases at the north-star bar (run_case: O, LSE, dQ, dK, dV, every head)."""
    print(f"case reference default Hkv={Hkv} {dtype}", flush=True)
    run_case(1, 16, Hkv, 4096, 16, 256, 4, dtype, seed=48, with_naive=False)


@pytest.mark.parametrize("dtype", [FP, BF], ids=["fp16", "bf16"])
@pytest.mark.parametrize("Hkv", [16, 8, 1])
def test_reference_correctness_check_protocol(gpu, Hkv, dtype):
    """correctness_check's own protocol (benchmark_backward_speed.py:682-717): q, k, v from
    torch.manual_seed(0) on the device, o from the registry form, dO = randn_like(o), then
    allclose(atol=5e-2, rtol=5e-2) on O, dQ, dK, dV -- here against the float32 oracle."""
    fa = load_pkg()
    print(f"case correctness_check Hkv={Hkv} {dtype}", flush=True)
    torch.manual_seed(0)
    shape_q, shape_kv = (1, 16, 4096, 16), (1, Hkv, 4096, 16)
    q = torch.randn(shape_q, device="cuda", dtype=dtype)
    k = torch.randn(shape_kv, device="cuda", dtype=dtype)
    v = torch.randn(shape_kv, device="cuda", dtype=dtype)
    qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
    o = fa.swa_sink_attention(qg, kg, vg, 256, 4)
    do = torch.randn_like(o)
    o.backward(do)
    torch.cuda.synchronize()
    ro, _, rdq, rdk, rdv = naive.attention_fwd_bwd(q, k, v, do, 256, 4, scale=0.25, row_chunk=2048)
    for name, got, ref in (("O", o, ro), ("dQ", qg.grad, rdq), ("dK", kg.grad, rdk), ("dV", vg.grad, rdv)):
        assert torch.allclose(got.detach().float(), ref, atol=5e-2, rtol=5e-2), (name, float((got - ref).abs().max()))
