"""CPU tests of the Python boundary (attention.py) with the tensor-level calls (_ops.forward /
_ops.backward) replaced, inside this test only, by the oracle.  They check the plumbing that
mirrors flash_attention_gpt_oss.py:340-438 -- defaults, assertion messages, the saved-tensor
set and the 7-tuple of gradients -- and that without a GPU the product path raises instead of
falling back to a CPU implementation."""
import math

import pytest
import torch

from conftest import load_mod, load_pkg
from oracle import naive

fa = load_pkg()
_ops = load_mod("_ops")


@pytest.fixture
def oracle_ops(monkeypatch):
    calls = {"fwd": [], "bwd": []}

    def fwd(q, k, v, window, sink, scale):
        calls["fwd"].append((window, sink, scale))
        o, lse, *_ = naive.attention_fwd_bwd(q, k, v, torch.zeros_like(q), window, sink, scale=scale,
                                             compute_dtype=torch.float64)
        return o.to(q.dtype), lse.float()

    def bwd(q, k, v, o, lse, do, window, sink, scale):
        calls["bwd"].append((window, sink, scale, o.shape, lse.shape))
        _, _, dq, dk, dv = naive.attention_fwd_bwd(q, k, v, do, window, sink, scale=scale,
                                                   compute_dtype=torch.float64)
        return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype)

    monkeypatch.setattr(_ops, "forward", fwd)
    monkeypatch.setattr(_ops, "backward", bwd)
    return calls


def _t(*shape, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float64)


def test_forward_backward_plumbing(oracle_ops):
    q = _t(1, 4, 16, 16, seed=1).requires_grad_()
    k = _t(1, 2, 16, 16, seed=2).requires_grad_()
    v = _t(1, 2, 16, 16, seed=3).requires_grad_()
    o = fa.flash_swda_with_sink(q, k, v, 5, 2)
    assert oracle_ops["fwd"] == [(5, 2, 1.0 / math.sqrt(16))]  # default scale 1/sqrt(D)
    do = _t(1, 4, 16, 16, seed=4)
    o.backward(do)
    window, sink, scale, oshape, lshape = oracle_ops["bwd"][0]
    assert (window, sink, scale) == (5, 2, 0.25)
    assert oshape == (1, 4, 16, 16) and lshape == (1, 4, 16)  # saved o and lse reach backward
    _, _, dq, dk, dv = naive.attention_fwd_bwd(q.detach(), k.detach(), v.detach(), do, 5, 2,
                                               compute_dtype=torch.float64)
    torch.testing.assert_close(q.grad, dq)
    torch.testing.assert_close(k.grad, dk)
    torch.testing.assert_close(v.grad, dv)


def test_backward_returns_seven_gradients(oracle_ops):
    q = _t(1, 2, 8, 16).requires_grad_()
    k = _t(1, 2, 8, 16).requires_grad_()
    v = _t(1, 2, 8, 16).requires_grad_()

    o = fa.FlashSWDAWithSink.apply(q, k, v, 3, 1, True, 0.5)
    grads = o.grad_fn.apply(torch.ones_like(o))
    assert len(grads) == 7 and all(g is None for g in grads[3:])
    assert oracle_ops["fwd"][0][2] == 0.5  # explicit softmax_scale is used as given


def test_registry_form(oracle_ops):
    q, k, v = _t(1, 2, 8, 32), _t(1, 1, 8, 32), _t(1, 1, 8, 32)
    fa.swa_sink_attention(q, k, v, 4, 1)
    assert oracle_ops["fwd"] == [(4, 1, 1.0 / math.sqrt(32))]


@pytest.mark.parametrize("args,msg", [
    (dict(is_causal=False), "Currently, only causal attention is supported"),
    (dict(q=(1, 4, 8, 16), v=(1, 2, 9, 16), k=(1, 2, 9, 16)), "Query and Value shapes must be compatible"),
    (dict(k=(1, 2, 8, 32)), "Key and Value shapes must be the same"),
    (dict(q=(1, 4, 8, 256), k=(1, 2, 8, 256), v=(1, 2, 8, 256)), "Head dimension must be less than or equal to 128"),
    (dict(q=(1, 3, 8, 16)), "Number of query heads must be divisible by number of K/V heads"),
])
def test_reference_assertions(oracle_ops, args, msg):
    shapes = dict(q=(1, 4, 8, 16), k=(1, 2, 8, 16), v=(1, 2, 8, 16))
    shapes.update({n: args[n] for n in ("q", "k", "v") if n in args})
    q, k, v = (_t(*shapes[n]) for n in ("q", "k", "v"))
    with pytest.raises(AssertionError, match=msg):
        fa.FlashSWDAWithSink.apply(q, k, v, 4, 1, args.get("is_causal", True), None)
    assert oracle_ops["fwd"] == []


def test_cpu_tensors_raise_without_fallback():
    q, k, v = (torch.randn(1, 2, 8, 16, dtype=torch.bfloat16) for _ in range(3))
    with pytest.raises(RuntimeError, match="need GPU tensors"):
        fa.flash_swda_with_sink(q, k, v, 4, 1)
