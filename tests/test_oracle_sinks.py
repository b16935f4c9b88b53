"""Pins the oracle's GPT-OSS learned sinks (naive.attention_fwd_bwd_sinks, naive.gpt_oss_eager).

A learned sink is a per-head logit in every row's softmax denominator with no value row.  The
checks below state that independently of the oracle's formula:
  * SDPA (a library routine) over K/V with one extra all-zero key whose additive-mask column
    holds the sink logit: its score is then exactly the sink and its value contributes nothing;
    autograd through the mask gives the sink gradient;
  * the installed transformers package's own GPT-OSS eager attention;
  * a sink of -inf is no sink at all, and a huge sink drives O to zero;
  * finite differences (gradcheck, float64) for dq, dk, dv and the sink gradient.
A dropped exp(sink) term, a sink added to the numerator, a wrong sign of the sink gradient or a
sink indexed by KV head instead of query head fails one of them.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import naive


def _inputs(B, Hq, Hkv, L, D, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, L, D, generator=g, dtype=torch.float64).to(dtype)
    k = torch.randn(B, Hkv, L, D, generator=g, dtype=torch.float64).to(dtype)
    v = torch.randn(B, Hkv, L, D, generator=g, dtype=torch.float64).to(dtype)
    do = torch.randn(B, Hq, L, D, generator=g, dtype=torch.float64).to(dtype)
    sinks = (2.0 * torch.randn(Hq, generator=g, dtype=torch.float64)).to(dtype)
    return q, k, v, do, sinks


def _sdpa_virtual_key(q, k, v, sinks, W, S, scale):
    """SDPA over [K; 0] and [V; 0] with an additive mask whose last column is the sink logit."""
    B, Hq, L, D = q.shape
    G = Hq // k.shape[1]
    kr = k.repeat_interleave(G, dim=1)
    vr = v.repeat_interleave(G, dim=1)
    zeros = torch.zeros(B, Hq, 1, D, dtype=q.dtype)
    kx = torch.cat([kr, zeros], dim=2)
    vx = torch.cat([vr, zeros], dim=2)
    keep = naive.allowed_mask(L, W, S)
    bias = torch.zeros(L, L, dtype=q.dtype).masked_fill(~keep, float("-inf"))
    bias = bias.view(1, 1, L, L).expand(B, Hq, L, L)
    col = sinks.view(1, Hq, 1, 1).expand(B, Hq, L, 1)
    mask = torch.cat([bias, col], dim=-1)
    o = F.scaled_dot_product_attention(q, kx, vx, attn_mask=mask, scale=scale)
    s = torch.matmul(q, kx.transpose(-1, -2)) * scale + mask
    return o, torch.logsumexp(s, dim=-1)


@pytest.mark.parametrize("B,Hq,Hkv,L,D,W,S", [(1, 4, 2, 19, 8, 5, 0), (2, 2, 1, 33, 16, 7, 3), (1, 3, 3, 12, 8, 12, 0)])
def test_sinks_match_sdpa_virtual_key(B, Hq, Hkv, L, D, W, S):
    q, k, v, do, sinks = _inputs(B, Hq, Hkv, L, D, seed=L + W)
    scale = 1.0 / math.sqrt(D)
    o, lse, dq, dk, dv, ds = naive.attention_fwd_bwd_sinks(q, k, v, sinks, do, W, S, scale,
                                                          compute_dtype=torch.float64)
    qq, kk, vv, ss = (t.clone().requires_grad_() for t in (q, k, v, sinks))
    ro, rlse = _sdpa_virtual_key(qq, kk, vv, ss, W, S, scale)
    ro.backward(do)
    torch.testing.assert_close(o, ro.detach(), rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(lse, rlse.detach(), rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(dq, qq.grad, rtol=1e-9, atol=1e-9)
    torch.testing.assert_close(dk, kk.grad, rtol=1e-9, atol=1e-9)
    torch.testing.assert_close(dv, vv.grad, rtol=1e-9, atol=1e-9)
    torch.testing.assert_close(ds, ss.grad, rtol=1e-9, atol=1e-9)


def test_sinks_match_transformers_gpt_oss_eager():
    mod = pytest.importorskip("transformers.models.gpt_oss.modeling_gpt_oss")
    from transformers.masking_utils import sliding_window_causal_mask_function

    B, Hq, Hkv, L, D, W = 2, 4, 2, 24, 16, 6
    q, k, v, do, sinks = _inputs(B, Hq, Hkv, L, D, seed=5)
    scale = 1.0 / math.sqrt(D)

    class Stub(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.sinks = torch.nn.Parameter(sinks.clone())
            self.num_key_value_groups = Hq // Hkv

    stub = Stub().eval()
    # transformers' own sliding-window predicate, evaluated index by index
    fn = sliding_window_causal_mask_function(W)
    t = torch.tensor
    keep = torch.tensor([[bool(fn(t(0), t(0), t(i), t(j))) for j in range(L)] for i in range(L)])
    assert torch.equal(keep, naive.allowed_mask(L, W, 0))
    add = torch.zeros(L, L, dtype=q.dtype).masked_fill(~keep, float("-inf")).view(1, 1, L, L)
    qq, kk, vv = (t.clone().requires_grad_() for t in (q, k, v))
    hf_o, _ = mod.eager_attention_forward(stub, qq, kk, vv, add, scaling=scale)
    hf_o = hf_o.transpose(1, 2)  # transformers returns [B, L, H, D]
    hf_o.backward(do)
    o, _, dq, dk, dv, ds = naive.attention_fwd_bwd_sinks(q, k, v, sinks, do, W, 0, scale,
                                                        compute_dtype=torch.float64)
    torch.testing.assert_close(o, hf_o.detach(), rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(dq, qq.grad, rtol=1e-9, atol=1e-9)
    torch.testing.assert_close(dk, kk.grad, rtol=1e-9, atol=1e-9)
    torch.testing.assert_close(dv, vv.grad, rtol=1e-9, atol=1e-9)
    torch.testing.assert_close(ds, stub.sinks.grad, rtol=1e-9, atol=1e-9)
    # the restatement of the eager path agrees as well (window and full layers)
    torch.testing.assert_close(naive.gpt_oss_eager(q, k, v, sinks, W, scale), o, rtol=1e-10, atol=1e-10)
    of, *_ = naive.attention_fwd_bwd_sinks(q, k, v, sinks, do, L, 0, scale, compute_dtype=torch.float64)
    torch.testing.assert_close(naive.gpt_oss_eager(q, k, v, sinks, None, scale), of, rtol=1e-10, atol=1e-10)


def test_sink_limits():
    q, k, v, do, _ = _inputs(1, 2, 1, 20, 8, seed=9)
    ref = naive.attention_fwd_bwd(q, k, v, do, 6, 2, None, compute_dtype=torch.float64)
    ninf = torch.full((2,), float("-inf"), dtype=torch.float64)
    got = naive.attention_fwd_bwd_sinks(q, k, v, ninf, do, 6, 2, None, compute_dtype=torch.float64)
    for a, b in zip(ref, got[:5]):
        torch.testing.assert_close(a, b, rtol=0, atol=0)
    assert torch.all(got[5] == 0)
    big = torch.full((2,), 80.0, dtype=torch.float64)
    o = naive.attention_fwd_bwd_sinks(q, k, v, big, do, 6, 2, None, compute_dtype=torch.float64)[0]
    assert o.abs().max() < 1e-20


def test_sink_gradient_depends_on_query_head():
    # two query heads share one KV head but have different sinks: each head's sink gradient
    # must come from its own rows only
    q, k, v, do, sinks = _inputs(1, 2, 1, 16, 8, seed=21)
    ds = naive.attention_fwd_bwd_sinks(q, k, v, sinks, do, 4, 0, None, compute_dtype=torch.float64)[5]
    do2 = do.clone()
    do2[:, 1] = 0
    ds2 = naive.attention_fwd_bwd_sinks(q, k, v, sinks, do2, 4, 0, None, compute_dtype=torch.float64)[5]
    assert ds2[1] == 0 and ds2[0] == ds[0] and ds[1] != 0


def test_sinks_gradcheck_float64():
    q, k, v, _, sinks = _inputs(1, 2, 1, 9, 4, seed=3)
    args = [t.clone().requires_grad_() for t in (q, k, v, sinks)]
    assert torch.autograd.gradcheck(lambda a, b, c, d: naive.OracleAttentionSinks.apply(a, b, c, d, 3, 1, 0.7),
                                    args, eps=1e-6, atol=1e-6)
