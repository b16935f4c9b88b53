"""CPU pins of the variable-length oracle (oracle/naive.py attention_fwd_bwd_varlen).

The oracle treats every packed sequence as an independent fixed-length problem.  It is checked
against an independent statement of a packed batch: ONE scaled_dot_product_attention call over
all packed rows with the block-diagonal, position-relative mask (packed_allowed_mask), with the
gradients from autograd -- and, for learned sinks, with one extra zero key whose additive mask
column holds the sink logit.  Float64 throughout.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import naive

CASES = [
    # cu_seqlens, Hq, Hkv, D, W, S
    ([0, 5, 5, 40, 97], 4, 2, 16, 7, 2),
    ([0, 64], 2, 1, 16, 64, 0),
    ([0, 1, 2, 130], 4, 4, 8, 33, 5),
    ([0, 70, 71, 150], 6, 2, 16, 1, 3),
]


def _inputs(total, Hq, Hkv, D, seed):
    g = torch.Generator().manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)
    return mk(total, Hq, D), mk(total, Hkv, D), mk(total, Hkv, D), mk(total, Hq, D)


def _packed_sdpa(q, k, v, do, cu, W, S, scale, sinks=None):
    """O, LSE and gradients of the packed batch from one SDPA call (+ autograd)."""
    total, Hq, D = q.shape
    G = Hq // k.shape[1]
    qb = q.permute(1, 0, 2).unsqueeze(0).clone().requires_grad_()
    kb = k.permute(1, 0, 2).unsqueeze(0).clone().requires_grad_()
    vb = v.permute(1, 0, 2).unsqueeze(0).clone().requires_grad_()
    ke, ve = kb.repeat_interleave(G, 1), vb.repeat_interleave(G, 1)
    keep = naive.packed_allowed_mask(torch.tensor(cu), W, S)
    bias = torch.zeros(total, total, dtype=torch.float64).masked_fill(~keep, float("-inf"))
    bias = bias.expand(1, Hq, total, total)
    sk = None
    if sinks is not None:  # one extra key: zero K and V, mask column = the head's sink logit
        sk = sinks.clone().requires_grad_()
        zero = torch.zeros(1, Hq, 1, D, dtype=torch.float64)
        ke, ve = torch.cat([ke, zero], 2), torch.cat([ve, zero], 2)
        bias = torch.cat([bias, sk.view(1, Hq, 1, 1).expand(1, Hq, total, 1)], 3)
    o = F.scaled_dot_product_attention(qb, ke, ve, attn_mask=bias, scale=scale)
    o.backward(do.permute(1, 0, 2).unsqueeze(0))
    s = torch.matmul(qb.detach(), ke.detach().transpose(-1, -2)) * scale + bias.detach()
    lse = torch.logsumexp(s, dim=-1)[0]
    to_packed = lambda t: t[0].permute(1, 0, 2)
    out = (to_packed(o.detach()), lse, to_packed(qb.grad), to_packed(kb.grad), to_packed(vb.grad))
    return out + ((sk.grad,) if sinks is not None else ())


@pytest.mark.parametrize("cu,Hq,Hkv,D,W,S", CASES)
def test_varlen_oracle_matches_one_packed_sdpa(cu, Hq, Hkv, D, W, S):
    q, k, v, do = _inputs(cu[-1], Hq, Hkv, D, seed=len(cu) + W)
    scale = 1.0 / math.sqrt(D)
    got = naive.attention_fwd_bwd_varlen(q, k, v, do, torch.tensor(cu), W, S, scale, compute_dtype=torch.float64)
    want = _packed_sdpa(q, k, v, do, cu, W, S, scale)
    for name, a, b in zip(("O", "LSE", "dQ", "dK", "dV"), got, want):
        assert torch.allclose(a, b, atol=1e-10, rtol=1e-10), (name, float((a - b).abs().max()))


@pytest.mark.parametrize("cu,Hq,Hkv,D,W,S", CASES[:2])
def test_varlen_oracle_learned_sinks_match_packed_sdpa(cu, Hq, Hkv, D, W, S):
    q, k, v, do = _inputs(cu[-1], Hq, Hkv, D, seed=7)
    sinks = torch.randn(Hq, generator=torch.Generator().manual_seed(3), dtype=torch.float64) * 2
    scale = 1.0 / math.sqrt(D)
    got = naive.attention_fwd_bwd_varlen(q, k, v, do, torch.tensor(cu), W, S, scale, sinks=sinks,
                                         compute_dtype=torch.float64)
    want = _packed_sdpa(q, k, v, do, cu, W, S, scale, sinks=sinks)
    for name, a, b in zip(("O", "LSE", "dQ", "dK", "dV", "dsinks"), got, want):
        assert torch.allclose(a, b, atol=1e-10, rtol=1e-10), (name, float((a - b).abs().max()))


def test_single_sequence_equals_the_fixed_length_oracle():
    q, k, v, do = _inputs(77, 4, 2, 16, seed=5)
    got = naive.attention_fwd_bwd_varlen(q, k, v, do, torch.tensor([0, 77]), 9, 3, 0.25, compute_dtype=torch.float64)
    as4 = lambda t: t.permute(1, 0, 2).unsqueeze(0)
    want = naive.attention_fwd_bwd(as4(q), as4(k), as4(v), as4(do), 9, 3, 0.25, compute_dtype=torch.float64)
    for a, b in zip(got[:1] + got[2:], want[:1] + want[2:]):
        assert torch.equal(a, b[0].permute(1, 0, 2))
    assert torch.equal(got[1], want[1][0])


def test_packed_mask_is_block_diagonal():
    keep = naive.packed_allowed_mask(torch.tensor([0, 3, 3, 7]), 2, 1)
    assert keep.shape == (7, 7)
    assert not keep[3:, :3].any() and not keep[:3, 3:].any()
    # second sequence (rows 3..6): positions 0..3, window 2, one sink
    assert keep[3:, 3:].tolist() == naive.allowed_mask(4, 2, 1).tolist()
