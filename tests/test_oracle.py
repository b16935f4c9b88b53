"""Pins the oracle (oracle/) before anything is compared with it.

Each check is chosen so that a plausible slip in the oracle (a wrong mask inequality, a
dropped sink term, a wrong GQA head map, a transposed operand or a missing scale in the
backward) fails at least one of them.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import loops, naive


def _inputs(B, Hq, Hkv, L, D, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, L, D, generator=g, dtype=torch.float64).to(dtype)
    k = torch.randn(B, Hkv, L, D, generator=g, dtype=torch.float64).to(dtype)
    v = torch.randn(B, Hkv, L, D, generator=g, dtype=torch.float64).to(dtype)
    do = torch.randn(B, Hq, L, D, generator=g, dtype=torch.float64).to(dtype)
    return q, k, v, do


@pytest.mark.parametrize("L,W,S", [(1, 1, 0), (9, 3, 2), (17, 1, 4), (16, 20, 0), (23, 0, 5), (12, 4, 12)])
def test_mask_matches_python_predicate(L, W, S):
    m = naive.allowed_mask(L, W, S)
    for i in range(L):
        for j in range(L):
            assert bool(m[i, j]) == loops.allowed(i, j, W, S)


def test_mask_known_rows():
    # W=3, S=2, L=8: row 6 sees window keys 4,5,6 and sinks 0,1; row 1 sees 0,1 only.
    m = naive.allowed_mask(8, 3, 2)
    assert m[6].nonzero().flatten().tolist() == [0, 1, 4, 5, 6]
    assert m[1].nonzero().flatten().tolist() == [0, 1]
    assert m[0].nonzero().flatten().tolist() == [0]


def test_expand_kv_head_mapping():
    x = torch.arange(2 * 3 * 1 * 1, dtype=torch.float64).view(2, 3, 1, 1)
    y = naive.expand_kv(x, 4)
    assert y.shape == (2, 12, 1, 1)
    for h in range(12):
        assert torch.equal(y[:, h], x[:, h // 4])


def _sdpa_masked(q, k, v, W, S, scale):
    group = q.shape[1] // k.shape[1]
    mask = naive.allowed_mask(q.shape[2], W, S)
    return F.scaled_dot_product_attention(q, naive.expand_kv(k, group), naive.expand_kv(v, group),
                                          attn_mask=mask, scale=scale)


@pytest.mark.parametrize("B,Hq,Hkv,L,D,W,S", [
    (1, 2, 2, 33, 8, 5, 3),
    (2, 4, 1, 40, 16, 7, 0),
    (1, 8, 2, 64, 16, 16, 4),
    (1, 3, 3, 29, 4, 1, 9),
    (1, 2, 1, 31, 8, 0, 6),
])
def test_fwd_bwd_matches_sdpa_autograd(B, Hq, Hkv, L, D, W, S):
    """Forward vs SDPA with an explicit boolean mask (independent library routine); backward vs
    autograd through SDPA; LSE vs logsumexp of explicitly masked scores."""
    q, k, v, do = _inputs(B, Hq, Hkv, L, D, seed=L * 7 + D)
    scale = 1.0 / math.sqrt(D)
    qr, kr, vr = (t.clone().requires_grad_() for t in (q, k, v))
    ref = _sdpa_masked(qr, kr, vr, W, S, scale)
    ref.backward(do)
    o, lse, dq, dk, dv = naive.attention_fwd_bwd(q, k, v, do, W, S, compute_dtype=torch.float64)
    torch.testing.assert_close(o, ref.detach(), rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(dq, qr.grad, rtol=1e-9, atol=1e-10)
    torch.testing.assert_close(dk, kr.grad, rtol=1e-9, atol=1e-10)
    torch.testing.assert_close(dv, vr.grad, rtol=1e-9, atol=1e-10)
    group = Hq // Hkv
    s = torch.matmul(q, naive.expand_kv(k, group).transpose(-1, -2)) * scale
    s = s.masked_fill(~naive.allowed_mask(L, W, S), float("-inf"))
    torch.testing.assert_close(lse, torch.logsumexp(s, dim=-1), rtol=1e-12, atol=1e-12)


def test_matches_python_loops():
    q, k, v, do = _inputs(1, 4, 2, 11, 3, seed=5)
    W, S, scale = 3, 2, 0.7
    o, lse, *_ = naive.attention_fwd_bwd(q, k, v, do, W, S, scale=scale, compute_dtype=torch.float64)
    lo, llse = loops.forward(q[0].tolist(), k[0].tolist(), v[0].tolist(), W, S, scale)
    np.testing.assert_allclose(o[0].numpy(), np.array(lo), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lse[0].numpy(), np.array(llse), rtol=1e-12, atol=1e-12)


def test_full_window_is_sdpa_causal():
    """W >= L and S = 0 is plain causal attention: SDPA's is_causal mode (no mask from us)."""
    q, k, v, do = _inputs(1, 4, 1, 37, 8, seed=11)
    qr, kr, vr = (t.clone().requires_grad_() for t in (q, k, v))
    ref = F.scaled_dot_product_attention(qr, naive.expand_kv(kr, 4), naive.expand_kv(vr, 4), is_causal=True)
    ref.backward(do)
    for W, S in [(37, 0), (1000, 0), (1, 37), (5, 40)]:  # S >= L is also full causal
        o, _, dq, dk, dv = naive.attention_fwd_bwd(q, k, v, do, W, S, compute_dtype=torch.float64)
        torch.testing.assert_close(o, ref.detach())
        torch.testing.assert_close(dq, qr.grad)
        torch.testing.assert_close(dk, kr.grad)
        torch.testing.assert_close(dv, vr.grad)


def test_window_one_closed_form():
    """W = 1, S = 0: each row sees only itself, so o = v, dq = dk = 0 and dv = group sum of dO."""
    q, k, v, do = _inputs(2, 6, 2, 19, 8, seed=3)
    o, lse, dq, dk, dv = naive.attention_fwd_bwd(q, k, v, do, 1, 0, compute_dtype=torch.float64)
    torch.testing.assert_close(o, naive.expand_kv(v, 3))
    assert dq.abs().max() < 1e-12 and dk.abs().max() < 1e-12
    torch.testing.assert_close(dv, do.view(2, 2, 3, 19, 8).sum(dim=2))
    torch.testing.assert_close(lse, (q * naive.expand_kv(k, 3)).sum(-1) / math.sqrt(8))


def test_gqa_equals_repeated_mha():
    q, k, v, do = _inputs(1, 8, 2, 24, 8, seed=9)
    o, lse, dq, dk, dv = naive.attention_fwd_bwd(q, k, v, do, 6, 2, compute_dtype=torch.float64)
    kr, vr = naive.expand_kv(k, 4), naive.expand_kv(v, 4)
    o2, lse2, dq2, dk2, dv2 = naive.attention_fwd_bwd(q, kr, vr, do, 6, 2, compute_dtype=torch.float64)
    torch.testing.assert_close(o, o2)
    torch.testing.assert_close(lse, lse2)
    torch.testing.assert_close(dq, dq2)
    torch.testing.assert_close(dk, dk2.view(1, 2, 4, 24, 8).sum(2))
    torch.testing.assert_close(dv, dv2.view(1, 2, 4, 24, 8).sum(2))


@pytest.mark.parametrize("W,S", [(4, 2), (1, 3), (7, 0), (20, 0), (0, 5)])
def test_gradcheck_float64(W, S):
    q, k, v, _ = _inputs(1, 4, 2, 10, 4, seed=W * 10 + S)
    q, k, v = (t.requires_grad_() for t in (q, k, v))
    assert torch.autograd.gradcheck(lambda a, b, c: naive.OracleAttention.apply(a, b, c, W, S, 0.6),
                                    (q, k, v), eps=1e-6, atol=1e-7, rtol=1e-5)


def test_invariants():
    q, k, v, do = _inputs(1, 2, 1, 50, 8, seed=21)
    W, S, scale = 9, 3, 1 / math.sqrt(8)
    o, lse, dq, dk, dv = naive.attention_fwd_bwd(q, k, v, do, W, S, compute_dtype=torch.float64)
    mask = naive.allowed_mask(50, W, S)
    s = torch.matmul(q, naive.expand_kv(k, 2).transpose(-1, -2)) * scale
    s = s.masked_fill(~mask, float("-inf"))
    p = torch.exp(s - lse[..., None])
    torch.testing.assert_close(p.sum(-1), torch.ones_like(lse))  # rows sum to 1
    assert bool((lse >= s.amax(-1) - 1e-12).all())                # lse >= row max
    vmin = naive.expand_kv(v, 2).amin(dim=2, keepdim=True)
    vmax = naive.expand_kv(v, 2).amax(dim=2, keepdim=True)
    assert bool((o >= vmin - 1e-12).all() and (o <= vmax + 1e-12).all())  # convex hull
    # Adding one vector c to every key shifts all scores of a row by scale*q.c, which softmax
    # ignores, so O is unchanged; dQ changes by scale * sum_k dS[q,k] c, which is 0 because the
    # rows of dS sum to zero.
    shift = torch.randn(1, 1, 1, 8, dtype=torch.float64, generator=torch.Generator().manual_seed(2))
    o2, _, dq2, _, _ = naive.attention_fwd_bwd(q, k + shift, v, do, W, S, compute_dtype=torch.float64)
    torch.testing.assert_close(o2, o)
    torch.testing.assert_close(dq2, dq)
    dp = torch.matmul(do, naive.expand_kv(v, 2).transpose(-1, -2))
    ds = p * (dp - (do * o).sum(-1, keepdim=True))
    assert ds.sum(-1).abs().max() < 1e-10


def test_row_chunking_and_head_subset_do_not_change_results():
    q, k, v, do = _inputs(1, 4, 2, 70, 8, seed=4)
    full = naive.attention_fwd_bwd(q, k, v, do, 9, 3, compute_dtype=torch.float64)
    chunked = naive.attention_fwd_bwd(q, k, v, do, 9, 3, compute_dtype=torch.float64, row_chunk=16)
    for a, b in zip(full, chunked):
        torch.testing.assert_close(a, b)
    sub = naive.attention_fwd_bwd(q, k, v, do, 9, 3, compute_dtype=torch.float64, heads=[0, 1])
    torch.testing.assert_close(sub[0][:, :2], full[0][:, :2])
    torch.testing.assert_close(sub[3][:, 0], full[3][:, 0])  # KV head 0 is fed by heads 0, 1 only


def test_naive_reference_dtype_path_close_to_fp64():
    """The reference-dtype baseline (scores in fp16/bf16, softmax fp32) agrees with the fp64
    oracle to low-precision accuracy."""
    q, k, v, _ = _inputs(1, 4, 2, 64, 16, seed=13)
    o64 = naive.attention_fwd_bwd(q, k, v, torch.zeros_like(q), 16, 4, compute_dtype=torch.float64)[0]
    for dt in (torch.bfloat16, torch.float16):
        o = naive.naive_attention(q.to(dt), k.to(dt), v.to(dt), 16, 4)
        assert o.dtype == dt
        assert (o.double() - o64).abs().max() < 5e-2


@pytest.mark.parametrize("L,W,S,r0,learned", [(900, 128, 4, 836, False), (900, 128, 4, 413, False),
                                              (1000, 300, 40, 936, False), (1000, 300, 40, 500, False),
                                              (900, 128, 0, 836, True), (900, 128, 0, 300, True)])
def test_long_context_subproblem_is_exact(L, W, S, r0, learned):
    """The sub-problem tests/test_gpu_long.py checks sampled rows with (the S sinks, then
    positions [r0 - W - 64, r0 + 64)) gives those rows the same O, LSE and dQ as the whole
    sequence, and at the sequence's end the last 64 keys the same dK and dV; with learned sink
    logits as well (they add a term per head to every row, not a key)."""
    from test_gpu_long import subproblem_keys

    q, k, v, do = _inputs(1, 4, 2, L, 8, seed=r0)
    sk = torch.randn(4, dtype=torch.float64, generator=torch.Generator().manual_seed(r0))
    run = (lambda *t: naive.attention_fwd_bwd_sinks(t[0], t[1], t[2], sk, t[3], W, S, compute_dtype=torch.float64)) \
        if learned else (lambda *t: naive.attention_fwd_bwd(*t, W, S, compute_dtype=torch.float64))
    full = run(q, k, v, do)
    idx = subproblem_keys(r0, W, S)
    sub = run(*(t.index_select(2, idx) for t in (q, k, v, do)))
    n, rows = idx.numel(), slice(r0, r0 + 64)
    for i in (0, 1, 2):  # O, LSE, dQ
        torch.testing.assert_close(sub[i][:, :, n - 64:], full[i][:, :, rows])
    if r0 + 64 == L:
        for i in (3, 4):  # dK, dV
            torch.testing.assert_close(sub[i][:, :, n - 64:], full[i][:, :, rows])
    else:  # away from the end, the keys also get gradient from rows past the sample
        assert not torch.allclose(sub[3][:, :, n - 64:], full[3][:, :, rows])


@pytest.mark.parametrize("L,W,S,chunk,learned", [(900, 128, 4, 100, False), (1000, 300, 40, 256, False),
                                                 (700, 1, 3, 64, False), (500, 2000, 5, 128, False),
                                                 (900, 128, 0, 128, True), (800, 64, 6, 97, True)])
def test_sink_key_grads_equal_the_whole_sequence(L, W, S, chunk, learned):
    """naive.sink_key_grads (row chunks on sub-problems, dO zeroed outside the chunk) gives the sink
    keys' dK/dV rows and the learned sinks' gradient of the whole-sequence oracle, in float64;
    keeping the sub-problems' other rows instead of zeroing their dO does not."""
    q, k, v, do = _inputs(1, 4, 2, L, 8, seed=L + W)
    sk = torch.randn(4, dtype=torch.float64, generator=torch.Generator().manual_seed(W)) if learned else None
    if learned:
        full = naive.attention_fwd_bwd_sinks(q, k, v, sk, do, W, S, compute_dtype=torch.float64)
    else:
        full = naive.attention_fwd_bwd(q, k, v, do, W, S, compute_dtype=torch.float64)
    dk, dv, ds, ds_terms = naive.sink_key_grads(q, k, v, do, W, S, sinks=sk, compute_dtype=torch.float64,
                                                row_chunk=chunk)
    torch.testing.assert_close(dk, full[3][:, :, :S])
    torch.testing.assert_close(dv, full[4][:, :, :S])
    if learned:
        torch.testing.assert_close(ds, full[5])
        delta = (do * full[0]).sum(-1)
        terms = (torch.exp(sk.view(1, -1, 1) - full[1]) * delta).abs().sum(dim=(0, 2))
        torch.testing.assert_close(ds_terms, terms)
    else:
        assert ds is None and ds_terms is None
    # without the zeroing, the rows before each chunk (whose windows the sub-problem truncates) count
    # again: a mistake this check is there to catch
    if S > 0 and L > chunk + W:
        wrong = torch.zeros_like(dk)
        for r0 in range(0, L, chunk):
            r1 = min(L, r0 + chunk)
            t0 = r0 - W + 1
            idx = torch.arange(r1) if t0 <= S else torch.cat([torch.arange(S), torch.arange(t0, r1)])
            r = naive.attention_fwd_bwd(*(t.index_select(2, idx) for t in (q, k, v, do)), W, S,
                                        compute_dtype=torch.float64)
            wrong += r[3][:, :, :S]
        assert not torch.allclose(wrong, full[3][:, :, :S])


@pytest.mark.parametrize("L,W,S,chunk,dt", [(1500, 128, 4, 256, torch.bfloat16), (1200, 300, 40, 200, torch.float16),
                                            (800, 50, 3, 100, torch.bfloat16), (300, 1000, 6, 64, torch.float16)])
def test_lowp_sink_key_grads_follow_the_naive_path(L, W, S, chunk, dt):
    """naive.naive_lowp_sink_key_grads (the naive 16-bit path's rounding points, banded, float32
    products) gives the sink keys' dK/dV of naive_attention's own autograd backward in that dtype:
    at least 99% of the values bit for bit, the rest within one unit in the last place at the
    tensor's largest magnitude (a float32 sum taken in another order can round one 16-bit value
    the other way); so its error against the float64 oracle is the naive path's."""
    g = torch.Generator().manual_seed(L + S)
    Hq, Hkv, D = 8, 2, 64
    q, k, v, do = (torch.randn(1, h, L, D, generator=g).to(dt) for h in (Hq, Hkv, Hkv, Hq))
    qc, kc, vc = (t.clone().requires_grad_() for t in (q, k, v))
    naive.naive_attention(qc, kc, vc, W, S).backward(do)
    dk, dv = naive.naive_lowp_sink_key_grads(q, k, v, do, W, S, row_chunk=chunk)
    ulp = 2.0 ** -7 if dt is torch.bfloat16 else 2.0 ** -10
    for got, want in ((dk, kc.grad[:, :, :S].float()), (dv, vc.grad[:, :, :S].float())):
        assert got.dtype == torch.float32 and torch.equal(got, got.to(dt).float())
        diff = (got - want).abs()
        assert float(diff.max()) <= ulp * float(want.abs().max()), float(diff.max())
        assert int((diff > 0).sum()) <= diff.numel() // 100, int((diff > 0).sum())
    ref = naive.attention_fwd_bwd(q, k, v, do, W, S, compute_dtype=torch.float64)
    err_naive = float((kc.grad[:, :, :S].double() - ref[3][:, :, :S]).abs().max())
    err_emul = float((dk.double() - ref[3][:, :, :S]).abs().max())
    assert abs(err_emul - err_naive) <= 0.1 * err_naive
