"""TEST INFRASTRUCTURE ONLY: restatement of the reference's naive attention.

Follows benchmark_backward_speed.py:40-54 (mask, KV repeat) and :68-85
(pytorch_naive_attention).  See oracle/__init__.py for how each function is pinned.
"""
from __future__ import annotations

import math
from typing import Optional

import torch


def allowed_mask(seq_len: int, window_size: int, sink_size: int, device=None) -> torch.Tensor:
    """[L, L] bool, True where query row q may attend key column k:
    k <= q and (q - k < W or k < S).  Same predicate as create_mask_bool
    (benchmark_backward_speed.py:40-46): its sliding term col >= row - (W-1) is q - k < W."""
    pos = torch.arange(seq_len, device=device)
    qq = pos.view(-1, 1)
    kk = pos.view(1, -1)
    return (kk <= qq) & (((qq - kk) < window_size) | (kk < sink_size))


def expand_kv(x: torch.Tensor, group: int) -> torch.Tensor:
    """[B, Hkv, L, D] -> [B, Hkv*group, L, D], head h reading KV head h // group
    (repeat_kv, benchmark_backward_speed.py:49-54)."""
    return x if group == 1 else x.repeat_interleave(group, dim=1)


def naive_attention(q, k, v, window_size: int, sink_size: int, scale: Optional[float] = None):
    """The reference's baseline path, in the input dtype: dense scores in q's dtype, boolean
    mask, softmax accumulated in float32 then cast back, probabilities @ V
    (benchmark_backward_speed.py:68-85).  Autograd provides its backward."""
    group = q.shape[1] // k.shape[1]
    k = expand_kv(k, group)
    v = expand_kv(v, group)
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    scores = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scale
    keep = allowed_mask(q.shape[2], window_size, sink_size, device=q.device)
    scores = scores.masked_fill(~keep, float("-inf"))
    probs = torch.softmax(scores, dim=-1, dtype=torch.float32).to(q.dtype)
    return torch.matmul(probs, v)


@torch.no_grad()
def attention_fwd_bwd(q, k, v, do, window_size: int, sink_size: int, scale: Optional[float] = None,
                      compute_dtype=torch.float32, row_chunk: Optional[int] = None, heads=None):
    """Explicit forward and backward of masked attention, evaluated in `compute_dtype`.

    Returns (o, lse, dq, dk, dv) in compute_dtype on the inputs' device, with
      s = scale * q.k over allowed keys, lse = logsumexp(s) (natural log), P = exp(s - lse),
      o = P V, delta = rowsum(dO o O), dS = P (dO V^T - delta),
      dq = scale * dS K, dk = scale * sum_heads dS^T Q, dv = sum_heads P^T dO.
    Work is done one (batch, query head) at a time and `row_chunk` query rows at a time, so
    memory stays at row_chunk x L scores.  `heads` optionally restricts the query heads that
    are evaluated (dq/o/lse of other heads stay 0; dk/dv then only sum the listed heads).
    """
    return _fwd_bwd(q, k, v, do, window_size, sink_size, scale, compute_dtype, row_chunk, heads, None)[:5]


@torch.no_grad()
def attention_fwd_bwd_sinks(q, k, v, sinks, do, window_size: int, sink_size: int = 0,
                            scale: Optional[float] = None, compute_dtype=torch.float32,
                            row_chunk: Optional[int] = None, heads=None):
    """attention_fwd_bwd with GPT-OSS learned sinks: `sinks` [Hq] holds one logit per query head
    that joins every row's softmax denominator without a value row (the eager GptOssAttention
    path of HF transformers, restated by gpt_oss_eager below):
      lse = log(sum_k exp(s) + exp(sink)),  P = exp(s - lse),  P_sink = exp(sink - lse),
      dsink = -sum over batch and rows of P_sink * delta.
    Returns (o, lse, dq, dk, dv, dsinks)."""
    return _fwd_bwd(q, k, v, do, window_size, sink_size, scale, compute_dtype, row_chunk, heads, sinks)


def _fwd_bwd(q, k, v, do, window_size, sink_size, scale, compute_dtype, row_chunk, heads, sinks):
    B, Hq, L, D = q.shape
    Hkv = k.shape[1]
    group = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    R = L if row_chunk is None else int(row_chunk)
    qf, kf, vf, gf = (t.to(compute_dtype) for t in (q, k, v, do))
    o = torch.zeros_like(qf)
    lse = torch.zeros((B, Hq, L), dtype=compute_dtype, device=q.device)
    dq = torch.zeros_like(qf)
    dk = torch.zeros_like(kf)
    dv = torch.zeros_like(vf)
    sk = None if sinks is None else sinks.to(compute_dtype)
    dsinks = None if sinks is None else torch.zeros(Hq, dtype=compute_dtype, device=q.device)
    pos = torch.arange(L, device=q.device)
    head_list = range(Hq) if heads is None else heads
    for b in range(B):
        for h in head_list:
            g = h // group
            K, V = kf[b, g], vf[b, g]
            Kt, Vt = K.t().contiguous(), V.t().contiguous()
            for r0 in range(0, L, R):
                r1 = min(L, r0 + R)
                rows = pos[r0:r1].view(-1, 1)
                keep = (pos.view(1, -1) <= rows) & (((rows - pos.view(1, -1)) < window_size) |
                                                    (pos.view(1, -1) < sink_size))
                Q, G = qf[b, h, r0:r1], gf[b, h, r0:r1]
                s = torch.matmul(Q, Kt) * scale
                s = s.masked_fill(~keep, float("-inf"))
                m = torch.logsumexp(s, dim=-1)
                if sk is not None:
                    m = torch.logaddexp(m, sk[h].expand_as(m))
                p = torch.exp(s - m.view(-1, 1))
                ob = torch.matmul(p, V)
                dp = torch.matmul(G, Vt)
                delta = (G * ob).sum(dim=-1, keepdim=True)
                ds = p * (dp - delta)
                if sk is not None:
                    dsinks[h] -= (torch.exp(sk[h] - m) * delta.view(-1)).sum()
                o[b, h, r0:r1] = ob
                lse[b, h, r0:r1] = m
                dq[b, h, r0:r1] = torch.matmul(ds, K) * scale
                dk[b, g] += torch.matmul(ds.t().contiguous(), Q) * scale
                dv[b, g] += torch.matmul(p.t().contiguous(), G)
    return o, lse, dq, dk, dv, dsinks


@torch.no_grad()
def sink_key_grads(q, k, v, do, window_size: int, sink_size: int, scale: Optional[float] = None, sinks=None,
                   compute_dtype=torch.float32, row_chunk: int = 2048):
    """The gradients that sum over every row of a sequence -- dK/dV of the positional sink keys
    [0, S) and, with learned `sinks`, dsinks -- for one long sequence ([1, H, L, D] tensors),
    without the L x L scores.  Rows are taken `row_chunk` at a time; each chunk [r0, r1) runs
    attention_fwd_bwd(_sinks) on the sub-problem of the sink positions and [r0 - W + 1, r1) (the
    whole prefix [0, r1) while the chunk's windows reach the sinks), in which every row of the
    chunk sees exactly its keys of the whole sequence, with dO set to zero on the sub-problem's
    other rows.  Every row's contribution to these gradients is linear in its dO row, so the
    zeroed rows add nothing and the chunk sums are exact.  Returns (dk [1, Hkv, S, D],
    dv [1, Hkv, S, D], dsinks [Hq] or None, sum over rows of |P_sink * delta| [Hq] or None: the
    size of dsinks' terms), accumulated in float64."""
    _, Hq, L, D = q.shape
    Hkv = k.shape[1]
    S = min(sink_size, L)
    dk = torch.zeros((1, Hkv, S, D), dtype=torch.float64, device=q.device)
    dv = torch.zeros_like(dk)
    ds = None if sinks is None else torch.zeros(Hq, dtype=torch.float64, device=q.device)
    ds_terms = None if sinks is None else torch.zeros(Hq, dtype=torch.float64, device=q.device)
    for r0 in range(0, L, row_chunk):
        r1 = min(L, r0 + row_chunk)
        t0 = r0 - window_size + 1
        if t0 <= S:
            idx = torch.arange(r1, device=q.device)
        else:
            idx = torch.cat([torch.arange(S, device=q.device), torch.arange(t0, r1, device=q.device)])
        sub = lambda t: t.index_select(2, idx)
        keep = ((idx >= r0) & (idx < r1)).view(1, 1, -1, 1)
        dos = torch.where(keep, sub(do), torch.zeros((), dtype=do.dtype, device=do.device))
        if sinks is None:
            r = attention_fwd_bwd(sub(q), sub(k), sub(v), dos, window_size, sink_size, scale, compute_dtype)
        else:
            r = attention_fwd_bwd_sinks(sub(q), sub(k), sub(v), sinks, dos, window_size, sink_size, scale,
                                        compute_dtype)
            ds += r[5].double()
            rows = keep.view(-1)
            delta = (dos[0][:, rows].to(compute_dtype) * r[0][0][:, rows]).sum(-1)
            p_sink = torch.exp(sinks.to(compute_dtype).view(-1, 1) - r[1][0][:, rows])
            ds_terms += (p_sink * delta).abs().sum(-1).double()
        dk += r[3][:, :, :S].double()
        dv += r[4][:, :, :S].double()
    return dk, dv, ds, ds_terms


@torch.no_grad()
def naive_lowp_sink_key_grads(q, k, v, do, window_size: int, sink_size: int, scale: Optional[float] = None,
                              row_chunk: int = 2048):
    """dK/dV of the positional sink keys [0, S) as the reference's naive path computes them in the
    inputs' 16-bit dtype (naive_attention plus autograd; benchmark_backward_speed.py:68-85), for
    one long sequence ([1, H, L, D] tensors), banded as sink_key_grads is.  The naive path's
    rounding points are kept: scores = dt(dt(q k^T) * scale), P = softmax in float32 rounded to dt,
    grad P = dt(dO V^T), grad scores = dt(float32 softmax backward), times scale in dt; each head's
    dk = dt(grad_scores^T q) and dv = dt(P^T dO) over all of the sequence's rows, then the sum over
    the KV group's heads rounded to dt once.  Products run in float32 on the 16-bit values (exact
    products, float32 sums, as the 16-bit GEMMs accumulate), so no 16-bit batched product runs on
    the GPU.  Returns (dk, dv) [1, Hkv, S, D] as float32 holding dt values."""
    dt = q.dtype
    rnd = lambda x: x.to(dt).float()
    _, Hq, L, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    S = min(sink_size, L)
    acc_k = torch.zeros((Hq, S, D), dtype=torch.float32, device=q.device)
    acc_v = torch.zeros_like(acc_k)
    for r0 in range(0, L, row_chunk):
        r1 = min(L, r0 + row_chunk)
        t0 = r0 - window_size + 1
        if t0 <= S:
            idx = torch.arange(r1, device=q.device)
        else:
            idx = torch.cat([torch.arange(S, device=q.device), torch.arange(t0, r1, device=q.device)])
        n = idx.numel()
        sub = lambda t: t[0].index_select(1, idx).float()
        qs, ks, vs, dos = sub(q), sub(k), sub(v), sub(do)
        dos = torch.where(((idx >= r0) & (idx < r1)).view(1, -1, 1), dos, torch.zeros((), device=q.device))
        kr, vr = ks.repeat_interleave(G, dim=0), vs.repeat_interleave(G, dim=0)
        sc = rnd(rnd(torch.matmul(qs, kr.transpose(-1, -2).contiguous())) * scale)
        sc = sc.masked_fill(~allowed_mask(n, window_size, sink_size, device=q.device) if t0 <= S else
                            ~_sub_allowed(idx, window_size, sink_size), float("-inf"))
        p32 = torch.softmax(sc, dim=-1)
        pb = rnd(p32)
        gp = rnd(torch.matmul(dos, vr.transpose(-1, -2).contiguous()))
        gs = rnd(rnd(p32 * (gp - (gp * p32).sum(-1, keepdim=True))) * scale)
        acc_k += torch.matmul(gs[:, :, :S].transpose(-1, -2).contiguous(), qs)
        acc_v += torch.matmul(pb[:, :, :S].transpose(-1, -2).contiguous(), dos)
    dk = rnd(rnd(acc_k).view(Hkv, G, S, D).sum(1)).unsqueeze(0)
    dv = rnd(rnd(acc_v).view(Hkv, G, S, D).sum(1)).unsqueeze(0)
    return dk, dv


def _sub_allowed(idx, window_size, sink_size):
    """allowed_mask over the true positions `idx` of a sub-problem (rows and keys alike)."""
    qq, kk = idx.view(-1, 1), idx.view(1, -1)
    return (kk <= qq) & (((qq - kk) < window_size) | (kk < sink_size))


def gpt_oss_eager(q, k, v, sinks, window_size: Optional[int], scale: float):
    """The eager GPT-OSS attention of HF transformers (modeling_gpt_oss.py eager_attention_forward),
    restated on [B, H, L, D] tensors in their own dtype: repeated K/V, scaled scores plus the
    causal (and sliding, q - k < window) mask, the sink logit appended as one more column,
    softmax, the column dropped, P @ V.  Returns o [B, Hq, L, D]; autograd gives its backward."""
    group = q.shape[1] // k.shape[1]
    k = expand_kv(k, group)
    v = expand_kv(v, group)
    L = q.shape[2]
    scores = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scale
    keep = allowed_mask(L, L if window_size is None else window_size, 0, device=q.device)
    scores = scores.masked_fill(~keep, float("-inf"))
    col = sinks.to(scores.dtype).reshape(1, -1, 1, 1).expand(q.shape[0], -1, L, 1)
    logits = torch.cat([scores, col], dim=-1)
    logits = logits - logits.max(dim=-1, keepdim=True).values
    probs = torch.softmax(logits, dim=-1)[..., :-1]
    return torch.matmul(probs.to(v.dtype), v)


class OracleAttention(torch.autograd.Function):
    """attention_fwd_bwd behind autograd (float64 on CPU), so torch.autograd.gradcheck can
    compare its explicit backward with finite differences of its forward."""

    @staticmethod
    def forward(ctx, q, k, v, window_size, sink_size, scale):
        ctx.save_for_backward(q, k, v)
        ctx.cfg = (window_size, sink_size, scale)
        o, _, _, _, _ = attention_fwd_bwd(q, k, v, torch.zeros_like(q), window_size, sink_size, scale,
                                          compute_dtype=q.dtype)
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v = ctx.saved_tensors
        window_size, sink_size, scale = ctx.cfg
        _, _, dq, dk, dv = attention_fwd_bwd(q, k, v, do, window_size, sink_size, scale, compute_dtype=q.dtype)
        return dq, dk, dv, None, None, None


class OracleAttentionSinks(torch.autograd.Function):
    """attention_fwd_bwd_sinks behind autograd (float64 on CPU), for gradcheck of the sink
    logits' gradient as well as dq, dk, dv."""

    @staticmethod
    def forward(ctx, q, k, v, sinks, window_size, sink_size, scale):
        ctx.save_for_backward(q, k, v, sinks)
        ctx.cfg = (window_size, sink_size, scale)
        return attention_fwd_bwd_sinks(q, k, v, sinks, torch.zeros_like(q), window_size, sink_size, scale,
                                       compute_dtype=q.dtype)[0]

    @staticmethod
    def backward(ctx, do):
        q, k, v, sinks = ctx.saved_tensors
        window_size, sink_size, scale = ctx.cfg
        _, _, dq, dk, dv, ds = attention_fwd_bwd_sinks(q, k, v, sinks, do, window_size, sink_size, scale,
                                                        compute_dtype=q.dtype)
        return dq, dk, dv, ds, None, None, None


@torch.no_grad()
def attention_fwd_bwd_varlen(q, k, v, do, cu_seqlens, window_size: int, sink_size: int, scale: Optional[float] = None,
                             sinks=None, compute_dtype=torch.float32, row_chunk: Optional[int] = None):
    """Variable-length batches: packed q/do [total, Hq, D], k/v [total, Hkv, D]; sequence b is
    rows [cu_seqlens[b], cu_seqlens[b + 1]) and is an independent instance of
    attention_fwd_bwd (or attention_fwd_bwd_sinks with `sinks`).  Returns (o [total, Hq, D],
    lse [Hq, total], dq, dk, dv) and, with sinks, dsinks summed over the sequences."""
    total, Hq, D = q.shape
    Hkv = k.shape[1]
    o = torch.zeros((total, Hq, D), dtype=compute_dtype, device=q.device)
    lse = torch.full((Hq, total), float("-inf"), dtype=compute_dtype, device=q.device)
    dq = torch.zeros((total, Hq, D), dtype=compute_dtype, device=q.device)
    dk = torch.zeros((total, Hkv, D), dtype=compute_dtype, device=q.device)
    dv = torch.zeros((total, Hkv, D), dtype=compute_dtype, device=q.device)
    dsinks = None if sinks is None else torch.zeros(Hq, dtype=compute_dtype, device=q.device)
    cu = [int(x) for x in cu_seqlens.tolist()]
    as4 = lambda t, lo, hi: t[lo:hi].permute(1, 0, 2).unsqueeze(0)  # [1, H, L_b, D]
    for lo, hi in zip(cu[:-1], cu[1:]):
        if hi <= lo:
            continue
        args = (as4(q, lo, hi), as4(k, lo, hi), as4(v, lo, hi))
        if sinks is None:
            r = attention_fwd_bwd(*args, as4(do, lo, hi), window_size, sink_size, scale, compute_dtype, row_chunk)
        else:
            r = attention_fwd_bwd_sinks(*args, sinks, as4(do, lo, hi), window_size, sink_size, scale, compute_dtype,
                                        row_chunk)
            dsinks += r[5]
        o[lo:hi] = r[0][0].permute(1, 0, 2)
        lse[:, lo:hi] = r[1][0]
        dq[lo:hi] = r[2][0].permute(1, 0, 2)
        dk[lo:hi] = r[3][0].permute(1, 0, 2)
        dv[lo:hi] = r[4][0].permute(1, 0, 2)
    if sinks is None:
        return o, lse, dq, dk, dv
    return o, lse, dq, dk, dv, dsinks


def packed_allowed_mask(cu_seqlens, window_size: int, sink_size: int, device=None) -> torch.Tensor:
    """[total, total] bool for a packed batch: row r may see column c when both lie in the same
    sequence and, with positions counted from that sequence's first row, allowed_mask holds."""
    cu = [int(x) for x in cu_seqlens.tolist()]
    total = cu[-1]
    seq = torch.empty(total, dtype=torch.long, device=device)
    start = torch.empty(total, dtype=torch.long, device=device)
    for b, (lo, hi) in enumerate(zip(cu[:-1], cu[1:])):
        seq[lo:hi] = b
        start[lo:hi] = lo
    pos = torch.arange(total, device=device) - start
    qq, kk = pos.view(-1, 1), pos.view(1, -1)
    same = seq.view(-1, 1) == seq.view(1, -1)
    return same & (kk <= qq) & (((qq - kk) < window_size) | (kk < sink_size))
