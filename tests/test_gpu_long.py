"""GPU parity at GPT-OSS's 128K context with tensors past 2^32 bytes.

B = 5, Hq = 64, Hkv = 8, L = 131072, D = 64, bf16: q, o, dO and dQ are 5.4 GB each, so the
(batch, head) slices of the last batches start past 2^31 and 2^32 bytes, where a 32-bit base
offset would wrap.  Two configurations cover both kernel families: the sliding kernels
(W = 128, S = 4, sink rows in the dQ kernel) and the generic ones (W = 300, S = 40, sink keys
in chunk workgroups and the fold).  The sliding one runs again in the [B, L, H, D] layout, where
one head's slice spans 1 GB, and once more as GPT-OSS runs it: learned sink logits and S = 0.

The float32 oracle cannot run the whole problem, so each sample of 64 rows [r0, r0 + 64) of one
sequence is checked against the oracle on a sub-problem: the S sink keys followed by positions
[t0, r0 + 64), t0 = r0 - W - 64.  Differences of positions inside the tail are kept and the sinks
stay the first S keys, so the sampled rows see exactly the keys they see in the full sequence
(every key they can reach lies at or past r0 - W + 1 > t0).  Their O, LSE and dQ must therefore
agree; at the end of a sequence (r0 = L - 64) every row that reaches the last 64 keys is sampled,
so those keys' dK and dV must agree too.  Every head is checked, at test_gpu_parity.py's bar.

The gradients that sum over every row of a sequence -- dK/dV of the positional sink keys, which
every row sees, and the learned sinks' gradient -- are checked over every row of every sequence:
naive.sink_key_grads runs the oracle over 2048-row chunks, each on a sub-problem in which the
chunk's rows see exactly their keys and the other rows' dO is zero.  dK/dV rows of sink keys sum
G x L (about a million) rounded terms each, so they get test_gpu_parity.py's bar for sink-key rows:
a = max(2e-2, 2 x the error of the reference's naive 16-bit path), that path's sink-key gradients
computed banded in the same way with its rounding points kept (naive.naive_lowp_sink_key_grads,
pinned against naive_attention's autograd backward on the CPU).  dsinks has test_gpu_sinks.py's
bound, 2e-2 (1 + sum |P_sink delta|).
"""
import math

import pytest
import torch

from conftest import load_mod
from oracle import naive
from test_gpu_parity import assert_close

pytestmark = pytest.mark.gpu

B, HQ, HKV, L, D = 5, 64, 8, 131072, 64


def subproblem_keys(r0, W, S):
    """Positions of the sub-problem for rows [r0, r0 + 64): the S sinks, then [r0 - W - 64, r0 + 64)."""
    t0 = r0 - W - 64
    assert t0 >= S
    return torch.cat([torch.arange(S), torch.arange(t0, r0 + 64)])


def check_sink_key_grads(tag, q, k, v, do, dk, dv, W, S, scale, sinks=None):
    """dK/dV rows [0, S) of one sequence ([1, H, L, D] views; dk, dv the kernel's [1, Hkv, S, D] rows)
    against naive.sink_key_grads over all of its rows; returns that function's (dsinks, terms)."""
    rdk, rdv, rds, terms = naive.sink_key_grads(q, k, v, do, W, S, scale, sinks=sinks, row_chunk=2048)
    if S > 0:
        ndk, ndv = naive.naive_lowp_sink_key_grads(q, k, v, do, W, S, scale, row_chunk=2048)
        every = torch.ones((1, 1, 1, 1), dtype=torch.bool)
        assert_close(f"dK sink keys {tag}", dk, rdk, ndk, every)
        assert_close(f"dV sink keys {tag}", dv, rdv, ndv, every)
    return rds, terms


def check_dsinks_sum(got, ref, terms):
    """dsinks summed over every row of every sequence, at 2e-2 (1 + sum |P_sink delta|) per head."""
    err = (got.double() - ref).abs()
    bound = 2e-2 * (1.0 + terms)
    print(f"  dsinks: max abs err {float(err.max()):.3e}, largest err / bound {float((err / bound).max()):.3f}")
    assert bool((err <= bound).all()), f"dsinks: err {err.tolist()} bound {bound.tolist()}"


def _randn(B, H, seed, layout):
    """A [B, H, L, D] bf16 tensor, or a [B, H, L, D] view of a [B, L, H, D] one (GPT-OSS's layout:
    each head's rows are H * D elements apart, so a head's slice spans 1 GB here)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    if layout == "blhd":
        return torch.randn((B, L, H, D), device="cuda", dtype=torch.bfloat16, generator=g).transpose(1, 2)
    return torch.randn((B, H, L, D), device="cuda", dtype=torch.bfloat16, generator=g)


@pytest.mark.parametrize("W,S,layout,learned", [
    pytest.param(128, 4, "bhld", False, id="sliding-kernels"),
    pytest.param(300, 40, "bhld", False, id="generic-kernels-sink-chunks"),
    pytest.param(128, 4, "blhd", False, id="sliding-kernels-BLHD-layout"),
    # GPT-OSS's sliding layer as its model runs it: learned sink logits, no positional sinks
    pytest.param(128, 0, "blhd", True, id="gpt-oss-learned-sinks-BLHD-layout"),
])
def test_long_context_past_4gb(gpu, W, S, layout, learned):
    ops = load_mod("_ops")
    print(f"case B={B} Hq={HQ} Hkv={HKV} L={L} D={D} W={W} S={S} bf16 {layout} learned={learned}", flush=True)
    q = _randn(B, HQ, 1, layout)
    k, v = _randn(B, HKV, 2, layout), _randn(B, HKV, 3, layout)
    do = _randn(B, HQ, 4, layout)
    assert q.numel() * q.element_size() > 1 << 32
    sc = 1.0 / math.sqrt(D)
    # learned sink logits exact in bf16, about the size of the scores
    sk = (2.0 * torch.randn(HQ, generator=torch.Generator().manual_seed(5))).to(torch.bfloat16).float().cuda() \
        if learned else None
    o, lse = ops.forward(q, k, v, W, S, sc, sinks=sk)
    grads = ops.backward(q, k, v, o, lse, do, W, S, sc, sinks=sk)
    dq, dk, dv = grads[:3]
    torch.cuda.synchronize()
    # the sums over every row: sink keys' dK/dV of every sequence, and dsinks over all of them
    ds_ref = torch.zeros(HQ, dtype=torch.float64, device="cuda")
    ds_terms = torch.zeros_like(ds_ref)
    for b in range(B):
        one = lambda t: t[b:b + 1]
        rds, terms = check_sink_key_grads(f"b={b}", one(q), one(k), one(v), one(do), dk[b:b + 1, :, :S],
                                          dv[b:b + 1, :, :S], W, S, sc, sinks=sk)
        if learned:
            ds_ref += rds
            ds_terms += terms
    if learned:
        check_dsinks_sum(grads[3], ds_ref, ds_terms)
    for b, r0 in ((B - 1, L - 64), (B - 1, L // 2 + 13), (3, 100000), (0, 4096)):
        idx = subproblem_keys(r0, W, S).cuda()
        sub = lambda t: t[b:b + 1].index_select(2, idx).contiguous()
        if learned:
            ro, rlse, rdq, rdk, rdv, _ = naive.attention_fwd_bwd_sinks(sub(q), sub(k), sub(v), sk, sub(do), W, S,
                                                                       scale=sc, compute_dtype=torch.float32)
        else:
            ro, rlse, rdq, rdk, rdv = naive.attention_fwd_bwd(sub(q), sub(k), sub(v), sub(do), W, S, scale=sc,
                                                              compute_dtype=torch.float32)
        n = idx.numel()
        rows = slice(r0, r0 + 64)
        tag = f"b={b} rows {r0}-{r0 + 63}"
        assert_close(f"O {tag}", o[b, :, rows], ro[0, :, n - 64:])
        assert_close(f"LSE {tag}", lse[b, :, rows], rlse[0, :, n - 64:])
        assert_close(f"dQ {tag}", dq[b, :, rows], rdq[0, :, n - 64:])
        if r0 + 64 == L:
            assert_close(f"dK {tag}", dk[b, :, rows], rdk[0, :, n - 64:])
            assert_close(f"dV {tag}", dv[b, :, rows], rdv[0, :, n - 64:])
    del q, k, v, do, o, lse, dq, dk, dv, grads
    torch.cuda.empty_cache()


def test_long_packed_batch(gpu):
    """A packed batch of 200000 rows: a 128K-row sequence, a 1-row one, then 8927 and 60000 rows,
    Hq = 64, Hkv = 8, D = 64, W = 128, S = 4, bf16.  Each head's slice spans the whole packed
    tensor (1.6 GB).  Sampled rows are checked on the same sub-problems, built from each
    sequence's own positions; the 1-row sequence is checked whole."""
    ops = load_mod("_ops")
    W, S = 128, 4
    cu = [0, 131072, 131073, 140000, 200000]
    total = cu[-1]
    print(f"case packed cu={cu} Hq={HQ} Hkv={HKV} D={D} W={W} S={S} bf16", flush=True)
    mk = lambda H, seed: torch.randn((total, H, D), device="cuda", dtype=torch.bfloat16,
                                     generator=torch.Generator(device="cuda").manual_seed(seed))
    q, k, v, do = mk(HQ, 11), mk(HKV, 12), mk(HKV, 13), mk(HQ, 14)
    sc = 1.0 / math.sqrt(D)
    cu_dev, max_len = ops.cu_seqlens_ready(torch.tensor(cu, dtype=torch.int32), total, q.device)
    o, lse = ops.forward_varlen(q, k, v, cu_dev, max_len, W, S, sc)
    dq, dk, dv = ops.backward_varlen(q, k, v, o, lse, do, cu_dev, max_len, W, S, sc)
    torch.cuda.synchronize()
    # the sink keys' dK/dV of each sequence, over all of its rows
    for s, (lo, hi) in enumerate(zip(cu[:-1], cu[1:])):
        as4 = lambda t: t[lo:hi].permute(1, 0, 2).unsqueeze(0)
        n_s = min(S, hi - lo)
        check_sink_key_grads(f"sequence {s}", as4(q), as4(k), as4(v), as4(do), as4(dk)[:, :, :n_s],
                             as4(dv)[:, :, :n_s], W, S, sc)
    # (sequence, first sampled row relative to its start; None: the whole sequence)
    for s, r0 in ((0, 131072 - 64), (0, 70001), (1, None), (2, 8927 - 64), (3, 33333)):
        lo, n_seq = cu[s], cu[s + 1] - cu[s]
        idx = torch.arange(n_seq) if r0 is None else subproblem_keys(r0, W, S)
        rel = slice(0, n_seq) if r0 is None else slice(r0, r0 + 64)
        rows = torch.arange(rel.start, rel.stop).cuda() + lo
        pos = idx.cuda() + lo
        sub = lambda t: t.index_select(0, pos).permute(1, 0, 2).unsqueeze(0).contiguous()
        ro, rlse, rdq, rdk, rdv = naive.attention_fwd_bwd(sub(q), sub(k), sub(v), sub(do), W, S, scale=sc,
                                                          compute_dtype=torch.float32)
        m = rel.stop - rel.start
        got = lambda t: t.index_select(0, rows).permute(1, 0, 2)
        tag = f"sequence {s} rows {rel.start}-{rel.stop - 1}"
        assert_close(f"O {tag}", got(o), ro[0, :, -m:])
        assert_close(f"LSE {tag}", lse.index_select(1, rows), rlse[0, :, -m:])
        assert_close(f"dQ {tag}", got(dq), rdq[0, :, -m:])
        if rel.stop == n_seq:
            assert_close(f"dK {tag}", got(dk), rdk[0, :, -m:])
            assert_close(f"dV {tag}", got(dv), rdv[0, :, -m:])
    del q, k, v, do, o, lse, dq, dk, dv
    torch.cuda.empty_cache()


@pytest.mark.parametrize("fp8_pv", [pytest.param(False, id="fa_fwd_fp8"), pytest.param(True, id="fa_fwd_fp8_pv")])
def test_long_fp8_forward_past_4gb(gpu, fp8_pv):
    """The fp8 forwards at 128K context with B = 9, so that the 1-byte q (4.8 GB) and the bf16 o
    (9.7 GB) both have slices past 2^32 bytes (W = 128, S = 4).  Sampled rows are checked on the
    sub-problems above with test_gpu_fp8.py's bars: the oracle on the dequantised inputs at the
    16-bit bar for fa_fwd_fp8, and the bound that rounding P to e4m3 allows for fa_fwd_fp8_pv."""
    from test_gpu_fp8 import assert_pv_close, pv_bound, reference

    ops = load_mod("_ops")
    Bf, W, S = 9, 128, 4
    print(f"case fp8 B={Bf} Hq={HQ} Hkv={HKV} L={L} D={D} W={W} S={S} fp8_pv={fp8_pv}", flush=True)
    mk = lambda H, seed: torch.randn((Bf, H, L, D), device="cuda", dtype=torch.bfloat16,
                                     generator=torch.Generator(device="cuda").manual_seed(seed)).to(torch.float8_e4m3fn)
    q8, k8, v8 = mk(HQ, 21), mk(HKV, 22), mk(HKV, 23)
    assert q8.numel() > 1 << 32
    ds = (0.5, 0.25, 1.0)  # q, k, v stand for ds[i] times their e4m3 values
    sc = 1.0 / math.sqrt(D)
    o, lse = ops.forward_fp8(q8, k8, v8, W, S, sc, ds, fp8_pv=fp8_pv)
    torch.cuda.synchronize()
    for b, r0 in ((Bf - 1, L - 64), (Bf - 1, 70001), (4, 100000), (0, 4096)):
        idx = subproblem_keys(r0, W, S).cuda()
        sub = lambda t: t[b:b + 1].view(torch.uint8).index_select(2, idx).contiguous().view(torch.float8_e4m3fn)
        qs, ks, vs = sub(q8), sub(k8), sub(v8)
        ro, rlse = reference(qs, ks, vs, ds, W, S, sc)
        got_o, got_lse = o[b:b + 1, :, r0:r0 + 64], lse[b:b + 1, :, r0:r0 + 64]
        if fp8_pv:
            bound, lse_bound = pv_bound(qs, ks, vs, ds, W, S, sc, ro)
            assert_pv_close(got_o, got_lse, ro[:, :, -64:], rlse[:, :, -64:], bound[:, :, -64:], lse_bound[:, :, -64:])
        else:
            assert_close(f"O b={b} rows {r0}-{r0 + 63}", got_o, ro[:, :, -64:])
            assert_close(f"LSE b={b} rows {r0}-{r0 + 63}", got_lse, rlse[:, :, -64:])
    del q8, k8, v8, o, lse
    torch.cuda.empty_cache()
