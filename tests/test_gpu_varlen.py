"""GPU parity of variable-length (packed) batches: fa_fwd_varlen / fa_bwd_varlen against the
float32 variable-length oracle on the same seeded inputs.

Same bar as tests/test_gpu_parity.py: elementwise |ours - ref| <= a + 2e-2 |ref| with a = 2e-2,
except on the dK/dV rows of each sequence's positional sink keys, where
a = max(2e-2, 2 x the max error over those rows of the reference's naive path in the input dtype),
the naive path being run per sequence on the CPU (with learned sinks, the GPT-OSS eager path of
tests/test_gpu_sinks.py).  The sink gradient uses that file's bound, which scales with the sum
over rows of |P_sink * delta|.  Cases mix long, short, length-1 and empty sequences,
both sink paths (S <= 16 in the dQ kernel, S > 16 in chunk workgroups), learned sinks, full
causal attention and D in {16, 32, 64, 128}.
"""
import math

import pytest
import torch

from conftest import load_mod, load_pkg
from oracle import naive
from test_gpu_parity import assert_close
from test_gpu_sinks import check_dsinks, naive_sinks_reference

pytestmark = pytest.mark.gpu

BF, FP = torch.bfloat16, torch.float16


def packed_inputs(total, Hq, Hkv, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g).to(dtype).cuda()
    return mk(total, Hq, D), mk(total, Hkv, D), mk(total, Hkv, D), mk(total, Hq, D)


def naive_packed(q, k, v, do, cu, W, S, scale, sinks=None):
    """The reference's naive path in the input dtype, sequence by sequence on the CPU; with learned
    sinks, the GPT-OSS eager path, whose sink gradients are summed over the sequences."""
    outs = [torch.zeros_like(t, device="cpu") for t in (q, q, k, v)]
    dsinks = None if sinks is None else torch.zeros(q.shape[1])
    for lo, hi in zip(cu[:-1], cu[1:]):
        if hi <= lo:
            continue
        as4 = lambda t: t[lo:hi].detach().cpu().permute(1, 0, 2).unsqueeze(0).contiguous()
        if sinks is None:
            qc, kc, vc = (as4(t).requires_grad_() for t in (q, k, v))
            o = naive.naive_attention(qc, kc, vc, W, S, scale=scale)
            o.backward(as4(do))
            res = (o.detach(), qc.grad, kc.grad, vc.grad)
        else:
            res = naive_sinks_reference(as4(q), as4(k), as4(v), sinks, as4(do), W, S, scale)
            dsinks += res[4].float()
        for dst, src in zip(outs, res[:4]):
            dst[lo:hi] = src[0].permute(1, 0, 2)
    return (*outs, dsinks)


def run_varlen(cu, Hq, Hkv, D, W, S, dtype, seed=0, sinks=False, with_naive=True):
    ops = load_mod("_ops")
    print(f"case cu={cu} Hq={Hq} Hkv={Hkv} D={D} W={W} S={S} {dtype} sinks={sinks}", flush=True)
    total = cu[-1]
    q, k, v, do = packed_inputs(total, Hq, Hkv, D, dtype, seed)
    # sink logits exact in bf16, so the low-precision naive path sees them unrounded
    sk = (torch.randn(Hq, generator=torch.Generator().manual_seed(seed + 1)).to(torch.bfloat16).float().cuda()
          if sinks else None)
    scale = 1.0 / math.sqrt(D)
    cu_dev, max_len = ops.cu_seqlens_ready(torch.tensor(cu, dtype=torch.int32), total, q.device)
    Wk = max_len if W is None else W
    o, lse = ops.forward_varlen(q, k, v, cu_dev, max_len, Wk, S, scale, sinks=sk)
    grads = ops.backward_varlen(q, k, v, o, lse, do, cu_dev, max_len, Wk, S, scale, sinks=sk)
    torch.cuda.synchronize()
    ref = naive.attention_fwd_bwd_varlen(q, k, v, do, torch.tensor(cu), Wk, S, scale, sinks=sk,
                                         compute_dtype=torch.float32, row_chunk=1024)
    nv = naive_packed(q, k, v, do, cu, Wk, S, scale, sinks=sk) if with_naive and (S > 0 or sinks) else (None,) * 5
    # rows [cu[b], cu[b] + S) of each sequence hold its sink keys
    pos = torch.arange(total)
    wide = torch.zeros(total, dtype=torch.bool)
    for lo, hi in zip(cu[:-1], cu[1:]):
        wide |= (pos >= lo) & (pos < min(hi, lo + S))
    wide = wide.view(total, 1, 1)
    assert_close("O", o, ref[0])
    assert_close("LSE", lse, ref[1])
    assert_close("dQ", grads[0], ref[2])
    assert_close("dK", grads[1], ref[3], nv[2], wide)
    assert_close("dV", grads[2], ref[4], nv[3], wide)
    if sinks:
        as_b1 = lambda t: t.permute(1, 0, 2).unsqueeze(0)
        check_dsinks(grads[3], ref[5], ref[1].unsqueeze(0), as_b1(ref[0]), as_b1(do), sk, range(Hq), nv[4])
    return o, lse, grads


@pytest.mark.parametrize("cu,Hq,Hkv,D,W,S,dtype", [
    pytest.param([0, 300, 301, 1000, 1000, 1777], 8, 1, 64, 128, 4, BF, id="dq-sinks-mixed-lengths"),
    pytest.param([0, 700, 1500], 4, 2, 64, 64, 40, FP, id="sink-chunks"),
    pytest.param([0, 130, 900], 8, 2, 128, 100, 0, BF, id="D128-G4"),
    pytest.param([0, 33, 97, 600], 4, 4, 16, 40, 16, FP, id="D16-G1"),
    pytest.param([0, 500, 1200], 4, 1, 32, None, 0, BF, id="full-causal-D32"),
    pytest.param([0, 64, 128, 192, 256], 16, 2, 64, 32, 4, BF, id="equal-lengths"),
    pytest.param([0, 0, 1, 1, 2], 2, 1, 64, 8, 1, FP, id="tiny-and-empty"),
    pytest.param([0, 2048, 4096], 64, 8, 64, 128, 4, BF, id="gpt-oss-shape-two-sequences"),
    # short sequences beside long ones on the sliding kernels, whose units are sized by the rows
    # the batch holds (not by B x the longest sequence): sink rows in the dQ kernel, then in
    # chunk workgroups
    pytest.param([0, 4096, 6144, 7168, 7680, 10680, 12180, 12880, 16384], 64, 8, 64, 128, 4, BF,
                 id="gpt-oss-eight-mixed-lengths"),
    pytest.param([0, 4096, 6144, 7168, 7680, 10680, 12180, 12880, 16384], 64, 8, 64, 100, 24, FP,
                 id="gpt-oss-eight-mixed-lengths-S24"),
])
def test_varlen_parity(gpu, cu, Hq, Hkv, D, W, S, dtype):
    run_varlen(cu, Hq, Hkv, D, W, S, dtype, seed=cu[-1] % 97 + D, with_naive=cu[-1] * Hq <= 1 << 16)


def _many_sequences(n, seed, max_len):
    import random

    rng = random.Random(seed)
    lens = [rng.choice([0, 1, rng.randint(2, 40), rng.randint(41, max_len)]) for _ in range(n)]
    return [0] + list(__import__("itertools").accumulate(lens))


@pytest.mark.parametrize("cu,Hq,Hkv,D,W,S,dtype", [
    # more sequences than a wave's 64 lanes: the kernels' enumeration of the pieces the batch holds
    # (a prefix sum over the sequences, 64 per round) runs several rounds; empty and one-row
    # sequences on the sliding kernels (sink rows in the dQ kernel) and on the 64-key dK/dV kernel
    pytest.param(_many_sequences(150, 7, 300), 8, 1, 64, 128, 4, BF, id="150-sequences-sliding"),
    pytest.param(_many_sequences(130, 8, 200), 8, 1, 64, 48, 20, FP, id="130-sequences-sink-chunks"),
    pytest.param(_many_sequences(70, 9, 500), 16, 2, 64, 160, 0, BF, id="70-sequences-G8-W160"),
])
def test_varlen_many_sequences(gpu, cu, Hq, Hkv, D, W, S, dtype):
    run_varlen(cu, Hq, Hkv, D, W, S, dtype, seed=len(cu), with_naive=cu[-1] * Hq <= 1 << 16)


def _random_varlen_cases(n=12, seed=777):
    """Packed batches drawn from a fixed seed: 1-6 sequences of 0-500 rows each (empty ones
    included), every head dim, groups 1-8, windows from 1 to full causal, 0-40 positional sinks,
    learned sinks on some."""
    import random

    rng = random.Random(seed)
    cases = []
    for i in range(n):
        lens = [rng.choice([0, rng.randint(1, 40), rng.randint(41, 500)]) for _ in range(rng.randint(1, 6))]
        if sum(lens) == 0:
            lens[0] = 17
        cu = [0]
        for x in lens:
            cu.append(cu[-1] + x)
        D = rng.choice([16, 32, 64, 128])
        Hkv, G = rng.choice([1, 2, 4]), rng.choice([1, 2, 3, 8])
        W = rng.choice([1, rng.randint(2, 150), None])
        S = rng.choice([0, rng.randint(1, 40)])
        sinks = rng.random() < 0.4
        dtype = rng.choice([BF, FP])
        cases.append(pytest.param(cu, Hkv * G, Hkv, D, W, S, dtype, sinks, i,
                                  id=f"RV{i}-n{len(lens)}-T{cu[-1]}-H{Hkv * G}x{Hkv}-D{D}-W{W}-S{S}"
                                     f"{'-sinks' if sinks else ''}"))
    return cases


@pytest.mark.parametrize("cu,Hq,Hkv,D,W,S,dtype,sinks,seed", _random_varlen_cases())
def test_varlen_random_batches(gpu, cu, Hq, Hkv, D, W, S, dtype, sinks, seed):
    run_varlen(cu, Hq, Hkv, D, W, S, dtype, seed=300 + seed, sinks=sinks, with_naive=cu[-1] * Hq <= 1 << 16)


@pytest.mark.parametrize("cu,Hq,Hkv,D,W,S,seed", [
    pytest.param([0, 250, 700, 701], 8, 1, 64, 128, 0, 11, id="gpt-oss-sliding"),
    # W = 1 (each row sees itself and the sink column): dsinks sums p (1 - p) dO.v over 355 rows
    pytest.param([0, 5, 7, 12, 12, 64, 355], 4, 2, 64, 1, 0, 2104, id="W1-short-sequences"),
    # 7 positional sink keys each summing dS Q over 16 heads x 363 rows: the bf16 rounding of dS
    # puts up to 0.05 on them, inside the naive path's own error (0.10)
    pytest.param([0, 0, 363, 363, 363, 374], 32, 2, 16, 1, 7, 2114, id="W1-S7-G16-leading-empty"),
])
def test_varlen_learned_sinks(gpu, cu, Hq, Hkv, D, W, S, seed):
    run_varlen(cu, Hq, Hkv, D, W, S, BF, seed=seed, sinks=True)


def test_varlen_matches_separate_fixed_length_calls(gpu):
    """Each packed sequence gets exactly what a fixed-length call on it alone gets: O, LSE and
    dQ bitwise; dK/dV to rounding (their sink rows are summed in a different grouping)."""
    ops = load_mod("_ops")
    cu = [0, 200, 650, 651, 1100]
    Hq, Hkv, D, W, S = 8, 1, 64, 64, 4
    q, k, v, do = packed_inputs(cu[-1], Hq, Hkv, D, BF, seed=3)
    cu_dev, max_len = ops.cu_seqlens_ready(torch.tensor(cu), cu[-1], q.device)
    o, lse = ops.forward_varlen(q, k, v, cu_dev, max_len, W, S, 0.125)
    dq, dk, dv = ops.backward_varlen(q, k, v, o, lse, do, cu_dev, max_len, W, S, 0.125)
    for lo, hi in zip(cu[:-1], cu[1:]):
        as4 = lambda t: t[lo:hi].permute(1, 0, 2).unsqueeze(0)
        o1, lse1 = ops.forward(as4(q), as4(k), as4(v), W, S, 0.125)
        dq1, dk1, dv1 = ops.backward(as4(q), as4(k), as4(v), o1, lse1, as4(do), W, S, 0.125)
        assert torch.equal(as4(o), o1)
        assert torch.equal(lse[:, lo:hi], lse1[0])
        assert torch.equal(as4(dq), dq1)
        assert torch.allclose(as4(dk).float(), dk1.float(), atol=2e-2, rtol=1e-2)
        assert torch.allclose(as4(dv).float(), dv1.float(), atol=2e-2, rtol=1e-2)


def test_varlen_autograd_api_and_determinism(gpu):
    fa = load_pkg()
    cu = torch.tensor([0, 300, 301, 900], dtype=torch.int32)
    q, k, v, do = packed_inputs(900, 8, 2, 64, BF, seed=4)
    runs = []
    for cu_arg, max_len in ((cu, None), (cu.cuda(), 600)):
        qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
        o = fa.flash_swda_with_sink_varlen(qg, kg, vg, cu_arg, max_len, 128, 4)
        o.backward(do)
        runs.append((o.detach(), qg.grad, kg.grad, vg.grad))
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    ops = load_mod("_ops")
    ref = ops.forward_varlen(q, k, v, cu.cuda(), 600, 128, 4, 1 / 8)[0]
    assert torch.equal(runs[0][0], ref)


def test_varlen_argument_errors(gpu):
    fa = load_pkg()
    q, k, v, _ = packed_inputs(100, 4, 2, 64, BF, seed=1)
    with pytest.raises(ValueError, match="non-decreasing"):
        fa.flash_swda_with_sink_varlen(q, k, v, torch.tensor([0, 60, 50, 100]), None, 16, 1)
    with pytest.raises(ValueError, match="number of packed rows"):
        fa.flash_swda_with_sink_varlen(q, k, v, torch.tensor([0, 60, 120]), None, 16, 1)
    with pytest.raises(ValueError, match="max_seqlen is required"):
        fa.flash_swda_with_sink_varlen(q, k, v, torch.tensor([0, 100], dtype=torch.int32).cuda(), None, 16, 1)
    with pytest.raises(ValueError, match="below the longest"):
        fa.flash_swda_with_sink_varlen(q, k, v, torch.tensor([0, 100]), 50, 16, 1)


@pytest.mark.parametrize("cu,total", [
    pytest.param([0, 300, 700], 900, id="trailing-rows"),
    pytest.param([100, 400, 800], 900, id="leading-and-trailing-rows"),
    pytest.param([0, 500], 500, id="all-rows-covered"),
])
def test_varlen_rows_outside_every_sequence(gpu, cu, total):
    """Packed rows that belong to no sequence ([0, cu[0]) and [cu[B], total)) come back as o = 0,
    lse = -inf and zero gradients -- not whatever the allocator held (the memory is filled with
    NaN first).  Rows inside the sequences equal a call on exactly those rows, bit for bit."""
    ops = load_mod("_ops")
    Hq, Hkv, D, W, S = 8, 2, 64, 64, 4
    print(f"case cu={cu} total={total}", flush=True)
    q, k, v, do = packed_inputs(total, Hq, Hkv, D, BF, seed=21)
    junk = torch.full((1 << 24,), float("nan"), device=q.device)  # dirty the caching allocator's blocks
    del junk
    cu_dev = torch.tensor(cu, dtype=torch.int32, device=q.device)  # device offsets: used as given
    max_len = max(b - a for a, b in zip(cu[:-1], cu[1:]))
    o, lse = ops.forward_varlen(q, k, v, cu_dev, max_len, W, S, 0.125)
    dq, dk, dv = ops.backward_varlen(q, k, v, o, lse, do, cu_dev, max_len, W, S, 0.125)
    torch.cuda.synchronize()
    lo, hi = cu[0], cu[-1]
    outside = torch.ones(total, dtype=torch.bool)
    outside[lo:hi] = False
    for name, t in (("o", o), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert bool((t[outside.cuda()] == 0).all()), name
    assert bool((lse[:, outside.cuda()] == float("-inf")).all())
    # the covered rows: the same call on the rows [lo, hi) alone, offsets shifted to start at 0
    cu2 = torch.tensor([c - lo for c in cu], dtype=torch.int32, device=q.device)
    sl = lambda t: t[lo:hi].contiguous()
    o2, lse2 = ops.forward_varlen(sl(q), sl(k), sl(v), cu2, max_len, W, S, 0.125)
    dq2, dk2, dv2 = ops.backward_varlen(sl(q), sl(k), sl(v), o2, lse2, sl(do), cu2, max_len, W, S, 0.125)
    assert torch.equal(o[lo:hi], o2) and torch.equal(lse[:, lo:hi], lse2)
    assert torch.equal(dq[lo:hi], dq2) and torch.equal(dk[lo:hi], dk2) and torch.equal(dv[lo:hi], dv2)
