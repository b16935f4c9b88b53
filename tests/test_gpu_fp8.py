"""GPU parity of the FP8 forward (fa_fwd_fp8): e4m3 q, k, v with per-tensor dequantisation
factors, bf16 output.

The kernel computes Q K^T exactly on the stored e4m3 values (fp32 accumulation) and widens V to
bf16 exactly, so its result is the 16-bit forward's on the dequantised inputs descale * x8.  The
oracle is therefore the float32 naive path (naive.attention_fwd_bwd / attention_fwd_bwd_sinks)
evaluated on those dequantised inputs (torch's e4m3 decode, pinned against the OCP definition in
test_oracle_fp8.py), with the 16-bit tolerance of test_gpu_parity.py:
    |ours - ref| <= 2e-2 + 2e-2 * |ref|   on O and LSE.
The inputs are drawn as in the other parity tests (seeded N(0, 1) on the CPU) and quantised with
quantize_fp8 (amax / 448 per tensor).  A second check runs the bf16 kernel on the same
dequantised values where they are exact in bf16 (power-of-two factors).  The two forwards then
differ only in how Q K^T is summed: the fp8 matrix instruction adds its 64 products at reduced
internal precision (an in-bounds probe of one 32x32x64 product measured errors of about 3e-5 of
the result's magnitude, against about 1e-7 for fp32 sums), which moves scores of magnitude ~30
by ~1e-3, so that check's bound is 1e-2 on LSE and 1e-2 + 1e-2 |O| on O -- tighter than the
oracle bar.

fa_fwd_fp8_pv (P V on the fp8 matrix cores as well) rounds the softmax weights to e4m3; its tests,
at the end of this file, check the error bound that rounding allows (derived there) on the same
cases, against the same oracle.
"""
import math

import pytest
import torch

from conftest import load_mod, load_pkg
from oracle import naive
from test_gpu_parity import assert_close

pytestmark = pytest.mark.gpu


def fp8_inputs(B, Hq, Hkv, L, D, seed, std=1.0, descale=None):
    fa = load_pkg()
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, L, D, generator=g) * std
    k = torch.randn(B, Hkv, L, D, generator=g) * std
    v = torch.randn(B, Hkv, L, D, generator=g) * std
    out = []
    for t in (q, k, v):
        x8, d = fa.quantize_fp8(t, descale)
        out.append((x8.cuda(), d))
    return out


def reference(q8, k8, v8, ds, W, S, scale, sinks=None):
    qf, kf, vf = (x.float() * d for x, d in zip((q8, k8, v8), ds))
    do = torch.zeros_like(qf)
    if sinks is None:
        ro, rlse = naive.attention_fwd_bwd(qf, kf, vf, do, W, S, scale=scale, compute_dtype=torch.float32)[:2]
    else:
        ro, rlse = naive.attention_fwd_bwd_sinks(qf, kf, vf, sinks, do, W, S, scale=scale,
                                                 compute_dtype=torch.float32)[:2]
    return ro, rlse


CASES = [
    # B, Hq, Hkv, L, D, W, S
    (1, 8, 2, 300, 64, 64, 4),
    (2, 4, 4, 257, 128, 32, 0),
    (1, 16, 8, 700, 64, 700, 0),   # full causal
    (1, 8, 8, 129, 128, 128, 16),
    (1, 6, 2, 200, 64, 50, 3),     # group of 3: one head per wave
    (1, 8, 1, 65, 64, 1, 1),       # window 1 and one sink key
    (1, 4, 2, 33, 128, 33, 40),    # sinks cover the whole sequence
    (1, 64, 8, 1024, 64, 128, 4),  # the GPT-OSS sliding layer shape
]


@pytest.mark.parametrize("case", CASES, ids=[f"B{c[0]}-H{c[1]}x{c[2]}-L{c[3]}-D{c[4]}-W{c[5]}-S{c[6]}" for c in CASES])
def test_fp8_forward_parity(gpu, case):
    B, Hq, Hkv, L, D, W, S = case
    ops = load_mod("_ops")
    (q8, qd), (k8, kd), (v8, vd) = fp8_inputs(B, Hq, Hkv, L, D, seed=L)
    sc = 1.0 / math.sqrt(D)
    print(f"fp8 case {case}", flush=True)
    o, lse = ops.forward_fp8(q8, k8, v8, W, S, sc, (qd, kd, vd))
    torch.cuda.synchronize()
    assert o.dtype == torch.bfloat16 and lse.dtype == torch.float32
    ro, rlse = reference(q8, k8, v8, (qd, kd, vd), W, S, sc)
    assert_close("O", o, ro)
    assert_close("LSE", lse, rlse)


def test_fp8_matches_the_bf16_kernel_on_exact_inputs(gpu):
    """Power-of-two factors make every dequantised value a bf16 value: the bf16 forward on those
    values and the fp8 forward differ only in how Q K^T is summed (see the module docstring)."""
    ops = load_mod("_ops")
    B, Hq, Hkv, L, D, W, S = 1, 16, 2, 600, 64, 128, 4
    (q8, qd), (k8, kd), (v8, vd) = fp8_inputs(B, Hq, Hkv, L, D, seed=3, std=2.0, descale=1.0 / 64)
    sc = 1.0 / math.sqrt(D)
    o8, lse8 = ops.forward_fp8(q8, k8, v8, W, S, sc, (qd, kd, vd))
    qb, kb, vb = ((x.float() * d).to(torch.bfloat16) for x, d in ((q8, qd), (k8, kd), (v8, vd)))
    assert bool(((qb.float() / qd).to(torch.float8_e4m3fn).view(torch.uint8) == q8.view(torch.uint8)).all())
    o16, lse16 = ops.forward(qb, kb, vb, W, S, sc)
    torch.cuda.synchronize()
    assert float((lse8 - lse16).abs().max()) < 1e-2
    # O: the score differences flip some bf16 roundings of P and O (one ulp = 2^-8 |O|)
    err = (o8.float() - o16.float()).abs()
    assert bool((err <= 1e-2 + 1e-2 * o16.float().abs()).all()), float(err.max())


@pytest.mark.parametrize("D", [64, 128])
def test_fp8_learned_sinks_and_negative_scale(gpu, D):
    ops = load_mod("_ops")
    B, Hq, Hkv, L, W, S = 1, 8, 2, 333, 100, 4
    (q8, qd), (k8, kd), (v8, vd) = fp8_inputs(B, Hq, Hkv, L, D, seed=D)
    g = torch.Generator().manual_seed(7)
    sinks = (2.0 * torch.randn(Hq, generator=g)).cuda()
    sc = -0.7 / math.sqrt(D)
    o, lse = ops.forward_fp8(q8, k8, v8, W, S, sc, (qd, kd, vd), sinks)
    torch.cuda.synchronize()
    ro, rlse = reference(q8, k8, v8, (qd, kd, vd), W, S, sc, sinks)
    assert_close("O", o, ro)
    assert_close("LSE", lse, rlse)


def test_fp8_blhd_layout_and_determinism(gpu):
    """[B, L, H, D] buffers viewed as [B, H, L, D] give bitwise the contiguous result; reruns are
    bitwise identical."""
    ops = load_mod("_ops")
    B, Hq, Hkv, L, D, W, S = 2, 8, 4, 160, 64, 64, 2
    (q8, qd), (k8, kd), (v8, vd) = fp8_inputs(B, Hq, Hkv, L, D, seed=11)
    sc = 1.0 / math.sqrt(D)
    o1, l1 = ops.forward_fp8(q8, k8, v8, W, S, sc, (qd, kd, vd))
    o2, l2 = ops.forward_fp8(q8, k8, v8, W, S, sc, (qd, kd, vd))
    qt, kt, vt = (x.transpose(1, 2).contiguous().transpose(1, 2) for x in (q8, k8, v8))
    o3, l3 = ops.forward_fp8(qt, kt, vt, W, S, sc, (qd, kd, vd))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    assert torch.equal(o1, o3) and torch.equal(l1, l3)
    assert o3.stride() == qt.stride()


def test_fp8_public_api_and_errors(gpu):
    fa = load_pkg()
    (q8, qd), (k8, kd), (v8, vd) = fp8_inputs(1, 4, 2, 64, 64, seed=5)
    o = fa.flash_swda_with_sink_fp8(q8, k8, v8, None, 0, descale=(qd, kd, vd))
    ro, _ = reference(q8, k8, v8, (qd, kd, vd), 64, 0, 1.0 / 8.0)
    assert_close("O", o, ro)
    with pytest.raises(ValueError, match="head_dim"):
        (a8, _), (b8, _), (c8, _) = fp8_inputs(1, 4, 2, 64, 32, seed=5)
        fa.flash_swda_with_sink_fp8(a8, b8, c8, 16, 0)
    with pytest.raises(ValueError, match="float8_e4m3fn"):
        fa.flash_swda_with_sink_fp8(q8.float().to(torch.bfloat16), k8, v8, 16, 0)
    with pytest.raises(AssertionError, match="Key and Value shapes must be the same"):
        fa.flash_swda_with_sink_fp8(q8, k8, v8[:, :1], 16, 0)


# ---- fa_fwd_fp8_pv: P V on the fp8 matrix cores as well --------------------------------------
#
# The kernel rounds the softmax weights P (scaled so that the largest of a row is >= 16) to e4m3
# before the product and divides by the sum of the rounded weights, so with p the exact
# normalised weights and O the oracle's output,
#     O_pv - O = sum_k (P~_k - P_k)(v_k - O) / sum_k P~_k.
# e4m3 rounding moves a weight >= 2^-6 by at most 2^-4 of itself and a smaller one by at most
# 2^-10 (half the subnormal spacing 2^-9); sum P~ >= (1 - 2^-4) sum P and sum P >= 16.  Hence
#     |O_pv - O| <= 2^-4 / (1 - 2^-4) * sum_k p_k |v_k - O| + n * 2^-14 * max_k |v_k - O|
# over the n allowed keys of the row; sum_k p_k |v_k - O| <= p @ |v| + |O| and
# max_k |v_k - O| <= max_k |v_k| + |O| make both terms cheap to evaluate.  The log-sum-exp moves
# by at most -ln(1 - 2^-4) + n 2^-14 / 16.  On top of those, the test keeps the 16-bit bar
# (2e-2 + 2e-2 |ref|) for the Q K^T sums and the bf16 output.  A wrong key or head-dim order in
# the product would move O by about the whole spread and fail the first term (0.07 of it).


def pv_bound(q8, k8, v8, ds, W, S, scale, ro, sinks=None):
    qf, kf, vf = (x.float().cpu() * d for x, d in zip((q8, k8, v8), ds))
    B, Hq, L, D = qf.shape
    g = Hq // kf.shape[1]
    kf, vf = naive.expand_kv(kf, g), naive.expand_kv(vf, g)
    allowed = naive.allowed_mask(L, W, S)
    s = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * scale
    s = s.masked_fill(~allowed, float("-inf"))
    if sinks is not None:
        sl = sinks.float().cpu().view(1, Hq, 1, 1).expand(B, Hq, L, 1)
        p = torch.softmax(torch.cat([s, sl], dim=-1), dim=-1)[..., :L]
    else:
        p = torch.softmax(s, dim=-1)
    o = ro.float().cpu().abs()
    spread = torch.matmul(p, vf.abs()) + o
    n = allowed.sum(-1).view(1, 1, L, 1).float()
    vmax = vf.abs().amax(dim=2, keepdim=True)  # over all keys: an upper bound of the allowed ones
    bound = 0.07 * spread + n * 2.0 ** -14 * (vmax + o)
    lse_bound = 0.0645 + n[..., 0] * 2.0 ** -18
    return bound, lse_bound


def assert_pv_close(o, lse, ro, rlse, bound, lse_bound):
    err = (o.float().cpu() - ro.float().cpu()).abs()
    lim = bound + 2e-2 + 2e-2 * ro.float().cpu().abs()
    assert bool((err <= lim).all()), f"O: worst excess {float((err - lim).max()):.4g}, max err {float(err.max()):.4g}"
    lerr = (lse.float().cpu() - rlse.float().cpu()).abs()
    llim = lse_bound + 2e-2 + 2e-2 * rlse.float().cpu().abs()
    assert bool((lerr <= llim).all()), f"LSE: max err {float(lerr.max()):.4g}"
    # rounding errors of independent weights mostly cancel: the typical error stays far below the bound
    assert float(err.mean()) < 0.25 * float(lim.mean()), (float(err.mean()), float(lim.mean()))


@pytest.mark.parametrize("case", CASES, ids=[f"B{c[0]}-H{c[1]}x{c[2]}-L{c[3]}-D{c[4]}-W{c[5]}-S{c[6]}" for c in CASES])
def test_fp8_pv_forward_parity(gpu, case):
    B, Hq, Hkv, L, D, W, S = case
    ops = load_mod("_ops")
    (q8, qd), (k8, kd), (v8, vd) = fp8_inputs(B, Hq, Hkv, L, D, seed=L)
    sc = 1.0 / math.sqrt(D)
    print(f"fp8_pv case {case}", flush=True)
    o, lse = ops.forward_fp8(q8, k8, v8, W, S, sc, (qd, kd, vd), fp8_pv=True)
    torch.cuda.synchronize()
    assert o.dtype == torch.bfloat16 and lse.dtype == torch.float32
    ro, rlse = reference(q8, k8, v8, (qd, kd, vd), W, S, sc)
    bound, lse_bound = pv_bound(q8, k8, v8, (qd, kd, vd), W, S, sc, ro)
    assert_pv_close(o, lse, ro, rlse, bound, lse_bound)


def test_fp8_pv_single_key_rows_are_exact(gpu):
    """W = 1, S = 0: every row sees one key, whose rounded weight divides out, so O is that key's
    value row whatever the rounding of P -- up to one fp32 rounding of the normalisation, which can
    flip the bf16 rounding of O by one unit (2^-8 relative)."""
    ops = load_mod("_ops")
    B, Hq, Hkv, L, D = 1, 8, 2, 200, 128
    (q8, qd), (k8, kd), (v8, vd) = fp8_inputs(B, Hq, Hkv, L, D, seed=21)
    o, _ = ops.forward_fp8(q8, k8, v8, 1, 0, 1.0 / math.sqrt(D), (qd, kd, vd), fp8_pv=True)
    torch.cuda.synchronize()
    want = naive.expand_kv(v8.float() * vd, Hq // Hkv).to(torch.bfloat16).float()
    err = (o.float() - want).abs()
    assert bool((err <= 2.0 ** -8 * want.abs()).all()), float(err.max())


@pytest.mark.parametrize("D", [64, 128])
def test_fp8_pv_learned_sinks_and_negative_scale(gpu, D):
    ops = load_mod("_ops")
    B, Hq, Hkv, L, W, S = 1, 8, 2, 333, 100, 4
    (q8, qd), (k8, kd), (v8, vd) = fp8_inputs(B, Hq, Hkv, L, D, seed=D)
    g = torch.Generator().manual_seed(7)
    sinks = (2.0 * torch.randn(Hq, generator=g)).cuda()
    sc = -0.7 / math.sqrt(D)
    o, lse = ops.forward_fp8(q8, k8, v8, W, S, sc, (qd, kd, vd), sinks, fp8_pv=True)
    torch.cuda.synchronize()
    ro, rlse = reference(q8, k8, v8, (qd, kd, vd), W, S, sc, sinks)
    bound, lse_bound = pv_bound(q8, k8, v8, (qd, kd, vd), W, S, sc, ro, sinks)
    assert_pv_close(o, lse, ro, rlse, bound, lse_bound)


def test_fp8_pv_blhd_layout_determinism_and_api(gpu):
    fa = load_pkg()
    ops = load_mod("_ops")
    B, Hq, Hkv, L, D, W, S = 2, 8, 4, 160, 64, 64, 2
    (q8, qd), (k8, kd), (v8, vd) = fp8_inputs(B, Hq, Hkv, L, D, seed=11)
    sc = 1.0 / math.sqrt(D)
    o1, l1 = ops.forward_fp8(q8, k8, v8, W, S, sc, (qd, kd, vd), fp8_pv=True)
    o2, l2 = ops.forward_fp8(q8, k8, v8, W, S, sc, (qd, kd, vd), fp8_pv=True)
    qt, kt, vt = (x.transpose(1, 2).contiguous().transpose(1, 2) for x in (q8, k8, v8))
    o3, l3 = ops.forward_fp8(qt, kt, vt, W, S, sc, (qd, kd, vd), fp8_pv=True)
    o4 = fa.flash_swda_with_sink_fp8(q8, k8, v8, W, S, descale=(qd, kd, vd), fp8_pv=True)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    assert torch.equal(o1, o3) and torch.equal(l1, l3)
    assert torch.equal(o1, o4)


def _random_fp8_cases(n=10, seed=8080):
    """Shapes drawn from a fixed seed for both fp8 entry points: D 64 or 128, groups 1-8, lengths
    1-700, windows from 1 to past L, 0-40 positional sinks, learned sinks on some, input scales
    0.25-4 (so the per-tensor factors differ from 1), the softmax scale around 1/sqrt(D)."""
    import random

    rng = random.Random(seed)
    cases = []
    while len(cases) < n:
        D = rng.choice([64, 128])
        Hkv, G, B = rng.choice([1, 2, 4]), rng.choice([1, 2, 3, 8]), rng.choice([1, 2])
        L = rng.choice([rng.randint(1, 64), rng.randint(65, 700)])
        W = rng.choice([1, rng.randint(2, 200), L, L + 9])
        S = rng.choice([0, rng.randint(1, 40)])
        if B * Hkv * G * L * L > (1 << 23):
            continue
        cases.append(pytest.param(B, Hkv * G, Hkv, L, D, W, S, rng.random() < 0.3, rng.choice([0.25, 1.0, 4.0]),
                                  rng.uniform(0.6, 1.4) / math.sqrt(D), len(cases),
                                  id=f"RF{len(cases)}-B{B}-H{Hkv * G}x{Hkv}-L{L}-D{D}-W{W}-S{S}"))
    return cases


@pytest.mark.parametrize("B,Hq,Hkv,L,D,W,S,learned,std,sc,seed", _random_fp8_cases())
def test_fp8_random_shapes_both_entry_points(gpu, B, Hq, Hkv, L, D, W, S, learned, std, sc, seed):
    ops = load_mod("_ops")
    print(f"random fp8 case B={B} Hq={Hq} Hkv={Hkv} L={L} D={D} W={W} S={S} learned={learned} std={std}", flush=True)
    (q8, qd), (k8, kd), (v8, vd) = fp8_inputs(B, Hq, Hkv, L, D, seed=400 + seed, std=std)
    sinks = (2.0 * torch.randn(Hq, generator=torch.Generator().manual_seed(seed))).cuda() if learned else None
    o, lse = ops.forward_fp8(q8, k8, v8, W, S, sc, (qd, kd, vd), sinks)
    op, lp = ops.forward_fp8(q8, k8, v8, W, S, sc, (qd, kd, vd), sinks, fp8_pv=True)
    torch.cuda.synchronize()
    ro, rlse = reference(q8, k8, v8, (qd, kd, vd), W, S, sc, sinks)
    assert_close("O", o, ro)
    assert_close("LSE", lse, rlse)
    bound, lse_bound = pv_bound(q8, k8, v8, (qd, kd, vd), W, S, sc, ro, sinks)
    assert_pv_close(op, lp, ro, rlse, bound, lse_bound)
