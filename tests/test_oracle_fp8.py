"""CPU checks behind the FP8 forward's parity tests.

The GPU tests compare fa_fwd_fp8 with the float32 oracle evaluated on the dequantised inputs
descale * x8, where x8 is decoded by torch.float8_e4m3fn.  That decode is pinned here against
the OCP e4m3 definition (sign, 4 exponent bits with bias 7, 3 mantissa bits; exponent 0 is
subnormal, 0x7F / 0xFF are NaN, no infinities), written out in closed form, for all 256
encodings.  The host-side quantiser quantize_fp8 is checked for its rounding bound.  The error
bound that the fa_fwd_fp8_pv tests allow for rounding the softmax weights to e4m3 is checked
against an emulation of that rounding.  The C ABI's argument checks for the fp8 entry points are
in test_capi.py.
"""
import math

import pytest
import torch

from conftest import load_pkg


def e4m3_value(b: int) -> float:
    sign = -1.0 if b & 0x80 else 1.0
    e, m = (b >> 3) & 0xF, b & 0x7
    if e == 0xF and m == 0x7:
        return math.nan
    if e == 0:
        return sign * 2.0 ** -6 * (m / 8.0)
    return sign * 2.0 ** (e - 7) * (1.0 + m / 8.0)


def test_torch_e4m3_decode_matches_the_ocp_closed_form():
    raw = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    got = raw.view(torch.float8_e4m3fn).float().tolist()
    for b in range(256):
        want = e4m3_value(b)
        if math.isnan(want):
            assert math.isnan(got[b]), b
        else:
            assert got[b] == want, (b, got[b], want)
    assert max(v for v in got if not math.isnan(v)) == 448.0


def test_quantize_fp8_rounding_bound():
    fa = load_pkg()
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 257, generator=g) * 3.0
    x[0, 0] = -11.5  # some exact and some large values
    x8, d = fa.quantize_fp8(x)
    assert x8.dtype == torch.float8_e4m3fn
    assert d == pytest.approx(float(x.abs().max()) / 448.0)
    y = x8.float() * d
    assert float(y.abs().max()) == pytest.approx(float(x.abs().max()), rel=1e-6)
    # round to nearest with 3 mantissa bits: relative error <= 2^-4 in the normal range
    # (|x| / d >= 2^-6), absolute error <= d * 2^-10 below it
    err = (y - x).abs()
    normal = (x.abs() / d) >= 2.0 ** -6
    assert bool((err[normal] <= x[normal].abs() * 2.0 ** -4 * (1 + 1e-6)).all())
    assert bool((err[~normal] <= d * 2.0 ** -10 * (1 + 1e-6)).all())


def test_quantize_fp8_given_descale_and_zeros():
    fa = load_pkg()
    z8, d = fa.quantize_fp8(torch.zeros(3, 4))
    assert d == 1.0 and bool((z8.float() == 0).all())
    x8, d = fa.quantize_fp8(torch.tensor([1.0, -2.0, 1000.0]), descale=0.5)
    assert d == 0.5
    assert x8.float().tolist() == [2.0, -4.0, 448.0]  # saturates at the largest finite value


def _rounded_p_attention(q, k, v, scale, shift_rows):
    """O with the softmax weights rounded as fa_fwd_fp8_pv rounds them: P = 2^(s c - m + 4)
    with the reference m up to 4 below the row maximum (the kernel's lazy rescale; `shift_rows`
    picks it per row), cast to e4m3 (torch's cast: round to nearest even, the rounding the GPU's
    v_cvt_pk_fp8_f32 was checked to match), normalised by the sum of the rounded weights."""
    s = (q @ k.transpose(-1, -2)) * scale * 1.4426950408889634  # log2 domain, unmasked (causal mask below)
    L = q.shape[-2]
    s = s.masked_fill(torch.ones(L, L, dtype=torch.bool).triu(1), float("-inf"))
    m = s.amax(-1, keepdim=True) - shift_rows
    p = torch.exp2(s - m + 4.0)
    assert float(p.max()) <= 256.0
    pr = p.to(torch.float8_e4m3fn).to(p.dtype)
    return (pr @ v) / pr.sum(-1, keepdim=True)


@pytest.mark.parametrize("std", [0.5, 1.0, 4.0])
def test_pv_rounding_bound_holds_for_emulated_rounding(std):
    """The bound test_gpu_fp8.pv_bound checks on the GPU, verified against an emulation of the
    rounding it is derived for, on inputs from flat (std 0.5) to one-key-dominated (std 4)
    softmax rows: it holds for every element, is not vacuous (the worst element uses a good part
    of it), and a bound missing its first term fails."""
    from test_gpu_fp8 import pv_bound

    g = torch.Generator().manual_seed(int(std * 10))
    B, H, L, D = 1, 2, 200, 64
    q, k, v = (torch.randn(B, H, L, D, generator=g, dtype=torch.float64) * std for _ in range(3))
    scale = 1.0 / math.sqrt(D)
    shift = torch.rand(B, H, L, 1, generator=g, dtype=torch.float64) * 4.0
    o_ref = torch.softmax(((q @ k.transpose(-1, -2)) * scale).masked_fill(
        torch.ones(L, L, dtype=torch.bool).triu(1), float("-inf")), -1) @ v
    o_pv = _rounded_p_attention(q, k, v, scale, shift)
    ones = (1.0, 1.0, 1.0)
    bound, _ = pv_bound(q.float(), k.float(), v.float(), ones, L, 0, scale, o_ref.float())
    err = (o_pv - o_ref).abs().float()
    assert bool((err <= bound).all()), float((err - bound).max())
    assert float((err / bound).max()) > 0.25  # 0.44-0.60 on these inputs
    # a plausible slip -- the bound without its relative term -- is violated
    n = torch.arange(1, L + 1, dtype=torch.float32).view(1, 1, L, 1)
    only_abs = n * 2.0 ** -14 * (v.abs().amax(2, keepdim=True).float() + o_ref.abs().float())
    assert bool((err > only_abs).any())
