"""CPU checks behind the FP8 forward's parity tests.

The GPU tests compare fa_fwd_fp8 with the float32 oracle evaluated on the dequantised inputs
descale * x8, where x8 is decoded by torch.float8_e4m3fn.  That decode is pinned here against
the OCP e4m3 definition (sign, 4 exponent bits with bias 7, 3 mantissa bits; exponent 0 is
subnormal, 0x7F / 0xFF are NaN, no infinities), written out in closed form, for all 256
encodings.  The host-side quantiser quantize_fp8 is checked for its rounding bound.  The C ABI's
argument checks for fa_fwd_fp8 are in test_capi.py.
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
