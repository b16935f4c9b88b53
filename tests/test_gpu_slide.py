"""GPU parity of the sliding dQ kernel (csrc/fa_bwd_slide.hip), which the backward runs for D = 64
16-bit inputs whose KV groups hold a multiple of 8 query heads, with 1 <= W <= 161 and S <= 32.

The cases walk the edges of its LDS ring and of the sink paths around it:
  * lengths of 1, 31 and 33 rows (one partial tile), long sequences (many tiles per workgroup);
  * W = 1, 33, 160 and 161 (one to six 32-key window halves per tile);
  * S = 0, 1, 4, 17 and 32 (the separate sink half; S = 32 fills it), and the sink keys' dK/dV
    partials it writes per workgroup, folded in the dK/dV kernel (S <= 4) or by the fold launch
    (4 < S <= 16);
  * two KV heads, two batches, and G = 16 (two workgroups' head groups per KV head);
  * learned sink logits and packed batches with short and empty sequences (workgroups with no
    tile, which the fold skips).
  * a seeded random sweep inside the kernels' range, with softmax scales of either sign and zero
    (a negative scale flips the sign of Q on its way into the products; zero makes every allowed
    key equally likely).
Oracles and tolerances as tests/test_gpu_parity.py, test_gpu_sinks.py and test_gpu_varlen.py.
"""
import random

import pytest
import torch

from test_gpu_parity import BF, FP, run_case
from test_gpu_sinks import run_sinks_case
from test_gpu_varlen import run_varlen

pytestmark = pytest.mark.gpu

# (B, Hq, Hkv, L, D, W, S, dtype)
SLIDE_CASES = [
    pytest.param(1, 8, 1, 1, 64, 1, 1, BF, id="L1"),
    pytest.param(1, 8, 1, 31, 64, 161, 4, FP, id="L31-W161"),
    pytest.param(1, 8, 1, 33, 64, 5, 0, BF, id="L33-W5"),
    pytest.param(1, 8, 1, 200, 64, 161, 4, BF, id="W161-six-halves"),
    pytest.param(1, 8, 1, 260, 64, 160, 0, FP, id="W160-no-sink"),
    pytest.param(1, 8, 1, 300, 64, 129, 32, BF, id="S32-whole-sink-half"),
    pytest.param(1, 8, 1, 333, 64, 33, 17, FP, id="S17"),
    pytest.param(1, 8, 1, 1000, 64, 128, 8, BF, id="sink-fold-launch-S8"),
    pytest.param(1, 8, 1, 1000, 64, 128, 16, FP, id="sink-fold-launch-S16"),
    pytest.param(1, 8, 1, 700, 64, 1, 1, BF, id="W1-S1"),
    pytest.param(2, 16, 2, 517, 64, 64, 4, BF, id="B2-Hkv2"),
    pytest.param(1, 16, 1, 700, 64, 100, 3, FP, id="G16"),
    pytest.param(1, 8, 1, 4096, 64, 128, 4, BF, id="c2-shard-shape"),
    pytest.param(2, 8, 1, 2000, 64, 31, 5, BF, id="B2-W31-S5"),
]


@pytest.mark.parametrize("B,Hq,Hkv,L,D,W,S,dtype", SLIDE_CASES)
def test_slide_parity(gpu, B, Hq, Hkv, L, D, W, S, dtype):
    print(f"case B={B} Hq={Hq} Hkv={Hkv} L={L} D={D} W={W} S={S} {dtype}", flush=True)
    run_case(B, Hq, Hkv, L, D, W, S, dtype, seed=31)


@pytest.mark.parametrize("L,W,S,dtype", [(600, 128, 4, BF), (450, 161, 0, FP), (1000, 64, 12, BF)])
def test_slide_learned_sinks(gpu, L, W, S, dtype):
    print(f"case learned sinks L={L} W={W} S={S} {dtype}", flush=True)
    run_sinks_case(1, 8, 1, L, 64, W, S, dtype, seed=7)


@pytest.mark.parametrize("cu,W,S,sinks", [
    ([0, 5, 300, 300, 301, 1000], 128, 4, False),
    ([0, 700, 733, 734], 161, 12, False),
    ([0, 64, 1064, 1100], 96, 4, True),
])
def test_slide_varlen(gpu, cu, W, S, sinks):
    run_varlen(cu, 8, 1, 64, W, S, BF, seed=3, sinks=sinks)


def _slide_random_cases(n=24, seed=77):
    """Shapes drawn from a fixed seed inside the sliding kernels' range (D = 64, G a multiple of 8,
    1 <= W <= 161, S <= 32; the sliding forward takes W <= 129): lengths 1-2500, one or two batches
    and KV heads, G = 8 or 16, both dtypes, scales of either sign around 1/sqrt(D)."""
    rng = random.Random(seed)
    cases = []
    while len(cases) < n:
        G = rng.choice([8, 8, 16])
        Hkv = rng.choice([1, 2])
        B = rng.choice([1, 1, 2])
        L = rng.choice([rng.randint(1, 100), rng.randint(101, 1000), rng.randint(1001, 2500)])
        W = rng.choice([1, rng.randint(2, 129), rng.randint(130, 161)])
        S = rng.choice([0, rng.randint(1, 8), rng.randint(9, 32)])
        if B * Hkv * G * L * L > (1 << 27):
            continue
        dtype = rng.choice([BF, FP])
        scale = rng.choice([1.0, 1.0, 1.0, -1.0]) * rng.uniform(0.5, 1.5) / 8.0
        cases.append(pytest.param(B, Hkv * G, Hkv, L, W, S, dtype, scale, len(cases),
                                  id=f"SR{len(cases)}-B{B}-H{Hkv * G}x{Hkv}-L{L}-W{W}-S{S}-"
                                     f"{'bf16' if dtype is BF else 'fp16'}-{'neg' if scale < 0 else 'pos'}"))
    return cases


@pytest.mark.parametrize("B,Hq,Hkv,L,W,S,dtype,scale,seed", _slide_random_cases())
def test_slide_random(gpu, B, Hq, Hkv, L, W, S, dtype, scale, seed):
    """Every case also runs the reference's naive 16-bit path (on the CPU), whose error widens the
    absolute tolerance as in tests/test_gpu_parity.py.  The dK/dV rows of sink keys sum G x L terms
    (up to 16 heads x 2500 rows here, values up to about 20), and the 16-bit rounding of P -- in
    the products and in the forward's row sums, which the LSE carries into the backward -- moves
    them by a few 1e-2: for the case SR16 an emulation of exactly that rounding in float32
    reproduces the kernel's dV of the sink keys to half a bf16 ulp, and sits 0.024 from the
    float32 oracle on one element."""
    print(f"slide random case B={B} Hq={Hq} Hkv={Hkv} L={L} W={W} S={S} {dtype} scale={scale:.4g}", flush=True)
    run_case(B, Hq, Hkv, L, 64, W, S, dtype, seed=500 + seed, scale=scale, with_naive=True)


@pytest.mark.parametrize("scale", [0.0, -0.125])
def test_slide_scale_edge(gpu, scale):
    print(f"slide case scale={scale}", flush=True)
    run_case(1, 8, 1, 777, 64, 128, 4, BF, seed=9, scale=scale)
