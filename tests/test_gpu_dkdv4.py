"""GPU parity of the 32-key dK/dV kernel (csrc/fa_bwd.hip bwd_dkdv4_kernel).  The backward runs it for
16-bit D <= 64 with KV groups of a multiple of 4 query heads, 1 <= W <= 512, no chunked sink rows,
and grids of 64-key blocks (B * Hkv * ceil(L / 64)) no larger than the CU count.

The cases walk its edges:
  * D = 16, 32 and 64; G = 4, 8 and 16 (one, two and four steps of 4 heads per row block);
  * workgroups of 8 and 16 waves (query-head slots), which small grids with G a multiple of 8 (or of
    16 at D = 16) take: the shard-sized G = 8 layer and the reference's Hkv = 1 default case;
  * L = 1 and partial last blocks; W = 1, 33, 128 and 512 (its largest window);
  * sink keys in dq_sink_mode (S <= 16 with rows past key block 0's window: the dQ kernel takes
    those rows, and key block 0's workgroup folds the partials), and S = 40 with every row inside
    the window (the sink keys span two 32-key workgroups, whose rows run to L);
  * packed batches with short and empty sequences, with learned sink logits;
  * a seeded random sweep inside its range, with scales of either sign.
Oracles and tolerances as tests/test_gpu_parity.py, test_gpu_sinks.py and test_gpu_varlen.py.
"""
import random

import pytest

from test_gpu_parity import BF, FP, run_case
from test_gpu_sinks import run_sinks_case
from test_gpu_varlen import run_varlen

pytestmark = pytest.mark.gpu

# (B, Hq, Hkv, L, D, W, S, dtype)
DKDV4_CASES = [
    pytest.param(1, 4, 1, 1, 16, 1, 1, FP, id="L1-D16"),
    pytest.param(1, 8, 2, 100, 32, 33, 0, BF, id="D32-W33"),
    pytest.param(1, 4, 1, 513, 64, 512, 4, BF, id="W512"),
    pytest.param(2, 8, 1, 300, 64, 1, 16, FP, id="W1-S16-dq-sink"),
    pytest.param(1, 4, 1, 150, 64, 128, 40, BF, id="S40-two-sink-blocks"),
    pytest.param(1, 16, 4, 700, 64, 64, 4, FP, id="G4"),
    pytest.param(1, 16, 1, 900, 64, 100, 8, BF, id="G16"),
    pytest.param(1, 8, 1, 2000, 64, 96, 12, BF, id="long-dq-sink"),
    pytest.param(1, 8, 2, 333, 16, 50, 3, FP, id="D16-G4"),
    pytest.param(2, 4, 1, 257, 32, 128, 0, BF, id="D32-B2"),
    pytest.param(1, 8, 1, 4096, 64, 128, 4, BF, id="G8-8-waves-shard"),
    pytest.param(1, 16, 1, 4096, 16, 256, 4, FP, id="G16-D16-16-waves-hkv1"),
    pytest.param(2, 32, 2, 700, 16, 40, 0, FP, id="G16-D16-16-waves-B2"),
]


@pytest.mark.parametrize("B,Hq,Hkv,L,D,W,S,dtype", DKDV4_CASES)
def test_dkdv4_parity(gpu, B, Hq, Hkv, L, D, W, S, dtype):
    print(f"case B={B} Hq={Hq} Hkv={Hkv} L={L} D={D} W={W} S={S} {dtype}", flush=True)
    run_case(B, Hq, Hkv, L, D, W, S, dtype, seed=41)


def test_dkdv4_learned_sinks(gpu):
    print("case learned sinks L=500 D=64 W=128 S=4", flush=True)
    run_sinks_case(1, 8, 2, 500, 64, 128, 4, BF, seed=5)


@pytest.mark.parametrize("cu,D,W,S,sinks", [
    ([0, 1, 130, 130, 600], 64, 128, 4, True),
    ([0, 300, 333, 1000], 32, 200, 0, False),
    ([0, 17, 17, 900, 1900], 16, 128, 4, True),
])
def test_dkdv4_varlen(gpu, cu, D, W, S, sinks):
    print(f"case varlen cu={cu} D={D} W={W} S={S} sinks={sinks}", flush=True)
    # D = 16: a G = 16 group (16-wave workgroups); otherwise G = 4
    Hq, Hkv = (16, 1) if D == 16 else (8, 2)
    run_varlen(cu, Hq, Hkv, D, W, S, BF, seed=13, sinks=sinks)


def _dkdv4_random_cases(n=16, seed=404):
    """Shapes drawn from a fixed seed inside the kernel's range: D 16-64, G = 4-16 (a multiple of 4),
    W 1-512, S 0-16 (sinks past the window go through the dQ kernel), grids of at most 256 key
    blocks of 64 (so that the kernel, not the 64-key one, runs on a 256-CU device), both dtypes,
    scales of either sign.  The naive 16-bit path runs too, for the sink keys' widened tolerance."""
    rng = random.Random(seed)
    cases = []
    while len(cases) < n:
        D = rng.choice([16, 32, 64, 64])
        G = rng.choice([4, 8, 12, 16])
        Hkv = rng.choice([1, 2])
        B = rng.choice([1, 1, 2])
        L = rng.choice([rng.randint(1, 64), rng.randint(65, 600), rng.randint(601, 1500)])
        W = rng.choice([1, rng.randint(2, 128), rng.randint(129, 512)])
        S = rng.choice([0, rng.randint(1, 4), rng.randint(5, 16)])
        if B * Hkv * ((L + 63) // 64) > 256 or B * Hkv * G * L * L > (1 << 25):
            continue
        dtype = rng.choice([BF, FP])
        scale = rng.choice([1.0, 1.0, -1.0]) * rng.uniform(0.5, 1.5) / D ** 0.5
        cases.append(pytest.param(B, Hkv * G, Hkv, L, D, W, S, dtype, scale, len(cases),
                                  id=f"K{len(cases)}-B{B}-H{Hkv * G}x{Hkv}-L{L}-D{D}-W{W}-S{S}-"
                                     f"{'bf16' if dtype is BF else 'fp16'}-{'neg' if scale < 0 else 'pos'}"))
    return cases


@pytest.mark.parametrize("B,Hq,Hkv,L,D,W,S,dtype,scale,seed", _dkdv4_random_cases())
def test_dkdv4_random(gpu, B, Hq, Hkv, L, D, W, S, dtype, scale, seed):
    print(f"dkdv4 random case B={B} Hq={Hq} Hkv={Hkv} L={L} D={D} W={W} S={S} {dtype} scale={scale:.4g}", flush=True)
    run_case(B, Hq, Hkv, L, D, W, S, dtype, seed=700 + seed, scale=scale, with_naive=True)
