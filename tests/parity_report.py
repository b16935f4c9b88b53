"""Achieved errors of the HIP path against the float32 oracle, per output tensor (not a test: a
report for the documentation; run on a GPU box from the repository root,
``python tests/parity_report.py [--small]``).

For each case and each of O, LSE, dQ, dK, dV it prints one JSON line with
  max_abs   max |ours - ref|
  max_rel   max |ours - ref| / max(|ref|, 1e-3)  over elements with |ref| >= 1e-2 (rel. error of
            the elements that are not near zero)
  need_a    the smallest a for which |ours - ref| <= a + 2e-2 |ref| holds everywhere (the tests'
            bar is a = 2e-2: need_a <= 0.02 passes at the north-star tolerance)
Inputs and oracle are those of tests/test_gpu_parity.py (seeded N(0, 1), float32 oracle on the
GPU, 2048 query rows at a time)."""
import argparse
import json
import math
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, HERE)

from conftest import load_mod  # noqa: E402
from oracle import naive  # noqa: E402  (the checker)
from test_gpu_parity import EDGE_CASES, make_inputs  # noqa: E402

BF, FP = torch.bfloat16, torch.float16
CONFIGS = {
    "c1": (1, 16, 16, 4096, 16, 256, 4, FP, 1.0),
    "c2": (1, 64, 8, 4096, 64, 128, 4, BF, 1.0),
    "c3": (1, 64, 8, 8192, 64, 8192, 0, BF, 1.0),
    "c4": (1, 64, 8, 32768, 64, 128, 4, BF, 0.1),
    "c5": (8, 32, 4, 2048, 128, 512, 16, FP, 1.0),
    "ref-Hkv8-fp16": (1, 16, 8, 4096, 16, 256, 4, FP, 1.0),
    "ref-Hkv1-fp16": (1, 16, 1, 4096, 16, 256, 4, FP, 1.0),
    "ref-Hkv8-bf16": (1, 16, 8, 4096, 16, 256, 4, BF, 1.0),
    "ref-Hkv1-bf16": (1, 16, 1, 4096, 16, 256, 4, BF, 1.0),
}


def errors(got, ref):
    got, ref = got.float(), ref.float()
    err = (got - ref).abs()
    big = ref.abs() >= 1e-2
    rel = (err[big] / ref.abs()[big]).max() if bool(big.any()) else torch.tensor(0.0)
    return dict(max_abs=float(err.max()), max_rel=float(rel), need_a=float((err - 2e-2 * ref.abs()).max()))


def report(name, B, Hq, Hkv, L, D, W, S, dtype, do_std=1.0, seed=0):
    ops = load_mod("_ops")
    q, k, v, do = make_inputs(B, Hq, Hkv, L, D, dtype, seed, do_std)
    sc = 1.0 / math.sqrt(D)
    o, lse = ops.forward(q, k, v, W, S, sc)
    dq, dk, dv = ops.backward(q, k, v, o, lse, do, W, S, sc)
    ref = naive.attention_fwd_bwd(q, k, v, do, W, S, scale=sc, row_chunk=2048)
    for t, got, r in zip(("O", "LSE", "dQ", "dK", "dV"), (o, lse, dq, dk, dv), ref):
        print(json.dumps({"case": name, "tensor": t, **{k_: round(v_, 6) for k_, v_ in errors(got, r).items()}}),
              flush=True)
    del q, k, v, do, o, lse, dq, dk, dv, ref
    torch.cuda.empty_cache()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--small", action="store_true", help="also the edge-case matrix of test_gpu_parity.py")
    args = ap.parse_args()
    for name, (B, Hq, Hkv, L, D, W, S, dt, std) in CONFIGS.items():
        report(name, B, Hq, Hkv, L, D, W, S, dt, std)
    if args.small:
        for p in EDGE_CASES:
            B, Hq, Hkv, L, D, W, S, dt = p.values
            report(p.id, B, Hq, Hkv, L, D, W, S, dt, seed=L + D + W)


if __name__ == "__main__":
    main()
