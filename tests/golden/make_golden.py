#!/usr/bin/env python3
"""Writes the golden fixtures tests/golden/cases.npz (run from the repository root:
``python tests/golden/make_golden.py``).

The reference ships no golden vectors or known-answer tests, so these are computed here,
independently of oracle/: the mask is built by a plain Python double loop from the reference's
predicate (benchmark_backward_speed.py:40-46: key k visible to query q when k <= q and
(q - k < W or k < S)), the forward is torch's scaled_dot_product_attention in float64 on K/V
repeated over the query-head group (repeat_kv, benchmark_backward_speed.py:49-54), the
gradients come from torch.autograd on that forward, and LSE is torch.logsumexp of the masked,
scaled float64 scores.  Inputs are drawn as the reference protocol does (a seeded CPU generator,
q, k, v, then dO from N(0, 1) in float32, benchmark_backward_speed.py:646-674) and rounded to the
case dtype; the fixture stores those exact 16-bit values as float32.

Each case stores, under the prefix "<name>/": meta [B, Hq, Hkv, L, D, W, S, dtype_code, seed]
(dtype_code 1 = bf16, 2 = fp16) and scale, the inputs q, k, v, do (float32 holding 16-bit values)
and the expected outputs o, lse, dq, dk, dv (float64 results rounded to float32).
"""
from __future__ import annotations

import math
import os

import numpy as np
import torch
import torch.nn.functional as F

# (name, B, Hq, Hkv, L, D, W, S, dtype_code, seed): sinks, windows, ragged and tiny L, GQA
# groups 1/2/8, every head dim, both dtypes, sink keys beyond one 64-key block
CASES = [
    ("gqa2_ragged_d16", 1, 4, 2, 70, 16, 8, 3, 1, 11),
    ("window1_d32_b2", 2, 2, 1, 33, 32, 1, 0, 2, 12),
    ("causal_d64", 1, 2, 2, 65, 64, 100, 0, 1, 13),
    ("sinks_beyond_block_g8", 1, 8, 1, 100, 32, 16, 70, 1, 14),
    ("single_row_fp16", 1, 2, 1, 1, 16, 4, 0, 2, 15),
    ("sink_only_d64", 1, 2, 1, 96, 64, 0, 5, 2, 16),
    ("window_d128_g2", 1, 2, 1, 80, 128, 40, 4, 1, 17),
]

DTYPES = {1: torch.bfloat16, 2: torch.float16}


def loop_mask(L: int, W: int, S: int) -> torch.Tensor:
    m = torch.zeros(L, L, dtype=torch.bool)
    for q in range(L):
        for k in range(L):
            m[q, k] = k <= q and (q - k < W or k < S)
    return m


def make_case(B, Hq, Hkv, L, D, W, S, code, seed):
    g = torch.Generator().manual_seed(seed)
    dt = DTYPES[code]
    q = torch.randn(B, Hq, L, D, generator=g).to(dt)
    k = torch.randn(B, Hkv, L, D, generator=g).to(dt)
    v = torch.randn(B, Hkv, L, D, generator=g).to(dt)
    do = torch.randn(B, Hq, L, D, generator=g).to(dt)
    scale = 1.0 / math.sqrt(D)
    G = Hq // Hkv
    mask = loop_mask(L, W, S)
    q64, k64, v64 = (t.double().requires_grad_() for t in (q, k, v))
    kr = k64.repeat_interleave(G, dim=1)
    vr = v64.repeat_interleave(G, dim=1)
    o = F.scaled_dot_product_attention(q64, kr, vr, attn_mask=mask, scale=scale)
    o.backward(do.double())
    with torch.no_grad():
        s = torch.matmul(q64, kr.transpose(-1, -2)) * scale
        lse = torch.logsumexp(s.masked_fill(~mask, float("-inf")), dim=-1)
    out = {
        "meta": np.array([B, Hq, Hkv, L, D, W, S, code, seed], dtype=np.int64),
        "scale": np.array(scale, dtype=np.float64),
        "q": q.float().numpy(), "k": k.float().numpy(), "v": v.float().numpy(), "do": do.float().numpy(),
        # computed in float64, stored rounded to float32 (relative 6e-8, far below every tolerance)
        "o": o.detach().float().numpy(), "lse": lse.float().numpy(),
        "dq": q64.grad.float().numpy(), "dk": k64.grad.float().numpy(), "dv": v64.grad.float().numpy(),
    }
    return out


def main():
    arrays = {}
    for name, *params in CASES:
        for key, val in make_case(*params).items():
            arrays[f"{name}/{key}"] = val
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cases.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {len(CASES)} cases to {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
