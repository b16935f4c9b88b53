"""TEST INFRASTRUCTURE ONLY: pure-Python loops over (q, k) for tiny shapes.

A second statement of the mask and of the forward (benchmark_backward_speed.py:40-46, 68-85),
written without tensors so that it shares no code with oracle/naive.py.
"""
from __future__ import annotations

import math


def allowed(q: int, k: int, window: int, sink: int) -> bool:
    if k > q:
        return False
    return (q - k) < window or k < sink


def forward(q, k, v, window: int, sink: int, scale: float):
    """q: nested lists [Hq][L][D]; k, v: [Hkv][L][D].  Returns (o [Hq][L][D], lse [Hq][L])."""
    Hq, Hkv = len(q), len(k)
    group = Hq // Hkv
    L, D = len(q[0]), len(q[0][0])
    o = [[[0.0] * D for _ in range(L)] for _ in range(Hq)]
    lse = [[0.0] * L for _ in range(Hq)]
    for h in range(Hq):
        kh, vh = k[h // group], v[h // group]
        for i in range(L):
            scores = {}
            for j in range(L):
                if allowed(i, j, window, sink):
                    scores[j] = scale * sum(q[h][i][d] * kh[j][d] for d in range(D))
            mx = max(scores.values())
            z = sum(math.exp(s - mx) for s in scores.values())
            lse[h][i] = mx + math.log(z)
            for j, s in scores.items():
                w = math.exp(s - mx) / z
                for d in range(D):
                    o[h][i][d] += w * vh[j][d]
    return o, lse
