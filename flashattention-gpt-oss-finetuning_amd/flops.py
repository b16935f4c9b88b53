"""Work and traffic accounting for sliding-window + sink causal attention.

Conventions (the FA-2 convention used by the reference's README comparison):
  * allowed(q, k) = k <= q and (q - k < W or k < S)  (benchmark_backward_speed.py:40-46);
  * useful FLOPs count only allowed pairs: forward 2 GEMMs (4*D per pair), backward 5 GEMMs
    (10*D per pair), forward+backward 14*D per pair, per query head and batch;
  * algorithmic bytes are each tensor read or written once:
        forward  = |Q| + |K| + |V| + |O| + |LSE|
        backward = |Q| + |K| + |V| + |O| + |dO| + |LSE| + |dQ| + |dK| + |dV|.
"""
from __future__ import annotations

from dataclasses import dataclass

MI355X_PEAK_BF16_FLOPS = 2.5e15   # dense bf16/fp16 MFMA, AMD published figure
MI355X_PEAK_HBM_BYTES = 8.0e12    # HBM3E, AMD published figure


def _clamp(x: int, lo: int, hi: int) -> int:
    return lo if x < lo else (hi if x > hi else x)


def sum_min(S: int, T: int) -> int:
    """sum_{t=1..T} min(S, t) for S, T >= 0."""
    m = min(S, T)
    return m * (m + 1) // 2 + (T - m) * S


def allowed_pairs_per_head(seq_len: int, window: int, sink: int) -> int:
    """Number of allowed (q, k) pairs of one head, with W and S clamped to [0, L].

    Row q sees min(q+1, W) window keys and max(0, min(S, q-W+1)) sink keys left of its window,
    so the total is sum_{n=1..L} min(W, n) + sum_{t=1..L-W} min(S, t).
    """
    L = int(seq_len)
    W = _clamp(int(window), 0, L)
    S = _clamp(int(sink), 0, L)
    return sum_min(W, L) + sum_min(S, L - W)


@dataclass(frozen=True)
class Workload:
    batch: int
    heads_q: int
    heads_kv: int
    seq_len: int
    head_dim: int
    window: int
    sink: int
    elem_bytes: int = 2

    @property
    def pairs(self) -> int:
        return allowed_pairs_per_head(self.seq_len, self.window, self.sink)

    def flops(self, mode: str) -> float:
        per_pair = {"fwd": 4, "bwd": 10, "fwdbwd": 14}[mode]
        return float(per_pair) * self.head_dim * self.pairs * self.batch * self.heads_q

    def _sizes(self):
        e = self.elem_bytes
        q = self.batch * self.heads_q * self.seq_len * self.head_dim * e
        kv = self.batch * self.heads_kv * self.seq_len * self.head_dim * e
        lse = self.batch * self.heads_q * self.seq_len * 4
        return q, kv, lse

    def bytes(self, mode: str) -> float:
        q, kv, lse = self._sizes()
        fwd = q + 2 * kv + q + lse
        bwd = (q + 2 * kv + q + q + lse) + (q + 2 * kv)
        return float({"fwd": fwd, "bwd": bwd, "fwdbwd": fwd + bwd}[mode])

    def roofline_seconds(self, mode: str) -> float:
        return max(self.flops(mode) / MI355X_PEAK_BF16_FLOPS, self.bytes(mode) / MI355X_PEAK_HBM_BYTES)
