"""CPU checks of the measurement code in bench.py: the FLOP accounting behind every TFLOP/s
figure, and the one-GPU contract of the command line.

The allowed-pair count (flops.allowed_pairs_per_head) sets every useful-FLOP figure.  It is
pinned two ways: against a brute-force count of the oracle's own mask (naive.allowed_mask) on
shapes where the sinks overlap the window, exceed it, or cover the sequence; and against the
per-config pair counts and GFLOP figures of the workload table computed when the hot path was
surveyed (allowed pairs per head, and 4 D pairs B Hq / 10 D pairs B Hq for forward / backward,
the FA-2 convention).
"""
import subprocess
import sys

import pytest
import torch

import bench
from oracle import naive


@pytest.mark.parametrize("L,W,S", [(1, 1, 0), (50, 1, 0), (300, 37, 5), (300, 37, 60), (129, 500, 3),
                                   (200, 0, 7), (64, 16, 64), (333, 128, 4)])
def test_allowed_pairs_match_a_brute_force_count_of_the_mask(L, W, S):
    flops = bench._mod("flops")
    assert flops.allowed_pairs_per_head(L, W, S) == int(naive.allowed_mask(L, W, S).sum())


# (config, allowed pairs per head, forward GFLOP, backward GFLOP), as surveyed
SURVEYED = [("c1", 1031290, 1.056, 2.640), ("c2", 532026, 8.717, 21.792), ("c3", 33558528, 549.8, 1374.6),
            ("c4", 4316730, 70.73, 176.81), ("c5", 942216, 123.5, 308.7)]


@pytest.mark.parametrize("name,pairs,gf_fwd,gf_bwd", SURVEYED)
def test_flop_accounting_matches_the_surveyed_workload_table(name, pairs, gf_fwd, gf_bwd):
    flops = bench._mod("flops")
    cfg = bench.CONFIGS[name]
    assert flops.allowed_pairs_per_head(cfg["L"], cfg["W"], cfg["S"]) == pairs
    wl = flops.Workload(cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["L"], cfg["D"], cfg["W"], cfg["S"])
    assert wl.flops("fwd") / 1e9 == pytest.approx(gf_fwd, rel=1e-3)
    assert wl.flops("bwd") / 1e9 == pytest.approx(gf_bwd, rel=1e-3)
    assert wl.flops("fwdbwd") == pytest.approx(wl.flops("fwd") + wl.flops("bwd"))
    # per kernel, its own products: the forward 2 (4 D pairs B Hq), dQ 3 (6) and dK/dV 4 (8) --
    # both backward kernels recompute S and dP -- against the step's 14 D pairs B Hq
    acc = bench.kernel_accounting(cfg)
    assert acc["fwd"]["flops"] == pytest.approx(wl.flops("fwd"))
    assert acc["bwd_dq"]["flops"] + acc["bwd_dkdv"]["flops"] == pytest.approx(wl.flops("bwd") * 14 / 10)


def test_bench_measures_one_gpu_only():
    r = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], capture_output=True, text=True, timeout=120,
                       cwd=bench.__file__.rsplit("/", 1)[0])
    assert r.returncode == 2
    assert "one GPU" in (r.stdout + r.stderr)


def test_cpu_baseline_reports_three_modes_on_a_small_workload():
    """The CPU baseline leg runs on a small workload: forward, fwd+bwd and backward-only times,
    the CPU model, cores and the host-memory rise are reported, and a sample smaller than the
    workload is labelled as extrapolated."""
    cfg = dict(B=1, Hq=4, Hkv=2, L=256, D=16, W=32, S=4, dtype="bf16", do_std=1.0, name="tiny")
    r = bench.cpu_baseline(cfg, budget_s=0.5)
    for k in ("fwd_ms", "fwdbwd_ms", "bwd_ms", "value", "cores", "cpu", "max_rss_delta_mb"):
        assert k in r, k
    assert r["fwd_ms"] > 0 and r["fwdbwd_ms"] > 0 and r["bwd_ms"] > 0
    assert r["kind"] == "port" and r["unit"] == "TFLOP/s"
    assert isinstance(r["extrapolated"], bool)
    assert "extrapolated" in r["sample"] if r["extrapolated"] else "full workload" in r["sample"]


def test_traffic_figure_names_its_source():
    t, src = bench.measured_traffic("c2", "bwd_dq")
    assert t is None or (t > 0 and "sha256" in src and "profiles/c2_hbm_traffic.txt" in src)
    assert bench.measured_traffic("nonexistent", "fwd") == (None, None)
