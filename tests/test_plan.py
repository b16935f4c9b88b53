"""Compiles tests/plan_check.cpp (the kernels' own visit plan, csrc/fa_plan.h, built with g++)
and checks that every allowed (query, key) pair is visited exactly once."""
import os
import subprocess
import tempfile

from conftest import ROOT


def test_visit_plan_covers_each_allowed_pair_once():
    exe = os.path.join(tempfile.mkdtemp(prefix="fa_plan_"), "plan_check")
    subprocess.run(["g++", "-O2", "-std=c++17", os.path.join(ROOT, "tests", "plan_check.cpp"), "-o", exe], check=True)
    out = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.startswith("OK "), out.stdout
    assert int(out.stdout.split()[1]) > 10000
