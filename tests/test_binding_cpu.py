"""The C++ PyTorch binding (csrc/fa_torch.cpp): loads, and keeps the error behaviour of the
ctypes path without a GPU (no compute call is made)."""
import importlib

import pytest
import torch

from conftest import load_pkg


def _binding():
    load_pkg()
    try:
        return importlib.import_module("flashattention-gpt-oss-finetuning_amd.fa_torch")
    except ImportError:
        pytest.skip("fa_torch binding not built (csrc/build_torch_ext.py)")


def test_binding_exports():
    b = _binding()
    assert callable(b.fwd) and callable(b.bwd)


def test_binding_rejects_cpu_tensors():
    b = _binding()
    q = torch.zeros(1, 2, 8, 16, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="need GPU tensors"):
        b.fwd(q, q, q, 4, 0, 0.25)
    with pytest.raises(RuntimeError, match="need GPU tensors"):
        b.bwd(q, q, q, q, torch.zeros(1, 2, 8), q, 4, 0, 0.25)


def test_ops_use_the_binding_when_built():
    b = _binding()
    ops = importlib.import_module("flashattention-gpt-oss-finetuning_amd._ops")
    assert ops._binding() is b
