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


def test_gpt_oss_adapter_host_checks(fa):
    """The GPT-OSS adapter's argument handling (no GPU needed: every case raises before a launch)."""
    import torch

    q = torch.zeros(1, 4, 8, 64, dtype=torch.bfloat16)
    k = torch.zeros(1, 2, 8, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="layout"):
        fa.attention(q, k, k, layout="lbhd")
    with pytest.raises(NotImplementedError, match="dropout"):
        fa.gpt_oss_attention_forward(None, q, k, k, None, dropout=0.1)
    with pytest.raises(NotImplementedError, match="KV cache"):
        fa.gpt_oss_attention_forward(None, q[:, :, :4], k, k, None)
    with pytest.raises(NotImplementedError, match="2-D"):
        fa.gpt_oss_attention_forward(None, q, k, k, torch.ones(1, 1, 8, 8, dtype=torch.bool))
    # a padded batch takes the packed path, which has no CPU implementation
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        fa.gpt_oss_attention_forward(None, q, k, k, torch.tensor([[1, 1, 1, 1, 1, 1, 1, 0]]))
    # CPU tensors reach the library boundary and fail loudly: there is no CPU implementation
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        fa.gpt_oss_attention_forward(None, q, k, k, None, s_aux=torch.zeros(4))


def test_gpt_oss_adapter_registers_with_transformers(fa):
    pytest.importorskip("transformers")
    from transformers import AttentionInterface
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS

    name = fa.register_transformers("fa_gfx950_test")
    assert AttentionInterface._global_mapping[name] is fa.gpt_oss_attention_forward
    assert name in ALL_MASK_ATTENTION_FUNCTIONS._global_mapping


def test_missing_binding_warns_once(monkeypatch):
    """Without the C++ binding the calls fall back to ctypes, which costs host time per step: the
    fallback is announced with a RuntimeWarning (once), not taken silently."""
    load_pkg()
    ops = importlib.import_module("flashattention-gpt-oss-finetuning_amd._ops")
    real = importlib.import_module

    def no_binding(name, *a, **k):
        if name.endswith(".fa_torch"):
            raise ImportError("simulated: binding not built")
        return real(name, *a, **k)

    monkeypatch.setattr(ops, "_BINDING", False)
    monkeypatch.setattr(ops.importlib, "import_module", no_binding)
    with pytest.warns(RuntimeWarning, match="ctypes"):
        assert ops._binding() is None
    import warnings
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        assert ops._binding() is None  # cached: no second warning
