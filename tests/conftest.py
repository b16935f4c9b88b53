import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PKG_NAME = "flashattention-gpt-oss-finetuning_amd"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def load_pkg():
    return importlib.import_module(PKG_NAME)


def load_mod(name):
    return importlib.import_module(f"{PKG_NAME}.{name}")


@pytest.fixture(scope="session")
def fa():
    return load_pkg()


@pytest.fixture(scope="session")
def gpu():
    """Skips when no GPU is visible; FAILS (does not skip) when the GPU is there but the HIP
    library is missing, so a GPU run never passes without the native code."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    lib = load_mod("_lib")
    lib.lib()  # raises if libfa_gfx950.so is missing
    return torch.device("cuda", 0)
