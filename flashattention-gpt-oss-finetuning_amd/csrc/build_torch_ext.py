#!/usr/bin/env python3
"""Builds the PyTorch binding fa_torch (csrc/fa_torch.cpp) next to libfa_gfx950.so.

Host C++ only (no device code): g++ with PyTorch's headers, linked against the PyTorch
libraries and against libfa_gfx950.so (found next to the module through $ORIGIN).  Run after
the Makefile has built libfa_gfx950.so:  python csrc/build_torch_ext.py
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)


def output_path() -> str:
    return os.path.join(PKG, "fa_torch" + sysconfig.get_config_var("EXT_SUFFIX"))


def main() -> None:
    import torch
    from torch.utils import cpp_extension

    if not os.path.exists(os.path.join(PKG, "libfa_gfx950.so")):
        sys.exit("build libfa_gfx950.so first (make -C csrc)")
    incs = cpp_extension.include_paths() + [sysconfig.get_paths()["include"], "/opt/rocm/include"]
    libdir = cpp_extension.library_paths()[0]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    out = output_path()
    cmd = (["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wno-unused-function",
            os.path.join(HERE, "fa_torch.cpp"), "-o", out + ".tmp",
            "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=fa_torch",
            "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={abi}"]
           + [f"-I{i}" for i in incs]
           + [f"-L{libdir}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip", "-ltorch_hip",
              f"-L{PKG}", "-l:libfa_gfx950.so", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{libdir}"])
    subprocess.run(cmd, check=True)
    os.replace(out + ".tmp", out)
    print(f"built {out}")


if __name__ == "__main__":
    main()
