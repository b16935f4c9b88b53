"""ctypes binding of libfa_gfx950.so (the C ABI declared in include/fa_gfx950.h).

The structures below mirror ``fa_fwd_params`` / ``fa_bwd_params`` field for field.  Loading
the library needs no GPU; launching needs one.  There is no fallback: if the shared library
is missing, :func:`lib` raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libfa_gfx950.so")
CSRC_DIR = os.path.join(PKG_DIR, "csrc")
HEADER_PATH = os.path.join(os.path.dirname(PKG_DIR), "include", "fa_gfx950.h")

FA_DTYPE_BF16 = 1
FA_DTYPE_F16 = 2
FA_DTYPE_FP8_E4M3 = 3
FA_DTYPE_F32 = 4

FA_OK = 0
FA_ERR_NULL = -1
FA_ERR_SHAPE = -2
FA_ERR_HEAD_DIM = -3
FA_ERR_DTYPE = -4
FA_ERR_ALIGN = -5
FA_ERR_MASK = -6
FA_ERR_WORKSPACE = -7
FA_ERR_LAUNCH = -8
FA_ERR_OVERFLOW = -9
FA_ERR_SCALE = -10
FA_ERR_SCRATCH = -11
FA_SCRATCH_BYTES = 72 << 20

# Every function the header declares; the tests check that the library exports each one.
EXPORTS = (
    "fa_fwd",
    "fa_bwd",
    "fa_bwd_dq",
    "fa_bwd_dkdv",
    "fa_bwd_scratch",
    "fa_fwd_sinks",
    "fa_bwd_sinks",
    "fa_fwd_varlen",
    "fa_bwd_varlen",
    "fa_fwd_fp8",
    "fa_fwd_fp8_pv",
    "fa_bwd_workspace_bytes",
    "fa_check_fwd",
    "fa_check_bwd",
    "fa_strerror",
    "fa_version",
)

_i64x3 = ctypes.c_int64 * 3


class FwdParams(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("q_stride", _i64x3),
        ("k_stride", _i64x3),
        ("v_stride", _i64x3),
        ("o_stride", _i64x3),
        ("lse_stride", _i64x3),
        ("batch", ctypes.c_int32),
        ("heads_q", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32),
        ("seqlen", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("window", ctypes.c_int32),
        ("sink", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("dtype", ctypes.c_int32),
    ]


class BwdParams(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("dout", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("dq", ctypes.c_void_p),
        ("dk", ctypes.c_void_p),
        ("dv", ctypes.c_void_p),
        ("q_stride", _i64x3),
        ("k_stride", _i64x3),
        ("v_stride", _i64x3),
        ("o_stride", _i64x3),
        ("do_stride", _i64x3),
        ("lse_stride", _i64x3),
        ("dq_stride", _i64x3),
        ("dk_stride", _i64x3),
        ("dv_stride", _i64x3),
        ("batch", ctypes.c_int32),
        ("heads_q", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32),
        ("seqlen", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("window", ctypes.c_int32),
        ("sink", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("dtype", ctypes.c_int32),
    ]


_lock = threading.Lock()
_lib = None


def lib() -> ctypes.CDLL:
    """Load the shared library once (thread-safe).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run `make -C {CSRC_DIR}` or __graft_entry__.build()"
                )
            L = ctypes.CDLL(LIB_PATH)
            L.fa_fwd.argtypes = [ctypes.POINTER(FwdParams), ctypes.c_void_p]
            L.fa_fwd.restype = ctypes.c_int
            for name in ("fa_bwd", "fa_bwd_dq", "fa_bwd_dkdv"):
                fn = getattr(L, name)
                fn.argtypes = [ctypes.POINTER(BwdParams), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
                fn.restype = ctypes.c_int
            L.fa_bwd_scratch.argtypes = [ctypes.POINTER(BwdParams), ctypes.c_void_p]
            L.fa_bwd_scratch.restype = ctypes.c_int
            L.fa_fwd_sinks.argtypes = [ctypes.POINTER(FwdParams), ctypes.c_void_p, ctypes.c_void_p]
            L.fa_fwd_sinks.restype = ctypes.c_int
            L.fa_bwd_sinks.argtypes = [ctypes.POINTER(BwdParams), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_size_t, ctypes.c_void_p]
            L.fa_bwd_sinks.restype = ctypes.c_int
            L.fa_fwd_varlen.argtypes = [ctypes.POINTER(FwdParams), ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p,
                                        ctypes.c_void_p]
            L.fa_fwd_varlen.restype = ctypes.c_int
            L.fa_bwd_varlen.argtypes = [ctypes.POINTER(BwdParams), ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p,
                                        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
            L.fa_bwd_varlen.restype = ctypes.c_int
            for fn in (L.fa_fwd_fp8, L.fa_fwd_fp8_pv):
                fn.argtypes = [ctypes.POINTER(FwdParams), ctypes.c_float, ctypes.c_float, ctypes.c_float,
                               ctypes.c_void_p, ctypes.c_void_p]
                fn.restype = ctypes.c_int
            L.fa_bwd_workspace_bytes.argtypes = [ctypes.c_int32] * 7
            L.fa_bwd_workspace_bytes.restype = ctypes.c_size_t
            L.fa_check_fwd.argtypes = [ctypes.POINTER(FwdParams)]
            L.fa_check_fwd.restype = ctypes.c_int
            L.fa_check_bwd.argtypes = [ctypes.POINTER(BwdParams)]
            L.fa_check_bwd.restype = ctypes.c_int
            L.fa_strerror.argtypes = [ctypes.c_int]
            L.fa_strerror.restype = ctypes.c_char_p
            L.fa_version.argtypes = []
            L.fa_version.restype = ctypes.c_int
            _lib = L
    return _lib


def strerror(status: int) -> str:
    return lib().fa_strerror(status).decode()


def raise_for_status(status: int, what: str) -> None:
    """Map an fa_status to the Python exception the reference would raise for the same case."""
    if status == FA_OK:
        return
    msg = f"{what}: {strerror(status)} (fa_status {status})"
    if status == FA_ERR_LAUNCH:
        raise RuntimeError(msg)
    raise ValueError(msg)
