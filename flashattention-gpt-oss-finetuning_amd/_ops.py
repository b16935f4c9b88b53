"""Tensor-level calls into libfa_gfx950.so: argument marshalling, output allocation, streams.

forward() / backward() go through the C++ binding fa_torch (csrc/fa_torch.cpp) when it is
built, else through the ctypes structures below; FwdCall / BwdCall are prepared ctypes launches
used to time single kernels.

PyTorch provides device memory (the caching allocator) and the current HIP stream; every
FLOP runs in the library's HIP kernels.  Inputs the kernels cannot read directly (head-dim
stride != 1, rows not 16-byte aligned) are first copied to a contiguous layout, as the
reference benchmark does for dO (benchmark_backward_speed.py:510).
"""
from __future__ import annotations

import ctypes
import importlib
import warnings

import torch

from . import _lib

_DTYPES = {torch.bfloat16: _lib.FA_DTYPE_BF16, torch.float16: _lib.FA_DTYPE_F16, torch.float32: _lib.FA_DTYPE_F32}
_I32_MIN, _I32_MAX = -(2 ** 31), 2 ** 31 - 1


def _i32(x: int) -> int:
    return _I32_MIN if x < _I32_MIN else (_I32_MAX if x > _I32_MAX else x)


def _kernel_ready(t: torch.Tensor) -> torch.Tensor:
    """t itself when the kernels can read it in place (head-dim stride 1, the other strides whole
    multiples of 16 bytes, 16-byte aligned base), else a contiguous copy."""
    st = t.stride()
    m = 16 // t.element_size() - 1
    if st[3] != 1 or (t.data_ptr() & 15) or (st[0] & m) or (st[1] & m) or (st[2] & m):
        t = t.contiguous()
        if t.data_ptr() & 15:
            t = t.clone(memory_format=torch.contiguous_format)
    return t


def _check(tensors, names):
    dev = tensors[0].device
    if dev.type != "cuda":
        raise RuntimeError(
            f"{names[0]} is on {dev}: the gfx950 attention kernels need GPU tensors "
            "(there is no CPU implementation)"
        )
    dt = tensors[0].dtype
    if dt not in _DTYPES:
        raise ValueError(f"{names[0]} has dtype {dt}; supported dtypes are bfloat16, float16 and float32")
    for t, n in zip(tensors, names):
        if t.dim() != 4:
            raise ValueError(f"{n} must be 4-D [B, H, L, D], got shape {tuple(t.shape)}")
        if t.device != dev:
            raise RuntimeError(f"{n} is on {t.device} but {names[0]} is on {dev}")
        if t.dtype != dt:
            raise ValueError(f"{n} has dtype {t.dtype} but {names[0]} has {dt}")


def _out_like(t: torch.Tensor) -> torch.Tensor:
    """An output with t's shape, dtype and memory layout (torch.empty_like keeps the strides of a
    dense tensor, e.g. a [B, L, H, D] buffer viewed as [B, H, L, D]), as the reference allocates
    o = torch.empty_like(q) (flash_attention_gpt_oss.py:356)."""
    return torch.empty_like(t)


def _sinks_ready(sinks: torch.Tensor, Hq: int, device: torch.device) -> torch.Tensor:
    """Learned sink logits as the C ABI takes them: float32 [Hq], contiguous, on the device."""
    if sinks.dim() != 1 or sinks.shape[0] != Hq:
        raise ValueError(f"sinks must have shape [{Hq}] (one logit per query head), got {tuple(sinks.shape)}")
    if sinks.device != device:
        raise RuntimeError(f"sinks is on {sinks.device} but q is on {device}")
    return sinks.to(torch.float32).contiguous()


def _strides3(t: torch.Tensor):
    s = t.stride()
    return (s[0], s[1], s[2])


class _DeviceGuard:
    """Makes `device` current for the HIP launch when it is not already (cheap no-op otherwise)."""

    __slots__ = ("idx", "prev")

    def __init__(self, device: torch.device):
        self.idx = device.index if device.index is not None else torch.cuda.current_device()
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if cur != self.idx:
            self.prev = cur
            torch.cuda.set_device(self.idx)

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False


class FwdCall:
    """A prepared forward launch: validated inputs, allocated outputs and a filled parameter
    block.  ``run()`` launches on the current stream of the inputs' device."""

    __slots__ = ("params", "inputs", "o", "lse", "device", "sinks")

    def __init__(self, q, k, v, window: int, sink: int, scale: float, sinks=None):
        _check((q, k, v), ("q", "k", "v"))
        q, k, v = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
        B, Hq, L, D = q.shape
        Hkv = k.shape[1]
        self.sinks = None if sinks is None else _sinks_ready(sinks, Hq, q.device)
        self.o = _out_like(q)
        self.lse = torch.empty((B, Hq, L), dtype=torch.float32, device=q.device)
        self.inputs = (q, k, v)  # keeps the (possibly copied) inputs alive
        self.device = q.device
        p = _lib.FwdParams()
        p.q, p.k, p.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
        p.o, p.lse = self.o.data_ptr(), self.lse.data_ptr()
        p.q_stride[:] = _strides3(q)
        p.k_stride[:] = _strides3(k)
        p.v_stride[:] = _strides3(v)
        p.o_stride[:] = _strides3(self.o)
        p.lse_stride[:] = self.lse.stride()
        p.batch, p.heads_q, p.heads_kv, p.seqlen, p.head_dim = B, Hq, Hkv, L, D
        p.window, p.sink = _i32(window), _i32(sink)
        p.softmax_scale = scale
        p.dtype = _DTYPES[q.dtype]
        self.params = p

    def run(self) -> None:
        with _DeviceGuard(self.device):
            stream = torch.cuda.current_stream(self.device).cuda_stream
            if self.sinks is None:
                rc, fn = _lib.lib().fa_fwd(ctypes.byref(self.params), ctypes.c_void_p(stream)), "fa_fwd"
            else:
                rc = _lib.lib().fa_fwd_sinks(ctypes.byref(self.params), ctypes.c_void_p(self.sinks.data_ptr()),
                                             ctypes.c_void_p(stream))
                fn = "fa_fwd_sinks"
        _lib.raise_for_status(rc, fn)


def _binding():
    """The C++ binding (csrc/fa_torch.cpp) when it is built, else None.  Both paths call the same
    C ABI of libfa_gfx950.so; the binding only does the per-call host work in C++."""
    global _BINDING
    if _BINDING is False:
        _lib.lib()  # the HIP library is required either way (raises when missing)
        try:
            _BINDING = importlib.import_module(__package__ + ".fa_torch")
        except ImportError as e:
            _BINDING = None
            warnings.warn(f"the C++ PyTorch binding fa_torch could not be imported ({e}); the attention calls go "
                          "through ctypes instead, which costs about 100 us of host time per forward + backward "
                          "(build it with csrc/build_torch_ext.py)", RuntimeWarning, stacklevel=3)
    return _BINDING


_BINDING = False


def autograd_binding(t: torch.Tensor):
    """The C++ binding when it is built and `t` is a GPU tensor, else None.  Its autograd functions
    (swda, swda_sinks) run the forward's bookkeeping and the whole backward in C++, which saves
    tens of microseconds of host time per training step; tensors that are not on a GPU go through
    the Python autograd functions, which raise for them."""
    if not t.is_cuda:
        return None
    return _binding()


def forward(q, k, v, window: int, sink: int, scale: float, sinks=None):
    """Returns (o, lse) for q [B,Hq,L,D], k/v [B,Hkv,L,D]; `sinks` ([Hq] learned sink logits or
    None) selects fa_fwd_sinks.  o has q's memory layout."""
    b = _binding()
    if b is not None:
        o, lse = b.fwd(q, k, v, int(window), int(sink), float(scale), sinks)
        return o, lse
    call = FwdCall(q, k, v, window, sink, scale, sinks)
    call.run()
    return call.o, call.lse


def _fp8_ready(t: torch.Tensor) -> torch.Tensor:
    """e4m3 inputs as fa_fwd_fp8 reads them: head-dim stride 1, strides multiples of 16 elements
    (bytes), 16-byte aligned base; otherwise a contiguous copy."""
    st = t.stride()
    if st[3] != 1 or (t.data_ptr() & 15) or (st[0] & 15) or (st[1] & 15) or (st[2] & 15):
        t = t.contiguous()
        if t.data_ptr() & 15:
            t = t.clone(memory_format=torch.contiguous_format)
    return t


class Fp8FwdCall:
    """A prepared fa_fwd_fp8 launch (fa_fwd_fp8_pv with ``fp8_pv``: P V on the fp8 matrix cores too):
    q [B,Hq,L,D], k/v [B,Hkv,L,D] in torch.float8_e4m3fn standing for descale[i] times their
    values; o is bfloat16 with q's memory layout, lse float32 [B,Hq,L]."""

    __slots__ = ("params", "inputs", "o", "lse", "device", "sinks", "descale", "entry")

    def __init__(self, q, k, v, window: int, sink: int, scale: float, descale=(1.0, 1.0, 1.0), sinks=None,
                 fp8_pv: bool = False):
        dev = q.device
        if dev.type != "cuda":
            raise RuntimeError(f"q is on {dev}: the gfx950 attention kernels need GPU tensors "
                               "(there is no CPU implementation)")
        for t, n in ((q, "q"), (k, "k"), (v, "v")):
            if t.dtype != torch.float8_e4m3fn:
                raise ValueError(f"{n} has dtype {t.dtype}; the fp8 forward takes torch.float8_e4m3fn")
            if t.dim() != 4:
                raise ValueError(f"{n} must be 4-D [B, H, L, D], got shape {tuple(t.shape)}")
            if t.device != dev:
                raise RuntimeError(f"{n} is on {t.device} but q is on {dev}")
        q, k, v = _fp8_ready(q), _fp8_ready(k), _fp8_ready(v)
        B, Hq, L, D = q.shape
        self.sinks = None if sinks is None else _sinks_ready(sinks, Hq, dev)
        self.o = torch.empty_like(q, dtype=torch.bfloat16)
        self.lse = torch.empty((B, Hq, L), dtype=torch.float32, device=dev)
        self.inputs = (q, k, v)
        self.device = dev
        self.descale = tuple(float(x) for x in descale)
        p = _lib.FwdParams()
        p.q, p.k, p.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
        p.o, p.lse = self.o.data_ptr(), self.lse.data_ptr()
        p.q_stride[:] = _strides3(q)
        p.k_stride[:] = _strides3(k)
        p.v_stride[:] = _strides3(v)
        p.o_stride[:] = _strides3(self.o)
        p.lse_stride[:] = self.lse.stride()
        p.batch, p.heads_q, p.heads_kv, p.seqlen, p.head_dim = B, Hq, k.shape[1], L, D
        p.window, p.sink = _i32(window), _i32(sink)
        p.softmax_scale = scale
        p.dtype = _lib.FA_DTYPE_FP8_E4M3
        self.params = p
        self.entry = "fa_fwd_fp8_pv" if fp8_pv else "fa_fwd_fp8"

    def run(self) -> None:
        qd, kd, vd = self.descale
        with _DeviceGuard(self.device):
            stream = torch.cuda.current_stream(self.device).cuda_stream
            rc = getattr(_lib.lib(), self.entry)(ctypes.byref(self.params), ctypes.c_float(qd), ctypes.c_float(kd),
                                                 ctypes.c_float(vd),
                                                 ctypes.c_void_p(None if self.sinks is None else self.sinks.data_ptr()),
                                                 ctypes.c_void_p(stream))
        _lib.raise_for_status(rc, self.entry)


def forward_fp8(q, k, v, window: int, sink: int, scale: float, descale=(1.0, 1.0, 1.0), sinks=None,
                fp8_pv: bool = False):
    """(o bf16, lse) of attention over the dequantised e4m3 inputs descale[0] q, descale[1] k,
    descale[2] v (fa_fwd_fp8; fa_fwd_fp8_pv with ``fp8_pv``)."""
    call = Fp8FwdCall(q, k, v, window, sink, scale, descale, sinks, fp8_pv)
    call.run()
    return call.o, call.lse


def workspace_bytes(B, Hq, Hkv, L, D, window, sink) -> int:
    return int(_lib.lib().fa_bwd_workspace_bytes(B, Hq, Hkv, L, D, _i32(window), _i32(sink)))


class BwdCall:
    """A prepared backward launch (outputs dq, dk, dv and the workspace allocated once).
    ``run(stage)`` launches fa_bwd ("all"), fa_bwd_dq ("dq") or fa_bwd_dkdv ("dkdv")."""

    __slots__ = ("params", "inputs", "dq", "dk", "dv", "ws", "device", "sinks", "dsinks")

    def __init__(self, q, k, v, o, lse, do, window: int, sink: int, scale: float, sinks=None):
        _check((q, k, v, o, do), ("q", "k", "v", "o", "do"))
        q, k, v, o, do = (_kernel_ready(t) for t in (q, k, v, o, do))
        B, Hq, L, D = q.shape
        Hkv = k.shape[1]
        dev = q.device
        self.sinks = None if sinks is None else _sinks_ready(sinks, Hq, dev)
        self.dsinks = None if sinks is None else torch.empty(Hq, dtype=torch.float32, device=dev)
        self.dq, self.dk, self.dv = _out_like(q), _out_like(k), _out_like(v)
        ws_bytes = workspace_bytes(B, Hq, Hkv, L, D, window, sink)
        self.ws = torch.empty((max(ws_bytes, 256),), dtype=torch.uint8, device=dev)
        self.inputs = (q, k, v, o, lse, do)
        self.device = dev
        p = _lib.BwdParams()
        p.q, p.k, p.v, p.o, p.dout = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr()
        p.lse = lse.data_ptr()
        p.dq, p.dk, p.dv = self.dq.data_ptr(), self.dk.data_ptr(), self.dv.data_ptr()
        p.q_stride[:] = _strides3(q)
        p.k_stride[:] = _strides3(k)
        p.v_stride[:] = _strides3(v)
        p.o_stride[:] = _strides3(o)
        p.do_stride[:] = _strides3(do)
        p.lse_stride[:] = lse.stride()
        p.dq_stride[:] = _strides3(self.dq)
        p.dk_stride[:] = _strides3(self.dk)
        p.dv_stride[:] = _strides3(self.dv)
        p.batch, p.heads_q, p.heads_kv, p.seqlen, p.head_dim = B, Hq, Hkv, L, D
        p.window, p.sink = _i32(window), _i32(sink)
        p.softmax_scale = scale
        p.dtype = _DTYPES[q.dtype]
        self.params = p

    def run(self, stage: str = "all") -> None:
        """stage "all" runs fa_bwd, or fa_bwd_sinks when learned sinks were given."""
        fn = {"all": "fa_bwd", "dq": "fa_bwd_dq", "dkdv": "fa_bwd_dkdv"}[stage]
        ws = (ctypes.c_void_p(self.ws.data_ptr()), ctypes.c_size_t(self.ws.numel()))
        with _DeviceGuard(self.device):
            stream = ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)
            if self.sinks is not None and stage == "all":
                fn = "fa_bwd_sinks"
                rc = _lib.lib().fa_bwd_sinks(ctypes.byref(self.params), ctypes.c_void_p(self.sinks.data_ptr()),
                                             ctypes.c_void_p(self.dsinks.data_ptr()), *ws, stream)
            else:
                rc = getattr(_lib.lib(), fn)(ctypes.byref(self.params), *ws, stream)
        _lib.raise_for_status(rc, fn)


def backward(q, k, v, o, lse, do, window: int, sink: int, scale: float, sinks=None):
    """Returns (dq, dk, dv) in the input dtype, each in the memory layout of q, k, v; with learned
    `sinks`, (dq, dk, dv, dsinks) with dsinks float32 [Hq]."""
    b = _binding()
    if b is not None:
        return tuple(b.bwd(q, k, v, o, lse, do, int(window), int(sink), float(scale), sinks))
    call = BwdCall(q, k, v, o, lse, do, window, sink, scale, sinks)
    call.run()
    if sinks is None:
        return call.dq, call.dk, call.dv
    return call.dq, call.dk, call.dv, call.dsinks


def backward_staged(q, k, v, o, lse, do, window: int, sink: int, scale: float):
    """(dq, dk, dv) through the two stages of the backward as separate C-ABI calls on one
    workspace: fa_bwd_dq (dq and the row statistic delta) then fa_bwd_dkdv (dk and dv), the
    benchmark's split backward (benchmark_backward_speed.py:574-612)."""
    call = BwdCall(q, k, v, o, lse, do, window, sink, scale)
    call.run("dq")
    call.run("dkdv")
    return call.dq, call.dk, call.dv


# ---- variable-length batches ------------------------------------------------------------------

def _check_packed(tensors, names):
    """[total, H, D] packed tensors on one GPU with one supported dtype, all with the same number
    of rows and head dim (the kernels bound every row they touch by q's row count)."""
    for t, n in zip(tensors, names):
        if t.dim() != 3:
            raise ValueError(f"{n} must be 3-D [total, H, D], got shape {tuple(t.shape)}")
    _check([t.unsqueeze(0) for t in tensors], names)
    total, _, D = tensors[0].shape
    for t, n in zip(tensors, names):
        if t.shape[0] != total or t.shape[2] != D:
            raise ValueError(f"{n} has shape {tuple(t.shape)}; packed tensors need {total} rows and head dim {D}")


def _as_bhld(t: torch.Tensor) -> torch.Tensor:
    """A packed [total, H, D] tensor as the [1, H, total, D] view the C ABI describes (the batch
    stride is not used by the varlen entry points)."""
    return _kernel_ready(t.permute(1, 0, 2).unsqueeze(0))


def cu_seqlens_ready(cu_seqlens: torch.Tensor, total: int, device: torch.device, max_seqlen=None):
    """cu_seqlens as the C ABI takes it -- int32 [B + 1] on the device -- and max_seqlen.

    Offsets given on the host are checked (start at 0, non-decreasing, end within the packed
    rows) and max_seqlen is computed when not given; offsets already on the device are used as
    they are (checking them would synchronise the host), with max_seqlen required.  The kernels
    clamp lengths and offsets either way, so bad device offsets give meaningless results, never
    out-of-range memory accesses."""
    if cu_seqlens.dim() != 1 or cu_seqlens.shape[0] < 2:
        raise ValueError(f"cu_seqlens must be 1-D [B + 1] with B >= 1, got shape {tuple(cu_seqlens.shape)}")
    if cu_seqlens.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"cu_seqlens must be an integer tensor, got {cu_seqlens.dtype}")
    if cu_seqlens.device.type == "cpu":
        c = cu_seqlens.to(torch.int64)
        lens = c[1:] - c[:-1]
        if int(c[0]) != 0 or bool((lens < 0).any()) or int(c[-1]) > total:
            raise ValueError("cu_seqlens must start at 0, be non-decreasing and end at most at the number of "
                             f"packed rows ({total}); got {c.tolist()}")
        if max_seqlen is None:
            max_seqlen = int(lens.max())
        elif int(lens.max()) > int(max_seqlen):
            raise ValueError(f"max_seqlen {max_seqlen} is below the longest sequence ({int(lens.max())})")
    elif cu_seqlens.device != device:
        raise RuntimeError(f"cu_seqlens is on {cu_seqlens.device} but q is on {device}")
    elif max_seqlen is None:
        raise ValueError("max_seqlen is required when cu_seqlens is on the GPU")
    return cu_seqlens.to(device=device, dtype=torch.int32).contiguous(), max(1, int(max_seqlen))


def forward_varlen(q, k, v, cu_seqlens, max_seqlen: int, window: int, sink: int, scale: float, sinks=None):
    """Returns (o [total, Hq, D], lse float32 [Hq, total]) for packed q [total, Hq, D] and
    k/v [total, Hkv, D]; cu_seqlens int32 [B + 1] on the device (see cu_seqlens_ready)."""
    _check_packed((q, k, v), ("q", "k", "v"))
    total, Hq, D = q.shape
    Hkv = k.shape[1]
    B = cu_seqlens.shape[0] - 1
    qv, kv, vv = _as_bhld(q), _as_bhld(k), _as_bhld(v)
    o = torch.empty((total, Hq, D), dtype=q.dtype, device=q.device)
    lse = torch.empty((Hq, total), dtype=torch.float32, device=q.device)
    ov = o.permute(1, 0, 2).unsqueeze(0)
    sk = None if sinks is None else _sinks_ready(sinks, Hq, q.device)
    p = _lib.FwdParams()
    p.q, p.k, p.v = qv.data_ptr(), kv.data_ptr(), vv.data_ptr()
    p.o, p.lse = ov.data_ptr(), lse.data_ptr()
    p.q_stride[:] = _strides3(qv)
    p.k_stride[:] = _strides3(kv)
    p.v_stride[:] = _strides3(vv)
    p.o_stride[:] = _strides3(ov)
    p.lse_stride[:] = (0, lse.stride(0), lse.stride(1))
    p.batch, p.heads_q, p.heads_kv, p.seqlen, p.head_dim = B, Hq, Hkv, _i32(max_seqlen), D
    p.window, p.sink = _i32(window), _i32(sink)
    p.softmax_scale = scale
    p.dtype = _DTYPES[q.dtype]
    with _DeviceGuard(q.device):
        stream = ctypes.c_void_p(torch.cuda.current_stream(q.device).cuda_stream)
        rc = _lib.lib().fa_fwd_varlen(ctypes.byref(p), ctypes.c_void_p(cu_seqlens.data_ptr()), _i32(total),
                                      ctypes.c_void_p(None if sk is None else sk.data_ptr()), stream)
    _lib.raise_for_status(rc, "fa_fwd_varlen")
    return o, lse


def backward_varlen(q, k, v, o, lse, do, cu_seqlens, max_seqlen: int, window: int, sink: int, scale: float,
                    sinks=None):
    """Returns (dq, dk, dv) packed like q, k, v (and dsinks float32 [Hq] with learned sinks)."""
    _check_packed((q, k, v, o, do), ("q", "k", "v", "o", "do"))
    total, Hq, D = q.shape
    Hkv = k.shape[1]
    B = cu_seqlens.shape[0] - 1
    qv, kv, vv, ovw, dov = (_as_bhld(t) for t in (q, k, v, o, do))
    dq = torch.empty_like(q, memory_format=torch.contiguous_format)
    dk = torch.empty_like(k, memory_format=torch.contiguous_format)
    dv = torch.empty_like(v, memory_format=torch.contiguous_format)
    dqv, dkv, dvv = (t.permute(1, 0, 2).unsqueeze(0) for t in (dq, dk, dv))
    sk = None if sinks is None else _sinks_ready(sinks, Hq, q.device)
    dsinks = None if sinks is None else torch.empty(Hq, dtype=torch.float32, device=q.device)
    ws_bytes = workspace_bytes(B, Hq, Hkv, int(max_seqlen), D, window, sink)
    ws = torch.empty((max(ws_bytes, 256),), dtype=torch.uint8, device=q.device)
    p = _lib.BwdParams()
    p.q, p.k, p.v, p.o, p.dout = qv.data_ptr(), kv.data_ptr(), vv.data_ptr(), ovw.data_ptr(), dov.data_ptr()
    p.lse = lse.data_ptr()
    p.dq, p.dk, p.dv = dqv.data_ptr(), dkv.data_ptr(), dvv.data_ptr()
    for field, t in (("q_stride", qv), ("k_stride", kv), ("v_stride", vv), ("o_stride", ovw), ("do_stride", dov),
                     ("dq_stride", dqv), ("dk_stride", dkv), ("dv_stride", dvv)):
        getattr(p, field)[:] = _strides3(t)
    p.lse_stride[:] = (0, lse.stride(0), lse.stride(1))
    p.batch, p.heads_q, p.heads_kv, p.seqlen, p.head_dim = B, Hq, Hkv, _i32(max_seqlen), D
    p.window, p.sink = _i32(window), _i32(sink)
    p.softmax_scale = scale
    p.dtype = _DTYPES[q.dtype]
    with _DeviceGuard(q.device):
        stream = ctypes.c_void_p(torch.cuda.current_stream(q.device).cuda_stream)
        rc = _lib.lib().fa_bwd_varlen(ctypes.byref(p), ctypes.c_void_p(cu_seqlens.data_ptr()), _i32(total),
                                      ctypes.c_void_p(None if sk is None else sk.data_ptr()),
                                      ctypes.c_void_p(None if dsinks is None else dsinks.data_ptr()),
                                      ctypes.c_void_p(ws.data_ptr()), ctypes.c_size_t(ws.numel()), stream)
    _lib.raise_for_status(rc, "fa_bwd_varlen")
    if sinks is None:
        return dq, dk, dv
    return dq, dk, dv, dsinks
