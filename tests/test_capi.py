"""CPU tests of the C ABI: the library loads, exports what include/fa_gfx950.h declares, and its
host-side validation returns the documented codes.  No kernel is launched (only argument
errors are exercised, which return before any HIP call)."""
import ctypes
import os
import re
import subprocess
import tempfile

import pytest

from conftest import ROOT, load_mod

_lib = load_mod("_lib")
HEADER = os.path.join(ROOT, "include", "fa_gfx950.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\**\s*(fa_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_python_export_list():
    assert _declared_functions() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    for name in _declared_functions():
        assert hasattr(L, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (fa_\w+)$", out, flags=re.M))
    assert set(_declared_functions()) <= exported


def test_version_and_strerror():
    L = _lib.lib()
    assert L.fa_version() == 10400
    codes = [0, -1, -2, -3, -4, -5, -6, -7, -8, -9, -10, -11]
    texts = [_lib.strerror(c) for c in codes]
    assert len(set(texts)) == len(codes)
    assert _lib.strerror(12345) == "unknown fa_status"


def test_struct_layouts_match_header():
    # the ctypes mirrors must have the C layout: 5 pointers + 5 x 3 int64 + 7 int32 + float + int32
    assert ctypes.sizeof(_lib.FwdParams) == 5 * 8 + 15 * 8 + 9 * 4 + 4  # padded to 8
    assert ctypes.sizeof(_lib.BwdParams) == 9 * 8 + 27 * 8 + 9 * 4 + 4
    # a C compiler agrees
    src = (
        '#include "fa_gfx950.h"\n#include <stdio.h>\n#include <stddef.h>\n'
        "int main(void){printf(\"%zu %zu %zu %zu\\n\", sizeof(fa_fwd_params), sizeof(fa_bwd_params),"
        " offsetof(fa_fwd_params, batch), offsetof(fa_bwd_params, softmax_scale));return 0;}\n"
    )
    tmp = tempfile.mkdtemp(prefix="fa_layout_")
    cfile, exe = os.path.join(tmp, "layout.c"), os.path.join(tmp, "layout")
    with open(cfile, "w") as f:
        f.write(src)
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), cfile, "-o", exe], check=True)
    vals = [int(x) for x in subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split()]
    assert vals == [ctypes.sizeof(_lib.FwdParams), ctypes.sizeof(_lib.BwdParams),
                    _lib.FwdParams.batch.offset, _lib.BwdParams.softmax_scale.offset]


def _fwd_params(**over):
    p = _lib.FwdParams()
    B, Hq, Hkv, L, D = 1, 8, 2, 128, 64
    fake = 1 << 20  # 16-byte aligned non-null addresses; never dereferenced (validation fails first or no launch)
    p.q, p.k, p.v, p.o, p.lse = fake, fake, fake, fake, fake
    p.q_stride[:] = (Hq * L * D, L * D, D)
    p.k_stride[:] = (Hkv * L * D, L * D, D)
    p.v_stride[:] = (Hkv * L * D, L * D, D)
    p.o_stride[:] = (Hq * L * D, L * D, D)
    p.lse_stride[:] = (Hq * L, L, 1)
    p.batch, p.heads_q, p.heads_kv, p.seqlen, p.head_dim = B, Hq, Hkv, L, D
    p.window, p.sink, p.softmax_scale, p.dtype = 16, 4, 0.125, _lib.FA_DTYPE_BF16
    for k, v in over.items():
        if k.endswith("_stride"):
            getattr(p, k)[:] = v
        else:
            setattr(p, k, v)
    return p


def _bwd_params(**over):
    p = _lib.BwdParams()
    f = _fwd_params()
    for name in ("q", "k", "v", "o", "lse"):
        setattr(p, name, getattr(f, name))
    p.dout, p.dq, p.dk, p.dv = f.q, f.q, f.k, f.v
    for name in ("q", "k", "v", "o", "lse"):
        getattr(p, name + "_stride")[:] = getattr(f, name + "_stride")[:]
    p.do_stride[:] = f.q_stride[:]
    p.dq_stride[:] = f.q_stride[:]
    p.dk_stride[:] = f.k_stride[:]
    p.dv_stride[:] = f.v_stride[:]
    for name in ("batch", "heads_q", "heads_kv", "seqlen", "head_dim", "window", "sink", "softmax_scale", "dtype"):
        setattr(p, name, getattr(f, name))
    for k, v in over.items():
        if k.endswith("_stride"):
            getattr(p, k)[:] = v
        else:
            setattr(p, k, v)
    return p


@pytest.mark.parametrize("over,code", [
    ({}, _lib.FA_OK),
    ({"q": None}, _lib.FA_ERR_NULL),
    ({"lse": None}, _lib.FA_ERR_NULL),
    ({"heads_q": 6}, _lib.FA_ERR_SHAPE),          # 6 % 4 != 0 ... with Hkv = 2 it divides; set below
    ({"batch": 0}, _lib.FA_ERR_SHAPE),
    ({"seqlen": 0}, _lib.FA_ERR_SHAPE),
    ({"heads_kv": 3}, _lib.FA_ERR_SHAPE),
    ({"head_dim": 48}, _lib.FA_ERR_HEAD_DIM),
    ({"head_dim": 256}, _lib.FA_ERR_HEAD_DIM),
    ({"head_dim": 8}, _lib.FA_ERR_HEAD_DIM),
    ({"dtype": 0}, _lib.FA_ERR_DTYPE),
    ({"dtype": 3}, _lib.FA_ERR_DTYPE),
    ({"dtype": 5}, _lib.FA_ERR_DTYPE),
    ({"dtype": _lib.FA_DTYPE_F32}, _lib.FA_OK),
    ({"dtype": _lib.FA_DTYPE_F32, "q_stride": (8 * 128 * 68, 128 * 68, 68)}, _lib.FA_OK),  # 68 floats: 272 B
    ({"dtype": _lib.FA_DTYPE_F32, "q_stride": (8 * 128 * 66, 128 * 66, 66)}, _lib.FA_ERR_ALIGN),  # 264 B
    ({"window": 0, "sink": 0}, _lib.FA_ERR_MASK),
    ({"window": -5, "sink": 0}, _lib.FA_ERR_MASK),
    ({"q": (1 << 20) + 8}, _lib.FA_ERR_ALIGN),
    ({"lse": (1 << 20) + 2}, _lib.FA_ERR_ALIGN),
    ({"q_stride": (8 * 128 * 64, 128 * 64, 68)}, _lib.FA_ERR_ALIGN),
    ({"k_stride": (-8, 128 * 64, 64)}, _lib.FA_ERR_ALIGN),
    ({"softmax_scale": float("nan")}, _lib.FA_ERR_SCALE),
    ({"softmax_scale": float("inf")}, _lib.FA_ERR_SCALE),
    ({"seqlen": (1 << 28) + 1}, _lib.FA_ERR_OVERFLOW),
])
def test_check_fwd_codes(over, code):
    if over == {"heads_q": 6}:
        over = {"heads_q": 6, "heads_kv": 4}
    assert _lib.lib().fa_check_fwd(ctypes.byref(_fwd_params(**over))) == code


def test_check_accepts_edge_values():
    L = _lib.lib()
    for over in ({"window": 0, "sink": 1}, {"window": 1, "sink": 0}, {"window": 10 ** 9, "sink": -3},
                 {"softmax_scale": 0.0}, {"softmax_scale": -0.3}, {"dtype": _lib.FA_DTYPE_F16},
                 {"head_dim": 16}, {"head_dim": 128}, {"seqlen": 1}):
        assert L.fa_check_fwd(ctypes.byref(_fwd_params(**over))) == _lib.FA_OK, over


@pytest.mark.parametrize("over,code", [
    ({}, _lib.FA_OK),
    ({"dout": None}, _lib.FA_ERR_NULL),
    ({"dv": None}, _lib.FA_ERR_NULL),
    ({"dq": (1 << 20) + 4}, _lib.FA_ERR_ALIGN),
    ({"do_stride": (8 * 128 * 64, 128 * 64, 65)}, _lib.FA_ERR_ALIGN),
    ({"head_dim": 96}, _lib.FA_ERR_HEAD_DIM),
    ({"window": 0, "sink": 0}, _lib.FA_ERR_MASK),
])
def test_check_bwd_codes(over, code):
    assert _lib.lib().fa_check_bwd(ctypes.byref(_bwd_params(**over))) == code


def test_check_bwd_rejects_slices_beyond_32bit_offsets():
    """The backward kernels address one (batch, head) slice of q/dout/lse with 32-bit byte
    offsets; a slice spanning 2^31 bytes or more is refused instead of wrapping."""
    L = _lib.lib()
    big = 1 << 20  # rows
    ok = _bwd_params(seqlen=big, q_stride=(64 * big * 64, big * 64, 64), do_stride=(64 * big * 64, big * 64, 64),
                     dq_stride=(64 * big * 64, big * 64, 64), lse_stride=(8 * big, big, 1))
    assert L.fa_check_bwd(ctypes.byref(ok)) == _lib.FA_OK  # (2^20 - 1) * 64 + 64 elements * 2 B < 2^31
    wide = _bwd_params(seqlen=big, q_stride=(8 * big * 1024, 1024, 8 * 1024), do_stride=(64 * big * 64, big * 64, 64),
                       dq_stride=(64 * big * 64, big * 64, 64), lse_stride=(8 * big, big, 1))
    assert L.fa_check_bwd(ctypes.byref(wide)) == _lib.FA_ERR_OVERFLOW


def test_check_rejects_kv_slices_beyond_32bit_offsets():
    """K and V are staged through buffer resources with 32-bit byte offsets inside one
    (batch, KV head) slice; both entry points refuse a slice spanning 2^31 bytes or more."""
    L = _lib.lib()
    big = 1 << 20
    assert L.fa_check_fwd(ctypes.byref(_fwd_params(seqlen=big))) == _lib.FA_OK
    wide = (2 * big * 8192, big * 8192, 8192)  # (2^20 - 1) rows of 8192 elements: 2^34 bytes
    for name in ("k_stride", "v_stride"):
        assert L.fa_check_fwd(ctypes.byref(_fwd_params(seqlen=big, **{name: wide}))) == _lib.FA_ERR_OVERFLOW
        assert L.fa_check_bwd(ctypes.byref(_bwd_params(seqlen=big, **{name: wide}))) == _lib.FA_ERR_OVERFLOW


def test_check_rejects_q_and_o_slices_beyond_32bit_offsets():
    """The forward stages q, and the dQ kernel stages q, dO and o, through buffer resources with
    32-bit byte offsets inside one (batch, head) slice.  The [B, L, H, D] layout of a GPT-OSS
    projection (sequence stride H * D) reaches 2^31 bytes per head slice at L = 300000 with
    Hq = 64, D = 64: such a q or o is refused, not read through wrapped offsets."""
    L = _lib.lib()
    Lg, Hq, D = 300000, 64, 64
    blhd = (Lg * Hq * D, D, Hq * D)  # [B, L, H, D] viewed as [B, H, L, D]
    assert (Lg - 1) * Hq * D * 2 >= 1 << 31
    fwd_ok = _fwd_params(seqlen=Lg)
    assert L.fa_check_fwd(ctypes.byref(fwd_ok)) == _lib.FA_OK
    assert L.fa_check_fwd(ctypes.byref(_fwd_params(seqlen=Lg, q_stride=blhd))) == _lib.FA_ERR_OVERFLOW
    # o is written through 64-bit addresses by the forward: accepted there
    assert L.fa_check_fwd(ctypes.byref(_fwd_params(seqlen=Lg, o_stride=blhd))) == _lib.FA_OK
    for name in ("q_stride", "o_stride", "do_stride"):
        assert L.fa_check_bwd(ctypes.byref(_bwd_params(seqlen=Lg, **{name: blhd}))) == _lib.FA_ERR_OVERFLOW, name
    # the gradients are written through 64-bit addresses
    for name in ("dq_stride", "dk_stride", "dv_stride"):
        assert L.fa_check_bwd(ctypes.byref(_bwd_params(seqlen=Lg, **{name: blhd}))) == _lib.FA_OK, name
    # the same shapes one row short of the limit are accepted: 2^31 / (Hq * D * 2) rows fit
    Lok = (1 << 31) // (Hq * D * 2)
    assert L.fa_check_fwd(ctypes.byref(_fwd_params(seqlen=Lok, q_stride=(Lok * Hq * D, D, Hq * D)))) == _lib.FA_OK
    assert L.fa_check_fwd(ctypes.byref(_fwd_params(seqlen=Lok + 1, q_stride=(Lok * Hq * D, D, Hq * D)))) == \
        _lib.FA_ERR_OVERFLOW


def test_entry_points_reject_before_any_hip_call():
    """fa_fwd / fa_bwd return the validation code for bad arguments (this runs without a GPU)."""
    L = _lib.lib()
    assert L.fa_fwd(None, None) == _lib.FA_ERR_NULL
    assert L.fa_fwd(ctypes.byref(_fwd_params(head_dim=48)), None) == _lib.FA_ERR_HEAD_DIM
    assert L.fa_bwd(ctypes.byref(_bwd_params(window=0, sink=0)), None, 0, None) == _lib.FA_ERR_MASK
    # valid arguments but no workspace
    assert L.fa_bwd(ctypes.byref(_bwd_params()), None, 0, None) == _lib.FA_ERR_WORKSPACE
    need = L.fa_bwd_workspace_bytes(1, 8, 2, 128, 64, 16, 4)
    assert L.fa_bwd(ctypes.byref(_bwd_params()), ctypes.c_void_p(1 << 20), need - 1, None) == _lib.FA_ERR_WORKSPACE
    assert L.fa_bwd(ctypes.byref(_bwd_params()), ctypes.c_void_p((1 << 20) + 16), need, None) == _lib.FA_ERR_WORKSPACE
    # learned-sink entry points: the parameter checks first, then the sink pointers
    assert L.fa_fwd_sinks(ctypes.byref(_fwd_params(head_dim=48)), ctypes.c_void_p(256), None) == _lib.FA_ERR_HEAD_DIM
    assert L.fa_fwd_sinks(ctypes.byref(_fwd_params()), None, None) == _lib.FA_ERR_NULL
    assert L.fa_fwd_sinks(ctypes.byref(_fwd_params()), ctypes.c_void_p(258), None) == _lib.FA_ERR_ALIGN
    ws_ok = (ctypes.c_void_p(1 << 20), need)
    assert L.fa_bwd_sinks(ctypes.byref(_bwd_params()), ctypes.c_void_p(256), ctypes.c_void_p(512), None, 0,
                          None) == _lib.FA_ERR_WORKSPACE
    assert L.fa_bwd_sinks(ctypes.byref(_bwd_params()), None, ctypes.c_void_p(512), *ws_ok, None) == _lib.FA_ERR_NULL
    assert L.fa_bwd_sinks(ctypes.byref(_bwd_params()), ctypes.c_void_p(256), None, *ws_ok, None) == _lib.FA_ERR_NULL
    assert L.fa_bwd_sinks(ctypes.byref(_bwd_params()), ctypes.c_void_p(256), ctypes.c_void_p(514), *ws_ok,
                          None) == _lib.FA_ERR_ALIGN


def test_workspace_bytes():
    L = _lib.lib()
    ws = L.fa_bwd_workspace_bytes
    # row statistics (lse * log2(e) and -delta): 2 * B*Hq*round_up(L, 32) floats, 256-aligned; no
    # sink split when every row is within the window of the sink block; the learned-sink partials:
    # B*Hq*ceil(L/32) floats, 256-aligned
    assert ws(1, 8, 2, 128, 64, 200, 4) == 2 * 8 * 128 * 4 + 256
    assert ws(1, 8, 2, 100, 64, 200, 4) == 2 * 8 * 128 * 4 + 256
    L_, D = 4096, 64
    expect_delta = 2 * 64 * 4096 * 4
    expect_dsink = 64 * (4096 // 32) * 4
    # S <= 16 sink keys, rows past block 0's window (row 191): the dK/dV kernel keeps one slot
    # (block 0's own rows) per KV head, dK and dV, S = 4 rows x D fp32; the dQ kernel's slots are
    # one per tile -- 4096 / 32 row tiles x 64 / 4 head groups
    expect_partial = 8 * 1 * 1 * 2 * 4 * D * 4
    expect_dq = 128 * 16 * 2 * 4 * D * 4
    assert ws(1, 64, 8, L_, D, 128, 4) == expect_delta + expect_partial + expect_dsink + expect_dq
    # S > 16: the sink rows are split into chunk workgroups of the dK/dV kernel: block 0's window
    # ends at row 191, chunks of 64 rows start at 160 (rounded down to 32):
    # ceil((4096 - 160) / 64) = 62 chunks + the regular slot, S = 40 sink rows
    expect_partial = 8 * 1 * (62 + 1) * 2 * 40 * D * 4
    assert ws(1, 64, 8, L_, D, 128, 40) == expect_delta + expect_partial + expect_dsink
    # invalid problems give 0
    assert ws(1, 8, 3, 128, 64, 16, 4) == 0
    assert ws(1, 8, 2, 128, 64, 0, 0) == 0


def test_varlen_entry_points_reject_before_any_hip_call():
    """fa_fwd_varlen / fa_bwd_varlen check their extra arguments on the host; no GPU needed."""
    L = _lib.lib()
    ws = (ctypes.c_void_p(256), ctypes.c_size_t(1 << 30))
    cu = ctypes.c_void_p(1024)
    assert L.fa_fwd_varlen(ctypes.byref(_fwd_params()), None, 100, None, None) == _lib.FA_ERR_NULL
    assert L.fa_fwd_varlen(ctypes.byref(_fwd_params()), ctypes.c_void_p(1026), 100, None, None) == _lib.FA_ERR_ALIGN
    assert L.fa_fwd_varlen(ctypes.byref(_fwd_params()), cu, -1, None, None) == _lib.FA_ERR_SHAPE
    assert L.fa_fwd_varlen(ctypes.byref(_fwd_params()), cu, 100, ctypes.c_void_p(514), None) == _lib.FA_ERR_ALIGN
    assert L.fa_fwd_varlen(ctypes.byref(_fwd_params(head_dim=48)), cu, 100, None, None) == _lib.FA_ERR_HEAD_DIM
    assert L.fa_bwd_varlen(ctypes.byref(_bwd_params()), None, 100, None, None, *ws, None) == _lib.FA_ERR_NULL
    assert L.fa_bwd_varlen(ctypes.byref(_bwd_params()), cu, 100, ctypes.c_void_p(256), None, *ws,
                           None) == _lib.FA_ERR_NULL
    assert L.fa_bwd_varlen(ctypes.byref(_bwd_params()), cu, 100, None, None, ctypes.c_void_p(256),
                           ctypes.c_size_t(0), None) == _lib.FA_ERR_WORKSPACE


@pytest.mark.parametrize("entry", ["fa_fwd_fp8", "fa_fwd_fp8_pv"])
def test_fp8_entry_point_rejects_before_any_hip_call(entry):
    """The fp8 entry points' own checks: e4m3 dtype code, D in {64, 128}, 16-byte strides of the
    e4m3 tensors (8-element strides of the bf16 output), finite dequantisation factors."""
    L = _lib.lib()
    F8 = _lib.FA_DTYPE_FP8_E4M3
    fn = getattr(L, entry)

    def call(p, qd=1.0, kd=1.0, vd=1.0, sinks=None):
        return fn(ctypes.byref(p), qd, kd, vd, sinks, None)

    assert fn(None, 1.0, 1.0, 1.0, None, None) == _lib.FA_ERR_NULL
    assert call(_fwd_params(dtype=F8, v=None)) == _lib.FA_ERR_NULL
    assert call(_fwd_params()) == _lib.FA_ERR_DTYPE  # bf16 code
    assert call(_fwd_params(dtype=F8, head_dim=32)) == _lib.FA_ERR_HEAD_DIM
    assert call(_fwd_params(dtype=F8, head_dim=16)) == _lib.FA_ERR_HEAD_DIM
    assert call(_fwd_params(dtype=F8, head_dim=48)) == _lib.FA_ERR_HEAD_DIM
    assert call(_fwd_params(dtype=F8), qd=float("nan")) == _lib.FA_ERR_SCALE
    assert call(_fwd_params(dtype=F8), vd=float("inf")) == _lib.FA_ERR_SCALE
    assert call(_fwd_params(dtype=F8, softmax_scale=1e30), qd=1e30) == _lib.FA_ERR_SCALE  # product overflows
    assert call(_fwd_params(dtype=F8, window=0, sink=0)) == _lib.FA_ERR_MASK
    # 72 is a valid 16-bit stride (a multiple of 8) but not 16 bytes of e4m3
    assert call(_fwd_params(dtype=F8, q_stride=(8 * 128 * 72, 128 * 72, 72))) == _lib.FA_ERR_ALIGN
    assert call(_fwd_params(dtype=F8, o_stride=(8 * 128 * 68, 128 * 68, 68))) == _lib.FA_ERR_ALIGN
    assert call(_fwd_params(dtype=F8, k=(1 << 20) + 8)) == _lib.FA_ERR_ALIGN
    assert call(_fwd_params(dtype=F8), sinks=ctypes.c_void_p(258)) == _lib.FA_ERR_ALIGN
    # the 16-bit entry points do not take the e4m3 code
    assert L.fa_check_fwd(ctypes.byref(_fwd_params(dtype=F8))) == _lib.FA_ERR_DTYPE


def test_scratch_entry_point_rejects_before_any_hip_call():
    """fa_bwd_scratch checks its arguments like fa_bwd, then refuses a problem whose workspace
    exceeds the library's static buffer (FA_ERR_SCRATCH), all before any HIP call."""
    L = _lib.lib()
    assert L.fa_bwd_scratch(None, None) == _lib.FA_ERR_NULL
    assert L.fa_bwd_scratch(ctypes.byref(_bwd_params(head_dim=48)), None) == _lib.FA_ERR_HEAD_DIM
    assert L.fa_bwd_scratch(ctypes.byref(_bwd_params(window=0, sink=0)), None) == _lib.FA_ERR_MASK
    # 64 heads x 2^20 rows of delta alone is 256 MiB > FA_SCRATCH_BYTES
    big = 1 << 20
    st = (64 * big * 64, big * 64, 64)
    p = _bwd_params(heads_q=64, heads_kv=8, seqlen=big, q_stride=st, o_stride=st, do_stride=st, dq_stride=st,
                    lse_stride=(64 * big, big, 1))
    assert L.fa_check_bwd(ctypes.byref(p)) == _lib.FA_OK
    assert L.fa_bwd_workspace_bytes(1, 64, 8, big, 64, 16, 4) > _lib.FA_SCRATCH_BYTES
    assert L.fa_bwd_scratch(ctypes.byref(p), None) == _lib.FA_ERR_SCRATCH


def test_float32_slices_are_bounded_with_4_byte_elements():
    """A float32 head slice spans twice the bytes of a 16-bit one: the 2^31-byte bound of the
    kernels' 32-bit offsets is reached at half the rows."""
    L = _lib.lib()
    F32 = _lib.FA_DTYPE_F32
    rows = (1 << 31) // (64 * 4)  # rows of 64 floats in 2^31 bytes: one too many
    st = (rows * 64, rows * 64, 64)
    assert L.fa_check_fwd(ctypes.byref(_fwd_params(dtype=F32, seqlen=rows - 1, q_stride=st, k_stride=st,
                                                   v_stride=st))) == _lib.FA_OK
    assert L.fa_check_fwd(ctypes.byref(_fwd_params(dtype=F32, seqlen=rows, q_stride=st))) == _lib.FA_ERR_OVERFLOW
    assert L.fa_check_fwd(ctypes.byref(_fwd_params(dtype=_lib.FA_DTYPE_BF16, seqlen=rows, q_stride=st))) == \
        _lib.FA_OK
