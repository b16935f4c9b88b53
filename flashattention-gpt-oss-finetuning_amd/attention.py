"""Drop-in replacement for the reference's autograd boundary.

``FlashSWDAWithSink`` and ``flash_swda_with_sink`` keep the calling surface of
flash_attention_gpt_oss.py:340-438 (same names, argument order, defaults, assertion messages,
saved tensors and 7-tuple of gradients); ``swa_sink_attention`` has the
``func(q, k, v, window_size, sink_size) -> o`` form of the benchmark's registries
(benchmark_backward_speed.py:615-643).  Compute goes to libfa_gfx950.so through :mod:`._ops`;
there is no CPU or PyTorch fallback: tensors that are not on a GPU raise.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _ops


class FlashSWDAWithSink(torch.autograd.Function):
    """Causal GQA attention with a sliding window and positional sink keys.

    forward(q [B,Hq,L,D], k [B,Hkv,L,D], v [B,Hkv,L,D], window_size, sink_size,
            is_causal=True, softmax_scale=None) -> o [B,Hq,L,D]
    (flash_attention_gpt_oss.py:341-385).  Saves (q, k, v, o, lse) for backward; lse is the
    natural-log log-sum-exp per query row, float32 [B,Hq,L].
    """

    @staticmethod
    def forward(ctx, q, k, v, window_size, sink_size, is_causal=True, softmax_scale=None):
        # Checks of flash_attention_gpt_oss.py:343-354, same conditions and messages.
        if not is_causal:
            raise AssertionError("Currently, only causal attention is supported")
        if softmax_scale is None:
            softmax_scale = 1.0 / math.sqrt(q.shape[-1])
        _check_shapes(q, k, v)

        o, lse = _ops.forward(q, k, v, int(window_size), int(sink_size), float(softmax_scale))

        ctx.save_for_backward(q, k, v, o, lse)
        ctx.softmax_scale = softmax_scale
        ctx.window_size = window_size
        ctx.sink_size = sink_size
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = _ops.backward(q, k, v, o, lse, do, int(ctx.window_size), int(ctx.sink_size),
                                   float(ctx.softmax_scale))
        return dq, dk, dv, None, None, None, None


class FlashSWDAWithLearnedSinks(torch.autograd.Function):
    """Causal GQA attention with a sliding window and GPT-OSS learned sink logits.

    forward(q [B,Hq,L,D], k [B,Hkv,L,D], v [B,Hkv,L,D], sinks [Hq], window_size, sink_size=0,
            softmax_scale=None) -> o [B,Hq,L,D]
    Every query head h has a learned logit sinks[h] that joins each row's softmax denominator
    without a value row (GPT-OSS; the reference's sinks are positional only,
    benchmark_backward_speed.py:45).  window_size None means full causal attention (GPT-OSS's
    full layers); positional sinks (sink_size) still apply.  The gradient of sinks comes back in
    sinks' dtype.  Saves (q, k, v, o, lse, sinks); lse includes the sink term.
    """

    @staticmethod
    def forward(ctx, q, k, v, sinks, window_size, sink_size=0, softmax_scale=None):
        if softmax_scale is None:
            softmax_scale = 1.0 / math.sqrt(q.shape[-1])
        _check_shapes(q, k, v)
        if window_size is None:
            window_size = q.shape[2]
        o, lse = _ops.forward(q, k, v, int(window_size), int(sink_size), float(softmax_scale), sinks=sinks)
        ctx.save_for_backward(q, k, v, o, lse, sinks)
        ctx.softmax_scale = softmax_scale
        ctx.window_size = window_size
        ctx.sink_size = sink_size
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse, sinks = ctx.saved_tensors
        dq, dk, dv, dsinks = _ops.backward(q, k, v, o, lse, do, int(ctx.window_size), int(ctx.sink_size),
                                           float(ctx.softmax_scale), sinks=sinks)
        return dq, dk, dv, dsinks.to(sinks.dtype), None, None, None


class FlashSWDAWithSinkVarlen(torch.autograd.Function):
    """Variable-length (packed) batches of the same attention.

    forward(q [total, Hq, D], k [total, Hkv, D], v [total, Hkv, D], cu_seqlens [B + 1],
            max_seqlen, window_size, sink_size, softmax_scale=None, sinks=None) -> o [total, Hq, D]
    Sequence b is rows [cu_seqlens[b], cu_seqlens[b + 1]) of every tensor; causality, the window
    and the sink_size positional sinks apply within each sequence.  `sinks` optionally adds
    GPT-OSS learned sink logits ([Hq]).  The reference takes fixed [B, H, L, D] batches only
    (flash_attention_gpt_oss.py:348); this is the layout of packed finetuning batches.
    """

    @staticmethod
    def forward(ctx, q, k, v, cu_seqlens, max_seqlen, window_size, sink_size, softmax_scale=None, sinks=None):
        if softmax_scale is None:
            softmax_scale = 1.0 / math.sqrt(q.shape[-1])
        if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
            raise AssertionError("Packed inputs must be 3-D [total, H, D]")
        _check_shapes(q.unsqueeze(0).transpose(1, 2), k.unsqueeze(0).transpose(1, 2), v.unsqueeze(0).transpose(1, 2))
        cu, max_seqlen = _ops.cu_seqlens_ready(cu_seqlens, q.shape[0], q.device, max_seqlen)
        if window_size is None:
            window_size = max_seqlen
        o, lse = _ops.forward_varlen(q, k, v, cu, max_seqlen, int(window_size), int(sink_size), float(softmax_scale),
                                     sinks=sinks)
        ctx.save_for_backward(q, k, v, o, lse, cu, sinks)
        ctx.softmax_scale = softmax_scale
        ctx.window_size = window_size
        ctx.sink_size = sink_size
        ctx.max_seqlen = max_seqlen
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse, cu, sinks = ctx.saved_tensors
        out = _ops.backward_varlen(q, k, v, o, lse, do, cu, ctx.max_seqlen, int(ctx.window_size), int(ctx.sink_size),
                                   float(ctx.softmax_scale), sinks=sinks)
        dsinks = None if sinks is None else out[3].to(sinks.dtype)
        return out[0], out[1], out[2], None, None, None, None, None, dsinks


def flash_swda_with_sink_varlen(q, k, v, cu_seqlens, max_seqlen, window_size, sink_size: int = 0,
                                scale: Optional[float] = None, sinks=None):
    """Functional form of FlashSWDAWithSinkVarlen: packed q [total, Hq, D], k/v [total, Hkv, D],
    cu_seqlens [B + 1] (int32 or int64; on the host it is validated, on the GPU max_seqlen is
    required), window_size None for full causal attention."""
    return FlashSWDAWithSinkVarlen.apply(q, k, v, cu_seqlens, max_seqlen, window_size, sink_size, scale, sinks)


E4M3_MAX = 448.0  # largest finite float8 e4m3 (OCP) value


def quantize_fp8(x: torch.Tensor, descale: Optional[float] = None):
    """Per-tensor e4m3 quantisation for flash_swda_with_sink_fp8: returns (x8, descale) with
    x ~= descale * x8 (x8 in torch.float8_e4m3fn, round to nearest even); descale defaults to
    amax(|x|) / 448, so the largest magnitude maps to the largest finite e4m3 value."""
    xf = x.detach().float()
    if descale is None:
        amax = float(xf.abs().max()) if xf.numel() else 0.0
        descale = amax / E4M3_MAX if amax > 0.0 else 1.0
    x8 = (xf / descale).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    return x8, float(descale)


def flash_swda_with_sink_fp8(q, k, v, window_size, sink_size: int = 0, scale: Optional[float] = None,
                             descale=(1.0, 1.0, 1.0), sinks=None, fp8_pv: bool = False):
    """Forward only, FP8 inputs: q [B,Hq,L,D], k/v [B,Hkv,L,D] in torch.float8_e4m3fn standing for
    descale[0] q, descale[1] k, descale[2] v (see quantize_fp8); D is 64 or 128.  Returns o in
    bfloat16: the same attention (window, positional sinks, optional learned sink logits
    `sinks` [Hq]) as flash_swda_with_sink on the dequantised inputs, with Q K^T on the fp8
    matrix cores.  With ``fp8_pv`` P V runs on them too, on softmax weights rounded to e4m3
    (a relative error of up to 2^-4 per weight; fa_fwd_fp8_pv in include/fa_gfx950.h).
    window_size None means full causal attention.  No autograd: the reference's kernels have no
    fp8 path (flash_attention_gpt_oss.py:356-383 take 16/32-bit tensors)."""
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    _check_shapes(q, k, v)
    if window_size is None:
        window_size = q.shape[2]
    o, _ = _ops.forward_fp8(q, k, v, int(window_size), int(sink_size), float(scale), descale, sinks, fp8_pv)
    return o


def _check_shapes(q, k, v):
    """The shape conditions of flash_attention_gpt_oss.py:347-354, same messages."""
    if not (q.shape[0] == v.shape[0] and q.shape[2] == v.shape[2] and q.shape[3] == v.shape[3]):
        raise AssertionError("Query and Value shapes must be compatible except for num_heads")
    if not (k.shape[0] == v.shape[0] and k.shape[1] == v.shape[1] and k.shape[2] == v.shape[2]
            and k.shape[3] == v.shape[3]):
        raise AssertionError("Key and Value shapes must be the same")
    if not q.shape[3] <= 128:
        raise AssertionError("Head dimension must be less than or equal to 128")
    if not q.shape[1] % k.shape[1] == 0:
        raise AssertionError("Number of query heads must be divisible by number of K/V heads")


def _swda(q, k, v, window_size, sink_size, is_causal=True, scale=None, sinks=None):
    """FlashSWDAWithSink (or, with `sinks`, FlashSWDAWithLearnedSinks) applied to GPU tensors
    through the binding's autograd functions in C++ (fa_torch.swda / swda_sinks): the same checks
    and messages, the same kernels, saved tensors and gradients, without Python in the backward.
    Without the binding, or for tensors that are not on a GPU, the Python autograd functions."""
    b = _ops.autograd_binding(q)
    if b is None:
        if sinks is None:
            return FlashSWDAWithSink.apply(q, k, v, window_size, sink_size, is_causal, scale)
        return FlashSWDAWithLearnedSinks.apply(q, k, v, sinks, window_size, sink_size, scale)
    if not is_causal:
        raise AssertionError("Currently, only causal attention is supported")
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    _check_shapes(q, k, v)
    if sinks is None:
        return b.swda(q, k, v, int(window_size), int(sink_size), float(scale))
    if window_size is None:
        window_size = q.shape[2]
    return b.swda_sinks(q, k, v, sinks, int(window_size), int(sink_size), float(scale))


def flash_swda_with_sink(q, k, v, window_size: int, sink_size: int = 0, is_causal: bool = True,
                         scale: Optional[float] = None):
    """Functional form, flash_attention_gpt_oss.py:437-438 (FlashSWDAWithSink.apply; on GPU
    tensors its C++ twin, see _swda)."""
    return _swda(q, k, v, window_size, sink_size, is_causal, scale)


def swa_sink_attention(q, k, v, window_size: int, sink_size: int):
    """Registry form ``func(q, k, v, window_size, sink_size) -> o`` with the default scale 1/sqrt(D)
    (triton_attention, benchmark_backward_speed.py:615-622): one backward call, fa_bwd."""
    return _swda(q, k, v, window_size, sink_size, True, None)


class FlashSWDAWithSinkSplit(torch.autograd.Function):
    """The benchmark's split-backward variant (TritonSWASinkAttentionSplit,
    benchmark_backward_speed.py:533-612): the same forward, and a backward made of two separate
    launches on one workspace -- fa_bwd_dq (dQ and the row statistic delta), then fa_bwd_dkdv
    (dK and dV).  Results equal FlashSWDAWithSink's bit for bit.

    forward(q, k, v, window_size, sink_size, softmax_scale=None) -> o; backward returns 6 values."""

    @staticmethod
    def forward(ctx, q, k, v, window_size, sink_size, softmax_scale=None):
        if softmax_scale is None:
            softmax_scale = 1.0 / math.sqrt(q.shape[-1])
        _check_shapes(q, k, v)
        o, lse = _ops.forward(q, k, v, int(window_size), int(sink_size), float(softmax_scale))
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.softmax_scale = softmax_scale
        ctx.window_size = window_size
        ctx.sink_size = sink_size
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = _ops.backward_staged(q, k, v, o, lse, do, int(ctx.window_size), int(ctx.sink_size),
                                          float(ctx.softmax_scale))
        return dq, dk, dv, None, None, None


def swa_sink_attention_split(q, k, v, window_size: int, sink_size: int):
    """Registry form of the split-backward variant (triton_attention_split,
    benchmark_backward_speed.py:625-632)."""
    return FlashSWDAWithSinkSplit.apply(q, k, v, window_size, sink_size, None)
