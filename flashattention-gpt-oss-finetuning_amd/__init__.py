"""MI355X (gfx950) sliding-window + sink FlashAttention-2, forward and backward.

Public surface (drop-in for flash_attention_gpt_oss.py:340-438):
    FlashSWDAWithSink.apply(q, k, v, window_size, sink_size, is_causal=True, softmax_scale=None)
    flash_swda_with_sink(q, k, v, window_size, sink_size=0, is_causal=True, scale=None)
    swa_sink_attention(q, k, v, window_size, sink_size)      # benchmark registry form
    swa_sink_attention_split(q, k, v, window_size, sink_size)  # split backward: fa_bwd_dq, fa_bwd_dkdv
    FlashSWDAWithSinkSplit.apply(q, k, v, window_size, sink_size, softmax_scale=None)

Variable-length (packed) batches, q [total, Hq, D] with cu_seqlens [B + 1]:
    flash_swda_with_sink_varlen(q, k, v, cu_seqlens, max_seqlen, window_size, sink_size=0,
                                scale=None, sinks=None)

FP8 (OCP e4m3) forward for the compute-bound shapes, D in {64, 128}, o in bfloat16:
    q8, qd = quantize_fp8(q); ...
    flash_swda_with_sink_fp8(q8, k8, v8, window_size, sink_size=0, scale=None,
                             descale=(qd, kd, vd), sinks=None)

GPT-OSS integration (gpt_oss.py): learned per-head sink logits, [B, L, H, D] tensors, full and
sliding layers, and transformers' attention-function interface:
    attention(q, k, v, window_size=None, sink_size=0, sinks=None, scale=None, layout="bhld")
    padded_attention(q, k, v, attention_mask, window_size=None, sinks=None, scale=None)  # [B, L] mask
    FlashSWDAWithLearnedSinks.apply(q, k, v, sinks, window_size, sink_size=0, softmax_scale=None)
    register_transformers("fa_gfx950")   # attn_implementation="fa_gfx950"

The directory name is not a Python identifier; import it with
``importlib.import_module("flashattention-gpt-oss-finetuning_amd")`` from the repository root.
"""
from .attention import (FlashSWDAWithLearnedSinks, FlashSWDAWithSink, FlashSWDAWithSinkSplit,  # noqa: F401
                        FlashSWDAWithSinkVarlen, flash_swda_with_sink, flash_swda_with_sink_fp8,
                        flash_swda_with_sink_varlen, quantize_fp8, swa_sink_attention, swa_sink_attention_split)
from .gpt_oss import attention, gpt_oss_attention_forward, padded_attention, register_transformers  # noqa: F401
from .flops import Workload, allowed_pairs_per_head  # noqa: F401

__all__ = [
    "FlashSWDAWithSink",
    "flash_swda_with_sink",
    "swa_sink_attention",
    "FlashSWDAWithSinkSplit",
    "swa_sink_attention_split",
    "FlashSWDAWithLearnedSinks",
    "FlashSWDAWithSinkVarlen",
    "flash_swda_with_sink_varlen",
    "flash_swda_with_sink_fp8",
    "quantize_fp8",
    "attention",
    "gpt_oss_attention_forward",
    "padded_attention",
    "register_transformers",
    "Workload",
    "allowed_pairs_per_head",
]
