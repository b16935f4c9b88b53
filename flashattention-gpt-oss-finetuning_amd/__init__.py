"""MI355X (gfx950) sliding-window + sink FlashAttention-2, forward and backward.

Public surface (drop-in for flash_attention_gpt_oss.py:340-438):
    FlashSWDAWithSink.apply(q, k, v, window_size, sink_size, is_causal=True, softmax_scale=None)
    flash_swda_with_sink(q, k, v, window_size, sink_size=0, is_causal=True, scale=None)
    swa_sink_attention(q, k, v, window_size, sink_size)      # benchmark registry form

The directory name is not a Python identifier; import it with
``importlib.import_module("flashattention-gpt-oss-finetuning_amd")`` from the repository root.
"""
from .attention import FlashSWDAWithSink, flash_swda_with_sink, swa_sink_attention  # noqa: F401
from .flops import Workload, allowed_pairs_per_head  # noqa: F401

__all__ = [
    "FlashSWDAWithSink",
    "flash_swda_with_sink",
    "swa_sink_attention",
    "Workload",
    "allowed_pairs_per_head",
]
