"""GPT-OSS integration: learned sinks, the [B, L, H, D] layout, sliding and full layers, and the
attention-function interface of HF transformers.

GPT-OSS alternates sliding-window layers (window 128) and full causal layers, and gives every
query head a learned sink logit that joins the softmax denominator without a value row.  The
reference's sinks are the first S key positions instead (benchmark_backward_speed.py:45); both
kinds run on the same gfx950 kernels (fa_fwd_sinks / fa_bwd_sinks of libfa_gfx950.so).

    attention(q, k, v, window_size=None, sink_size=0, sinks=None, scale=None, layout="bhld")
    gpt_oss_attention_forward(module, query, key, value, attention_mask, ...)  # transformers form
    register_transformers("fa_gfx950")   # then attn_implementation="fa_gfx950"

Layouts: "bhld" tensors are [B, H, L, D]; "blhd" tensors are [B, L, H, D] (the projection
output before the transpose).  Any head/sequence strides that are multiples of 8 elements are
read in place, and outputs take the inputs' memory layout, so neither layout is copied.
"""
from __future__ import annotations

from typing import Optional

import torch

from .attention import FlashSWDAWithLearnedSinks, FlashSWDAWithSink, flash_swda_with_sink_varlen


def attention(q, k, v, window_size: Optional[int] = None, sink_size: int = 0, sinks: Optional[torch.Tensor] = None,
              scale: Optional[float] = None, layout: str = "bhld"):
    """Causal GQA attention with an optional sliding window (None: full causal), positional sinks
    and learned per-head sink logits `sinks` [Hq] (None: none).  Returns o in `layout`."""
    if layout not in ("bhld", "blhd"):
        raise ValueError(f"layout must be 'bhld' or 'blhd', got {layout!r}")
    if layout == "blhd":
        q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    W = q.shape[2] if window_size is None else int(window_size)
    if sinks is None:
        o = FlashSWDAWithSink.apply(q, k, v, W, sink_size, True, scale)
    else:
        o = FlashSWDAWithLearnedSinks.apply(q, k, v, sinks, W, sink_size, scale)
    return o.transpose(1, 2) if layout == "blhd" else o


def gpt_oss_attention_forward(module, query, key, value, attention_mask, dropout: float = 0.0,
                              scaling: Optional[float] = None, sliding_window: Optional[int] = None,
                              s_aux: Optional[torch.Tensor] = None, **kwargs):
    """The attention-function form that transformers' GptOssAttention calls
    (query/key/value [B, H, L, D], s_aux = the module's sinks, sliding_window None for full
    layers).  Returns (attn_output [B, L, H, D], None), as the eager function does.

    Supported: training and prefill, no dropout.  attention_mask is None or the 2-D [B, L] padding
    mask that transformers' flash-attention mask function hands over (True or 1 = a token); a
    padded batch runs as a packed variable-length batch (padded_attention).  KV caches (query
    shorter than key), other mask forms and dropout raise NotImplementedError rather than
    computing something else."""
    if dropout:
        raise NotImplementedError("attention dropout is not implemented by the gfx950 kernels")
    if query.shape[2] != key.shape[2]:
        raise NotImplementedError("query and key lengths differ (KV cache decoding); only full sequences are supported")
    if attention_mask is not None:
        if attention_mask.dim() != 2:
            raise NotImplementedError("only the 2-D [batch, seq] padding mask of the flash-attention mask function "
                                      f"is supported, got a {attention_mask.dim()}-D mask")
        if not bool(attention_mask.all()):
            o = padded_attention(query, key, value, attention_mask, window_size=sliding_window, sinks=s_aux,
                                 scale=scaling)
            return o, None
    o = attention(query, key, value, window_size=sliding_window, sinks=s_aux, scale=scaling)
    return o.transpose(1, 2), None


def padded_attention(q, k, v, attention_mask, window_size: Optional[int] = None, sinks: Optional[torch.Tensor] = None,
                     scale: Optional[float] = None):
    """Attention over a padded batch: q [B, Hq, L, D], k/v [B, Hkv, L, D], attention_mask [B, L]
    (nonzero = token).  The tokens of each row are gathered, in order, into one packed batch with
    cu_seqlens and run through flash_swda_with_sink_varlen, so causality, the window and the sinks
    count positions from each sequence's first token (left and right padding alike; a row with
    gaps is concatenated, as flash-attention's unpadding does).  Returns o [B, L, Hq, D] with
    zeros at padded positions; gradients flow through the gather and scatter."""
    B, Hq, L, D = q.shape
    if tuple(attention_mask.shape) != (B, L):
        raise ValueError(f"attention_mask must be [B, L] = [{B}, {L}], got {tuple(attention_mask.shape)}")
    m = attention_mask.to(device=q.device, dtype=torch.bool)
    idx = m.reshape(-1).nonzero().squeeze(1)  # token rows of the [B * L] flattening, in order
    lens = m.sum(1, dtype=torch.int32)
    cu = torch.zeros(B + 1, dtype=torch.int32, device=q.device)
    cu[1:] = lens.cumsum(0)
    max_len = int(lens.max()) if B else 0
    if max_len == 0:
        return q.new_zeros(B, L, Hq, D)

    def pack(x):  # [B, H, L, D] -> [tokens, H, D]
        return x.transpose(1, 2).reshape(B * L, x.shape[1], D).index_select(0, idx)

    W = max_len if window_size is None else int(window_size)
    op = flash_swda_with_sink_varlen(pack(q), pack(k), pack(v), cu, max_len, W, 0, scale, sinks)
    return op.new_zeros(B * L, Hq, D).index_copy(0, idx, op).view(B, L, Hq, D)


def register_transformers(name: str = "fa_gfx950") -> str:
    """Registers gpt_oss_attention_forward with transformers' attention interface under `name`
    (with the flash-attention mask function, which hands over no mask for unpadded batches), so
    that models load with attn_implementation=name.  Returns name."""
    from transformers import AttentionInterface
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, flash_attention_mask

    AttentionInterface.register(name, gpt_oss_attention_forward)
    ALL_MASK_ATTENTION_FUNCTIONS.register(name, flash_attention_mask)
    return name
