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

import weakref
from typing import Optional

import torch

from .attention import _swda, flash_swda_with_sink_varlen


class _BatchFacts:
    """Host-side facts about one batch's padding mask or position ids (which rows hold tokens,
    where the packed sequences start, the longest one).  Working them out reads device memory,
    i.e. synchronises the host once; transformers hands the same tensor object to every attention
    layer of a forward pass, so the facts are kept for that tensor (while it lives and is not
    modified in place) and the other layers enqueue their kernels without waiting for the GPU.

    The entry is one tuple, replaced by a single store and read once per call, so threads that
    share the cache (replicas running layers at once) never pair one tensor's facts with
    another's key."""

    __slots__ = ("_entry",)

    def __init__(self):
        self._entry = None  # (weakref to the tensor, key, facts)

    def get(self, t: torch.Tensor, compute):
        key = (t.data_ptr(), t._version, tuple(t.shape), t.dtype, t.device)
        entry = self._entry
        if entry is not None and entry[0]() is t and entry[1] == key:
            return entry[2]
        val = compute(t)
        self._entry = (weakref.ref(t), key, val)
        return val


_MASK_FACTS = _BatchFacts()
_POSITION_FACTS = _BatchFacts()
_CU_FACTS = _BatchFacts()


def _mask_facts(attention_mask: torch.Tensor):
    """(all rows are tokens, token row indices of the [B * L] flattening, cu_seqlens int32 [B + 1],
    longest sequence) of a [B, L] padding mask (nonzero = token)."""
    m = attention_mask.to(dtype=torch.bool)
    if bool(m.all()):
        return True, None, None, m.shape[1]
    B = m.shape[0]
    idx = m.reshape(-1).nonzero().squeeze(1)
    lens = m.sum(1, dtype=torch.int32)
    cu = torch.zeros(B + 1, dtype=torch.int32, device=m.device)
    cu[1:] = lens.cumsum(0)
    return False, idx, cu, int(lens.max()) if B else 0


def _position_facts(position_ids: torch.Tensor):
    """(cu_seqlens int32 [n + 1], longest sequence) of a packed row of several sequences, or None.
    As transformers' flash-attention path does (_is_packed_sequence,
    prepare_fa_kwargs_from_position_ids): a single row whose position ids are not one increasing
    run holds several sequences, each starting where the ids return to their minimum."""
    if position_ids.dim() != 2 or position_ids.shape[0] != 1:
        return None
    p = position_ids.reshape(-1)
    first = p.min()
    if bool((p == torch.arange(p.numel(), device=p.device) + first).all()):
        return None
    starts = (p == first).nonzero().view(-1).to(torch.int32)
    cu = torch.cat((starts, torch.tensor([p.numel()], dtype=torch.int32, device=p.device)))
    return cu, int(cu.diff().max())


def attention(q, k, v, window_size: Optional[int] = None, sink_size: int = 0, sinks: Optional[torch.Tensor] = None,
              scale: Optional[float] = None, layout: str = "bhld"):
    """Causal GQA attention with an optional sliding window (None: full causal), positional sinks
    and learned per-head sink logits `sinks` [Hq] (None: none).  Returns o in `layout`."""
    if layout not in ("bhld", "blhd"):
        raise ValueError(f"layout must be 'bhld' or 'blhd', got {layout!r}")
    if layout == "blhd":
        q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    W = q.shape[2] if window_size is None else int(window_size)
    o = _swda(q, k, v, W, sink_size, True, scale, sinks=sinks)
    return o.transpose(1, 2) if layout == "blhd" else o


def gpt_oss_attention_forward(module, query, key, value, attention_mask, dropout: float = 0.0,
                              scaling: Optional[float] = None, sliding_window: Optional[int] = None,
                              s_aux: Optional[torch.Tensor] = None, **kwargs):
    """The attention-function form that transformers' GptOssAttention calls
    (query/key/value [B, H, L, D], s_aux = the module's sinks, sliding_window None for full
    layers).  Returns (attn_output [B, L, H, D], None), as the eager function does.

    Supported: training and prefill, no dropout.  attention_mask is None or the 2-D [B, L] padding
    mask that transformers' flash-attention mask function hands over (True or 1 = a token); a
    padded batch runs as a packed variable-length batch (padded_attention).  Without a mask,
    several sequences packed into one row (padding-free finetuning) are recognised as
    transformers' flash-attention path recognises them: from the data collator's cu_seq_lens_q /
    max_length_q keyword arguments, or from position_ids that restart inside the row; they run as
    a packed batch too, so no token attends across a sequence boundary.  The host reads the mask
    or the position ids once per batch (the first layer); the other layers reuse what it found.
    KV caches (query shorter than key), other mask forms and dropout raise NotImplementedError
    rather than computing something else."""
    if dropout:
        raise NotImplementedError("attention dropout is not implemented by the gfx950 kernels")
    if query.shape[2] != key.shape[2]:
        raise NotImplementedError("query and key lengths differ (KV cache decoding); only full sequences are supported")
    if attention_mask is not None:
        if attention_mask.dim() != 2:
            raise NotImplementedError("only the 2-D [batch, seq] padding mask of the flash-attention mask function "
                                      f"is supported, got a {attention_mask.dim()}-D mask")
        facts = _MASK_FACTS.get(attention_mask, lambda m: _mask_facts(m.to(query.device)))
        if not facts[0]:
            o = padded_attention(query, key, value, attention_mask, window_size=sliding_window, sinks=s_aux,
                                 scale=scaling, _facts=facts)
            return o, None
    else:
        packed = _packed_sequences(query, kwargs)
        if packed is not None:
            return _packed_row_attention(query, key, value, packed[0], packed[1], sliding_window, s_aux, scaling), None
    o = attention(query, key, value, window_size=sliding_window, sinks=s_aux, scale=scaling)
    return o.transpose(1, 2), None


def _packed_sequences(query, kwargs):
    """(cu_seqlens, longest sequence) when the unmasked batch packs several sequences per row,
    else None: the collator's cu_seq_lens_q (with max_length_q), or restarting position_ids."""
    cu_q = kwargs.get("cu_seq_lens_q")
    if cu_q is not None:
        cu_k = kwargs.get("cu_seq_lens_k")
        if cu_k is not None and cu_k is not cu_q and not torch.equal(cu_k.to(cu_q.device), cu_q):
            raise NotImplementedError("cu_seq_lens_k differs from cu_seq_lens_q; only self-attention over the same "
                                      "packed sequences is supported")
        max_len = kwargs.get("max_length_q")

        def facts(cu):
            n = int(cu.diff().max()) if max_len is None else int(max_len)
            return cu.to(device=query.device, dtype=torch.int32), n
        return _CU_FACTS.get(cu_q, facts)
    position_ids = kwargs.get("position_ids")
    if position_ids is None or query.shape[0] != 1:
        return None
    return _POSITION_FACTS.get(position_ids, lambda p: _position_facts(p.to(query.device)))


def _packed_row_attention(q, k, v, cu, max_len, window_size, sinks, scale):
    """Attention over B x L rows flattened into one packed batch with offsets cu (sequence b is
    flattened rows [cu[b], cu[b + 1])).  Returns [B, L, Hq, D]."""
    B, Hq, L, D = q.shape
    flat = lambda x: x.transpose(1, 2).reshape(B * L, x.shape[1], D)
    W = max_len if window_size is None else int(window_size)
    o = flash_swda_with_sink_varlen(flat(q), flat(k), flat(v), cu, max_len, W, 0, scale, sinks)
    return o.view(B, L, Hq, D)


def padded_attention(q, k, v, attention_mask, window_size: Optional[int] = None, sinks: Optional[torch.Tensor] = None,
                     scale: Optional[float] = None, _facts=None):
    """Attention over a padded batch: q [B, Hq, L, D], k/v [B, Hkv, L, D], attention_mask [B, L]
    (nonzero = token).  The tokens of each row are gathered, in order, into one packed batch with
    cu_seqlens and run through flash_swda_with_sink_varlen, so causality, the window and the sinks
    count positions from each sequence's first token (left and right padding alike; a row with
    gaps is concatenated, as flash-attention's unpadding does).  Returns o [B, L, Hq, D] with
    zeros at padded positions; gradients flow through the gather and scatter."""
    B, Hq, L, D = q.shape
    if tuple(attention_mask.shape) != (B, L):
        raise ValueError(f"attention_mask must be [B, L] = [{B}, {L}], got {tuple(attention_mask.shape)}")
    if _facts is None:
        _facts = _mask_facts(attention_mask.to(device=q.device))
    # token rows of the [B * L] flattening (in order), their offsets, the longest sequence
    _, idx, cu, max_len = _facts
    if idx is None:  # every row is a token
        return attention(q, k, v, window_size=window_size, sinks=sinks, scale=scale).transpose(1, 2)
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
