"""TEST INFRASTRUCTURE ONLY -- the parity oracle, never a product path.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package,
and only as the checker (or, for bench.py, as the timed CPU baseline).  The library in
flashattention-gpt-oss-finetuning_amd/ never imports it and has no CPU fallback.

Contents
  naive.py  -- restatement of the reference's naive PyTorch attention
               (benchmark_backward_speed.py:40-54, 68-85): the mask, the KV repeat, the
               textbook forward in the input dtype (the reference's baseline), and an explicit
               float32/float64 forward + backward returning O, LSE, dQ, dK, dV; the same with
               GPT-OSS learned per-head sink logits (also returning their gradient), and a
               restatement of HF transformers' eager GPT-OSS attention; variable-length
               (packed) batches as independent sequences, and the packed batch's
               block-diagonal mask.
  loops.py  -- pure-Python double loop over (q, k) for tiny shapes: a second, independent
               statement of the mask and of the forward.

How each function is pinned (tests/test_oracle.py): against PyTorch's SDPA (an independent
library routine) with an explicit boolean mask and in its is_causal mode, against the Python
loops, against closed forms (W = 1, W >= L, S >= L, Hq = Hkv, GQA equals repeated-KV MHA),
against torch.autograd.gradcheck (finite differences in float64) for the backward, and
against the committed fixtures in tests/golden/ (computed with SDPA in float64).  The learned
sinks are pinned against SDPA with one extra zero key whose additive mask column holds the sink
logit (an independent statement of "a logit in the denominator without a value"), against the
installed transformers package's own eager_attention_forward, against the no-sink oracle for a
sink of -inf, and by gradcheck for the sink gradient.  The variable-length oracle is pinned
against one SDPA call over the whole packed batch with the block-diagonal mask (and autograd
for the gradients), and against single-sequence batches of the fixed-length oracle.  The
reference ships no golden vectors of its own (it has no test suite).
"""
