"""TEST INFRASTRUCTURE ONLY -- the parity oracle, never a product path.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package,
and only as the checker (or, for bench.py, as the timed CPU baseline).  The library in
flashattention-gpt-oss-finetuning_amd/ never imports it and has no CPU fallback.

Contents
  naive.py  -- restatement of the reference's naive PyTorch attention
               (benchmark_backward_speed.py:40-54, 68-85): the mask, the KV repeat, the
               textbook forward in the input dtype (the reference's baseline), and an explicit
               float32/float64 forward + backward returning O, LSE, dQ, dK, dV.
  loops.py  -- pure-Python double loop over (q, k) for tiny shapes: a second, independent
               statement of the mask and of the forward.

How each function is pinned (tests/test_oracle.py): against PyTorch's SDPA (an independent
library routine) with an explicit boolean mask and in its is_causal mode, against the Python
loops, against closed forms (W = 1, W >= L, S >= L, Hq = Hkv, GQA equals repeated-KV MHA),
against torch.autograd.gradcheck (finite differences in float64) for the backward, and
against the committed fixtures in tests/golden/ (computed with SDPA in float64).  The
reference ships no golden vectors of its own (it has no test suite).
"""
