#!/usr/bin/env python3
"""Benchmark of the sliding-window + sink FlashAttention-2 hot path on one MI355X.

A step is one forward + backward of the attention layer through the drop-in boundary
(flash_swda_with_sink, then o.backward(dO)) on synthetic, seeded inputs already resident in HBM.
The default workload is BASELINE config c2 (GPT-OSS sliding-window layer: B=1, Hq=64, Hkv=8,
L=4096, D=64, W=128, S=4, bf16).  Protocol after the reference's timers
(benchmark_backward_speed.py:720-783): W warm-up steps, then K timed steps bracketed by
torch.cuda.synchronize() and wall-clock perf_counter; forward-only and backward-only are timed the
same way.  Prints ONE JSON line.

  value        effective TFLOP/s of fwd+bwd, counting only allowed (unmasked) score pairs
               (14*D FLOPs per pair per head), whole job
  ms_per_step  fwd+bwd milliseconds
  roofline     the dominant kernel: algorithmic bytes (or FLOPs) per launch / its average
               duration measured with HIP events on the launch stream; `traffic` is its HBM
               bytes per launch from the copy-calibrated rocprofv3 FETCH_SIZE / WRITE_SIZE summary
               in profiles/<config>_hbm_traffic.txt (null without one)
  cpu_baseline the reference's naive PyTorch path (oracle/naive.py, in the config dtype) timed
               on the host cores on a bounded sample (whole KV groups of the same workload)
  sdpa_baseline the reference's other baseline, torch SDPA with a boolean mask, on the GPU
"""
from __future__ import annotations

import argparse
import importlib
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "fwd+bwd ms & effective TFLOP/s (unmasked FLOPs), Hq64/Hkv8 D64 W128 bf16"

CONFIGS = {
    "c1": dict(B=1, Hq=16, Hkv=16, L=4096, D=16, W=256, S=4, dtype="fp16", do_std=1.0,
               name="README benchmark shape"),
    "c2": dict(B=1, Hq=64, Hkv=8, L=4096, D=64, W=128, S=4, dtype="bf16", do_std=1.0,
               name="GPT-OSS sliding-window attention layer"),
    "c3": dict(B=1, Hq=64, Hkv=8, L=8192, D=64, W=8192, S=0, dtype="bf16", do_std=1.0,
               name="GPT-OSS full-causal layer"),
    "c4": dict(B=1, Hq=64, Hkv=8, L=32768, D=64, W=128, S=4, dtype="bf16", do_std=0.1,
               name="long-context window layer"),
    "c5": dict(B=8, Hq=32, Hkv=4, L=2048, D=128, W=512, S=16, dtype="fp16", do_std=1.0,
               name="batched wide-head variant"),
}

HBM_PEAK_GBS = 8000.0
COPY_BYTES = 256 << 20
MFMA_PEAK_TFLOPS = 2500.0


def _pkg():
    return importlib.import_module("flashattention-gpt-oss-finetuning_amd")


def _mod(name):
    return importlib.import_module("flashattention-gpt-oss-finetuning_amd." + name)


def make_inputs(cfg, device, seed=0):
    import torch

    dt = {"bf16": torch.bfloat16, "fp16": torch.float16}[cfg["dtype"]]
    g = torch.Generator().manual_seed(seed)
    B, Hq, Hkv, L, D = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["L"], cfg["D"]
    q = torch.randn(B, Hq, L, D, generator=g)
    k = torch.randn(B, Hkv, L, D, generator=g)
    v = torch.randn(B, Hkv, L, D, generator=g)
    do = torch.randn(B, Hq, L, D, generator=g) * cfg["do_std"]
    return [t.to(dt).to(device) for t in (q, k, v, do)]


def kernel_accounting(cfg):
    """Algorithmic FLOPs and bytes of each kernel launch (allowed pairs only; each tensor moved once)."""
    flops_mod = _mod("flops")
    B, Hq, Hkv, L, D = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["L"], cfg["D"]
    pairs = flops_mod.allowed_pairs_per_head(L, cfg["W"], cfg["S"])
    qb = B * Hq * L * D * 2
    kvb = B * Hkv * L * D * 2
    rowb = B * Hq * L * 4
    per = lambda n: float(n) * D * pairs * B * Hq
    return {
        # forward: QK^T, PV; reads Q K V, writes O and LSE
        "fwd": dict(flops=per(4), bytes=float(qb + 2 * kvb + qb + rowb)),
        # dQ: QK^T, dO V^T, dS K; reads Q K V O dO LSE, writes dQ and delta
        "bwd_dq": dict(flops=per(6), bytes=float(4 * qb + 2 * kvb + 2 * rowb)),
        # dK/dV: QK^T, dO V^T, P^T dO, dS^T Q; reads Q dO K V LSE delta, writes dK dV
        "bwd_dkdv": dict(flops=per(8), bytes=float(2 * qb + 4 * kvb + 2 * rowb)),
    }


# Kernels launched by each stage of the C ABI: the forward and dQ stages run one of two kernels
# (the sliding ones for the GPT-OSS sliding layers); fa_bwd_dkdv may also launch the sink fold.
STAGE_KERNELS = {"fwd": ["fwd_kernel", "fwd_slide_kernel"], "bwd_dq": ["bwd_dq_kernel", "bwd_dq_slide_kernel"],
                 "bwd_dkdv": ["bwd_dkdv_kernel", "bwd_sink_fold_kernel"]}


def measured_traffic(config, stage):
    """(HBM bytes per launch of a stage, where the figure comes from).  Hardware counters cannot be
    read inside this run, so the figure is the one in the rocprofv3 FETCH_SIZE / WRITE_SIZE summary
    committed as profiles/<config>_hbm_traffic.txt (copy-calibrated), identified by the file's
    sha256 prefix: it goes stale when a kernel changes and the profile is not regenerated.
    (None, None) when there is no summary."""
    import hashlib

    rel = os.path.join("profiles", f"{config}_hbm_traffic.txt")
    path = os.path.join(ROOT, rel)
    if not os.path.exists(path):
        return None, None
    rows = {}
    with open(path, "rb") as f:
        data = f.read()
    for line in data.decode().splitlines():
        parts = line.split()
        if len(parts) == 4 and parts[0].endswith("_kernel") and parts[3].isdigit():
            rows[parts[0]] = int(parts[3])
    names = STAGE_KERNELS[stage]
    if not any(n in rows and not n.startswith("bwd_sink") for n in names):
        return None, None
    src = f"{rel} (committed rocprofv3 --pmc summary, sha256 {hashlib.sha256(data).hexdigest()[:12]})"
    return float(sum(rows.get(n, 0) for n in names)), src


def time_kernels(cfg, q, k, v, do, iters=50):
    """Average duration of each kernel, launched alone through the C ABI, measured with HIP events
    recorded on the stream the kernel is launched on (torch's current stream)."""
    import torch

    ops = _mod("_ops")
    scale = 1.0 / math.sqrt(cfg["D"])
    fc = ops.FwdCall(q, k, v, cfg["W"], cfg["S"], scale)
    fc.run()
    bc = ops.BwdCall(q, k, v, fc.o, fc.lse, do, cfg["W"], cfg["S"], scale)
    bc.run()
    stages = {"fwd": fc.run, "bwd_dq": lambda: bc.run("dq"), "bwd_dkdv": lambda: bc.run("dkdv")}
    out = {}
    stream = torch.cuda.current_stream()
    for name, fn in stages.items():
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for _ in range(iters):
            fn()
        t1.record(stream)
        torch.cuda.synchronize()
        out[name] = t0.elapsed_time(t1) / iters * 1e3  # microseconds
    return out


def profile_launches(cfg, q, k, v, do, n):
    """A short program for hardware-counter runs: n launches of a plain 256 MiB device copy (the
    calibration for FETCH_SIZE / WRITE_SIZE: it reads and writes exactly 256 MiB), then n launches
    of each kernel of the path, with a synchronization between the groups."""
    import torch

    ops = _mod("_ops")
    scale = 1.0 / math.sqrt(cfg["D"])
    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=q.device).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(n):
        dst.copy_(src)
    torch.cuda.synchronize()
    fc = ops.FwdCall(q, k, v, cfg["W"], cfg["S"], scale)
    bc = ops.BwdCall(q, k, v, fc.o, fc.lse, do, cfg["W"], cfg["S"], scale)
    for fn in (fc.run, lambda: bc.run("dq"), lambda: bc.run("dkdv")):
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
    print(f"profile_launches: {n} x copy {COPY_BYTES} B, fwd, bwd_dq, bwd_dkdv on {cfg['name']}", flush=True)


def warm_clocks(fa, cfg, q, k, v, do, seconds):
    """Untimed fwd+bwd steps for about `seconds` (synchronising every 50 steps to read the clock);
    returns how many ran."""
    import torch

    qg, kg, vg = (t.detach().clone().requires_grad_() for t in (q, k, v))

    def steps(m):
        for _ in range(m):
            qg.grad = kg.grad = vg.grad = None
            fa.flash_swda_with_sink(qg, kg, vg, cfg["W"], cfg["S"]).backward(do)
        torch.cuda.synchronize()

    steps(2)  # first calls: library and code-object loading, allocator growth
    n = 2
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        steps(50)
        n += 50
    return n


def time_steps(fa, cfg, q, k, v, do, steps, warmup):
    import torch

    qg, kg, vg = (t.detach().clone().requires_grad_() for t in (q, k, v))
    W, S = cfg["W"], cfg["S"]

    def step():
        qg.grad = kg.grad = vg.grad = None
        o = fa.flash_swda_with_sink(qg, kg, vg, W, S)
        o.backward(do)

    # forward + backward
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    fb_ms = (time.perf_counter() - t0) * 1e3 / steps
    fb_event_ms = ev0.elapsed_time(ev1) / steps
    # per-step durations (an event before every step and after the last), for the median
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    for i in range(steps):
        evs[i].record()
        step()
    evs[steps].record()
    torch.cuda.synchronize()
    per_step = sorted(evs[i].elapsed_time(evs[i + 1]) for i in range(steps))
    fb_median_ms = per_step[steps // 2]
    peak_gb = torch.cuda.max_memory_allocated() / 2 ** 30

    # forward only (no autograd graph)
    with torch.no_grad():
        for _ in range(warmup):
            fa.flash_swda_with_sink(q, k, v, W, S)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        t0 = time.perf_counter()
        for _ in range(steps):
            fa.flash_swda_with_sink(q, k, v, W, S)
        torch.cuda.synchronize()
        f_ms = (time.perf_counter() - t0) * 1e3 / steps
        f_peak_gb = torch.cuda.max_memory_allocated() / 2 ** 30

    # backward only: forward, sync, then time backward (benchmark_backward_speed.py:761-783).  That
    # wall clock includes the host's autograd work before the first backward kernel starts on an
    # idle GPU.
    total = 0.0
    for i in range(warmup + steps):
        if i == warmup:
            torch.cuda.reset_peak_memory_stats()
        qg.grad = kg.grad = vg.grad = None
        o = fa.flash_swda_with_sink(qg, kg, vg, W, S)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        o.backward(do)
        torch.cuda.synchronize()
        if i >= warmup:
            total += time.perf_counter() - t0
    b_ms = total * 1e3 / steps
    b_peak_gb = torch.cuda.max_memory_allocated() / 2 ** 30
    # The GPU's backward throughput: the same backward repeated back to back on one retained graph
    # (torch.autograd.grad returns fresh gradients, so no accumulation kernels run), timed with
    # events, so the host queues ahead as in a training loop.
    o = fa.flash_swda_with_sink(qg, kg, vg, W, S)
    for _ in range(warmup):
        torch.autograd.grad(o, (qg, kg, vg), do, retain_graph=True)
    torch.cuda.synchronize()
    be0, be1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    be0.record()
    for _ in range(steps):
        torch.autograd.grad(o, (qg, kg, vg), do, retain_graph=True)
    be1.record()
    torch.cuda.synchronize()
    b_event_ms = be0.elapsed_time(be1) / steps
    del o
    return dict(fwdbwd_ms=fb_ms, fwdbwd_event_ms=fb_event_ms, fwdbwd_median_ms=fb_median_ms, fwd_ms=f_ms,
                bwd_ms=b_ms, bwd_event_ms=b_event_ms, peak_mem_gb=peak_gb, fwd_peak_mem_gb=f_peak_gb,
                bwd_peak_mem_gb=b_peak_gb)


def mode_figures(wl, t):
    """fwd, bwd and fwd+bwd of one time_steps result: ms, useful TFLOP/s, the fraction of that
    mode's roofline (max of its useful FLOPs at the MFMA peak and its algorithmic bytes at the HBM
    peak) and peak memory, as the reference reports them (benchmark_backward_speed.py:720-783)."""
    out = {}
    for mode, ms, peak in (("fwd", t["fwd_ms"], t["fwd_peak_mem_gb"]), ("bwd", t["bwd_ms"], t["bwd_peak_mem_gb"]),
                           ("fwdbwd", t["fwdbwd_ms"], t["peak_mem_gb"])):
        out[mode] = {"ms": round(ms, 4), "tflops": round(wl.flops(mode) / (ms * 1e-3) / 1e12, 2),
                     "roofline_us": round(wl.roofline_seconds(mode) * 1e6, 2),
                     "roofline_frac": round(wl.roofline_seconds(mode) / (ms * 1e-3), 4),
                     "peak_mem_gb": round(peak, 4)}
    # backward only as the GPU runs it back to back (time_steps), beside the reference's protocol
    ev = t["bwd_event_ms"]
    out["bwd"]["event_ms"] = round(ev, 4)
    out["bwd"]["event_roofline_frac"] = round(wl.roofline_seconds("bwd") / (ev * 1e-3), 4)
    return out


# The reference's own default cases (parse_cases, benchmark_backward_speed.py:829-835): B=1, Hq=16,
# Hkv in {16, 8, 1}, L=4096, D=16, W=256, S=4; the first is c1, the shape of its published numbers.
REFERENCE_CASES = {"hkv16": 16, "hkv8": 8, "hkv1": 1}


def reference_cases_measure(fa, dev, steps, warmup):
    """fwd, fwd+bwd and bwd-only times and peak memory of the reference's three default cases in
    fp16, with mode_figures' roofline fractions."""
    out = {}
    for name, hkv in REFERENCE_CASES.items():
        c = dict(CONFIGS["c1"], Hkv=hkv)
        qq, kk, vv, dd = make_inputs(c, dev)
        warm_clocks(fa, c, qq, kk, vv, dd, 0.1)  # the GPU idled while the inputs were drawn
        tt = time_steps(fa, c, qq, kk, vv, dd, steps, warmup)
        w = _mod("flops").Workload(c["B"], c["Hq"], c["Hkv"], c["L"], c["D"], c["W"], c["S"])
        out[name] = {"shape": f"B=1 Hq=16 Hkv={hkv} L=4096 D=16 W=256 S=4 fp16", **mode_figures(w, tt)}
        del qq, kk, vv, dd
    return out


def fp32_measure(fa, cfg, dev, steps, warmup):
    """The float32 path (q, k, v, o, dq, dk, dv in fp32 on the fp32 matrix instruction) on the
    config's shape: the three modes, with its useful TFLOP/s against the fp32 MFMA peak."""
    import torch

    q, k, v, do = (t.float() for t in make_inputs(cfg, dev))
    warm_clocks(fa, cfg, q, k, v, do, 0.1)
    tt = time_steps(fa, cfg, q, k, v, do, steps, warmup)
    w = _mod("flops").Workload(cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["L"], cfg["D"], cfg["W"], cfg["S"], elem_bytes=4)
    figs = mode_figures(w, tt)
    for mode in figs:  # the fp32 roofline: 157.3 TFLOP/s dense fp32 MFMA, 8 TB/s
        rs = max(w.flops(mode) / 157.3e12, w.bytes(mode) / 8.0e12)
        figs[mode]["roofline_us"] = round(rs * 1e6, 2)
        figs[mode]["roofline_frac"] = round(rs / (figs[mode]["ms"] * 1e-3), 4)
        if "event_ms" in figs[mode]:
            figs[mode]["event_roofline_frac"] = round(rs / (figs[mode]["event_ms"] * 1e-3), 4)
    del q, k, v, do
    torch.cuda.empty_cache()
    return {"dtype": "fp32", "peak_tflops": 157.3, **figs}


def graph_step_measure(fa, cfg, q, k, v, do, steps):
    """The fwd+bwd step captured once in a HIP graph (torch.cuda.CUDAGraph) and replayed: the
    time per replay, with no per-step host work (autograd and the launches are recorded once).
    A finetuning loop whose step is launch-bound can run its attention this way."""
    import torch

    qg, kg, vg = (t.detach().clone().requires_grad_() for t in (q, k, v))
    W, S = cfg["W"], cfg["S"]

    def step():
        fa.flash_swda_with_sink(qg, kg, vg, W, S).backward(do)

    side = torch.cuda.Stream()  # warm-up on a side stream, as capture requires
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            qg.grad = kg.grad = vg.grad = None
            step()
    torch.cuda.current_stream().wait_stream(side)
    qg.grad = kg.grad = vg.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(10):
        graph.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(steps):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    flops = _mod("flops").Workload(cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["L"], cfg["D"], W, S).flops("fwdbwd")
    return {"ms_per_step": round(ms, 4), "event_ms_per_step": round(ev0.elapsed_time(ev1) / steps, 4),
            "value": round(flops / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s"}


VARLEN_SEQS = (4096, 2048, 1024, 512, 3000, 1500, 700, 3504)  # 16384 packed rows


def varlen_measure(steps, warmup, seqs=VARLEN_SEQS):
    """fwd + bwd of a packed batch of GPT-OSS sliding-layer sequences of mixed lengths (Hq = 64,
    Hkv = 8, D = 64, W = 128, S = 4, bf16) through flash_swda_with_sink_varlen, cu_seqlens on the
    device; useful FLOPs count each sequence's allowed pairs."""
    import torch

    fa = _pkg()
    flops_mod = _mod("flops")
    Hq, Hkv, D, W, S = 64, 8, 64, 128, 4
    total = sum(seqs)
    g = torch.Generator().manual_seed(0)
    dev = torch.device("cuda", 0)
    q, k, v, do = (torch.randn(total, h, D, generator=g).to(torch.bfloat16).to(dev) for h in (Hq, Hkv, Hkv, Hq))
    cu = torch.tensor([0] + list(__import__("itertools").accumulate(seqs)), dtype=torch.int32, device=dev)
    qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))

    def step():
        qg.grad = kg.grad = vg.grad = None
        o = fa.flash_swda_with_sink_varlen(qg, kg, vg, cu, max(seqs), W, S)
        o.backward(do)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # then 0.1 s more: a switch of shapes leaves the clocks and the allocator's pools to settle
    # (measured: 0.474 ms per step after 5 warm-up steps, 0.382 ms after 100)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.1:
        for _ in range(10):
            step()
        torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    flops = sum(14.0 * D * flops_mod.allowed_pairs_per_head(L, W, S) * Hq for L in seqs)
    return {"workload": f"packed batch of {len(seqs)} sequences ({', '.join(map(str, seqs))}; {total} rows), "
                        f"Hq={Hq} Hkv={Hkv} D={D} W={W} S={S} bf16, fwd+bwd", "ms_per_step": round(ms, 4),
            "value": round(flops / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s"}


def long_context_measure(steps=10, warmup=3, L=131072):
    """fwd + bwd of GPT-OSS's sliding layer at its 128K context as its model runs it: learned sink
    logits (with their gradient), no positional sinks, q/k/v in the projections' [B, L, H, D]
    layout, through the adapter gpt_oss.attention.  B = 1, Hq = 64, Hkv = 8, D = 64, W = 128,
    bf16; useful FLOPs count the allowed pairs (a learned sink adds no key)."""
    import torch

    gpt_oss = _mod("gpt_oss")
    flops_mod = _mod("flops")
    Hq, Hkv, D, W = 64, 8, 64, 128
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(0)
    mk = lambda H: torch.randn(1, L, H, D, device=dev, dtype=torch.bfloat16, generator=g)
    q, k, v, do = mk(Hq).requires_grad_(), mk(Hkv).requires_grad_(), mk(Hkv).requires_grad_(), mk(Hq)
    sinks = torch.randn(Hq, device=dev, generator=g).requires_grad_()

    def step():
        q.grad = k.grad = v.grad = sinks.grad = None
        o = gpt_oss.attention(q, k, v, window_size=W, sinks=sinks, layout="blhd")
        o.backward(do)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    flops = 14.0 * D * flops_mod.allowed_pairs_per_head(L, W, 0) * Hq
    return {"workload": f"GPT-OSS sliding layer at {L // 1024}K context: B=1 Hq={Hq} Hkv={Hkv} L={L} D={D} W={W}, "
                        "learned sinks (and their gradient), [B, L, H, D] layout via gpt_oss.attention, bf16, fwd+bwd",
            "ms_per_step": round(ms, 4), "value": round(flops / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s"}


def shard_proxy_measure(steps, warmup, name="c2", parts=8):
    """One GPU's share of `name` split over `parts` GPUs by KV-head groups (zero communication:
    dK/dV reduce only inside a group): the same fwd + bwd on Hq / parts query heads and
    Hkv / parts KV heads, seq_len and everything else unchanged.  `value` is the device
    throughput of the three kernels (their HIP-event times summed, as time_kernels measures
    them); the autograd step is reported beside it, and at this size it is bound by the host's
    enqueue cost rather than the GPU."""
    import torch

    fa = _pkg()
    flops_mod = _mod("flops")
    cfg = dict(CONFIGS[name])
    cfg["Hq"] //= parts
    cfg["Hkv"] //= parts
    dev = torch.device("cuda", 0)
    q, k, v, do = make_inputs(cfg, dev)
    t = time_steps(fa, cfg, q, k, v, do, steps, warmup)
    kt = time_kernels(cfg, q, k, v, do)
    wl = flops_mod.Workload(cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["L"], cfg["D"], cfg["W"], cfg["S"])
    flops = wl.flops("fwdbwd")
    ksum = sum(kt.values())
    del q, k, v, do
    return {"workload": f"{name} on one GPU of {parts} (KV-group shard): B={cfg['B']} Hq={cfg['Hq']} "
                        f"Hkv={cfg['Hkv']} L={cfg['L']} D={cfg['D']} W={cfg['W']} S={cfg['S']} {cfg['dtype']}, "
                        f"fwd+bwd", "kernel_us": {n: round(x, 2) for n, x in kt.items()},
            "kernel_sum_us": round(ksum, 2), "value": round(flops / (ksum * 1e-6) / 1e12, 2), "unit": "TFLOP/s",
            "autograd_step_ms": round(t["fwdbwd_ms"], 4)}


FP8_CONFIGS = ("c3", "c5", "c2")


def fp8_forward_measure(iters=20, warmup=10, reps=3, names=FP8_CONFIGS):
    """Forward kernel time of the FP8 paths (e4m3 q, k, v quantised per tensor with quantize_fp8,
    bf16 o; fa_fwd_fp8: Q K^T in fp8, fa_fwd_fp8_pv: P V in fp8 as well) beside the 16-bit forward
    (fa_fwd) on the same configs, inputs resident in HBM: `reps` rotations through the three paths,
    each `warmup` launches and then HIP events around `iters` back-to-back launches, and the best
    rotation per path (so that a path measured while the clocks still ramp up is not penalised).
    Useful FLOPs are the forward's (4 D pairs B Hq)."""
    import torch

    fa = _pkg()
    ops = _mod("_ops")
    flops_mod = _mod("flops")
    dev = torch.device("cuda", 0)
    out = {}
    for name in names:
        cfg = CONFIGS[name]
        q, k, v, _ = make_inputs(cfg, dev)
        sc = 1.0 / math.sqrt(cfg["D"])
        (q8, qd), (k8, kd), (v8, vd) = (fa.quantize_fp8(t) for t in (q, k, v))
        calls = {"16bit": ops.FwdCall(q, k, v, cfg["W"], cfg["S"], sc),
                 "fp8": ops.Fp8FwdCall(q8, k8, v8, cfg["W"], cfg["S"], sc, (qd, kd, vd)),
                 "fp8_pv": ops.Fp8FwdCall(q8, k8, v8, cfg["W"], cfg["S"], sc, (qd, kd, vd), fp8_pv=True)}
        us = {}
        for _ in range(reps):
            for tag, call in calls.items():
                for _ in range(warmup):
                    call.run()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(iters):
                    call.run()
                e1.record()
                torch.cuda.synchronize()
                us[tag] = min(us.get(tag, float("inf")), e0.elapsed_time(e1) / iters * 1e3)
        wl = flops_mod.Workload(cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["L"], cfg["D"], cfg["W"], cfg["S"])
        f = wl.flops("fwd")
        out[name] = {"fwd_us_16bit": round(us["16bit"], 2), "fwd_us_fp8": round(us["fp8"], 2),
                     "fwd_us_fp8_pv": round(us["fp8_pv"], 2),
                     "tflops_16bit": round(f / us["16bit"] / 1e6, 1), "tflops_fp8": round(f / us["fp8"] / 1e6, 1),
                     "tflops_fp8_pv": round(f / us["fp8_pv"] / 1e6, 1),
                     "speedup": round(us["16bit"] / us["fp8"], 3), "speedup_pv": round(us["16bit"] / us["fp8_pv"], 3),
                     "dtype_16bit": cfg["dtype"]}
        del q, k, v, q8, k8, v8, calls
    return out


def sdpa_baseline(cfg, q, k, v, do, steps=10, warmup=3):
    """PyTorch-ROCm SDPA with a boolean mask, the reference's second baseline
    (pytorch_sdpa_attention, benchmark_backward_speed.py:57-65), fwd + autograd bwd on the GPU in
    the config dtype, timed with HIP events.  On this ROCm build scaled_dot_product_attention has
    no fused kernel for enable_gqa=True (it would fall back to the math path), so K/V are repeated
    to Hq heads inside the timed step (as the reference's repeat_kv does) and SDPA is held to the
    memory-efficient backend: it raises rather than fall back."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    flops_mod = _mod("flops")
    B, Hq, Hkv, L, D, W, S = (cfg[x] for x in ("B", "Hq", "Hkv", "L", "D", "W", "S"))
    G = Hq // Hkv
    pos = torch.arange(L, device=q.device)
    mask = (pos[None, :] <= pos[:, None]) & (((pos[:, None] - pos[None, :]) < W) | (pos[None, :] < S))
    qg, kg, vg = (t.detach().clone().requires_grad_() for t in (q, k, v))

    def step():
        qg.grad = kg.grad = vg.grad = None
        with sdpa_kernel([SDPBackend.EFFICIENT_ATTENTION]):
            o = F.scaled_dot_product_attention(qg, kg.repeat_interleave(G, 1), vg.repeat_interleave(G, 1),
                                               attn_mask=mask)
            o.backward(do)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    wl = flops_mod.Workload(B, Hq, Hkv, L, D, W, S)
    return {"value": round(wl.flops("fwdbwd") / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
            "peak_mem_gb": round(torch.cuda.max_memory_allocated() / 2 ** 30, 3),
            "backend": "torch SDPA, memory-efficient kernel, boolean [L, L] mask, K/V repeated to Hq heads",
            "steps": steps, "dtype": cfg["dtype"]}


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), else what platform reports."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(cfg, budget_s, fp32=False):
    """The reference's naive path (benchmark_backward_speed.py:68-85, restated in oracle/naive.py)
    on the host cores, in the config dtype (fp32 with `fp32`, on the same values), timed as the
    reference times its modes (benchmark_backward_speed.py:720-783): forward only (no autograd
    graph), forward + backward, and backward only (a forward, then backward() timed alone); one
    warm-up and three timed iterations per mode, median.  An iteration runs the naive path over a
    sample of whole KV groups of the same workload (every query head of a group with its K/V
    head), sized from the warm-up so that the whole measurement takes about `budget_s` seconds;
    times are scaled by (all KV groups / sample groups) to the full workload, and labelled so.
    Host memory: the rise of the process's peak resident set during the measurement."""
    import resource

    import torch

    from oracle import naive  # the CPU baseline leg

    flops_mod = _mod("flops")
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    B, Hq, Hkv, L, D, W, S = (cfg[x] for x in ("B", "Hq", "Hkv", "L", "D", "W", "S"))
    G = Hq // Hkv
    q, k, v, do = make_inputs(cfg, "cpu")
    if fp32:
        q, k, v, do = (x.float() for x in (q, k, v, do))
    dname = "fp32" if fp32 else cfg["dtype"]
    rss0 = resource.getrusage(resource.RUSAGE_SELF).ru_maxrss  # KiB
    all_groups = [(b, g) for g in range(Hkv) for b in range(B)]

    def slices(groups):
        return [(q[b:b + 1, g * G:(g + 1) * G], k[b:b + 1, g:g + 1], v[b:b + 1, g:g + 1], do[b:b + 1, g * G:(g + 1) * G])
                for b, g in groups]

    def fwd(groups):
        t0 = time.perf_counter()
        with torch.no_grad():
            for qs, ks, vs, _ in slices(groups):
                naive.naive_attention(qs, ks, vs, W, S)
        return time.perf_counter() - t0

    def fwdbwd(groups):
        t0 = time.perf_counter()
        for qs, ks, vs, ds in slices(groups):
            qg, kg, vg = (x.clone().requires_grad_() for x in (qs, ks, vs))
            naive.naive_attention(qg, kg, vg, W, S).backward(ds)
        return time.perf_counter() - t0

    def bwd(groups):
        total = 0.0
        for qs, ks, vs, ds in slices(groups):
            qg, kg, vg = (x.clone().requires_grad_() for x in (qs, ks, vs))
            o = naive.naive_attention(qg, kg, vg, W, S)
            t0 = time.perf_counter()
            o.backward(ds)
            total += time.perf_counter() - t0
        return total

    # warm-up on one group; it also sizes the sample (a mode's 3 iterations plus the others'
    # take about 8 fwd+bwd passes of the sample)
    t_one = fwdbwd(all_groups[:1])
    n = max(1, min(len(all_groups), int(budget_s / (8.0 * max(t_one, 1e-3)))))
    sample = all_groups[:n]
    modes = {}
    for name, fn in (("fwd", fwd), ("fwdbwd", fwdbwd), ("bwd", bwd)):
        fn(sample[:1])  # warm-up
        ts = sorted(fn(sample) for _ in range(3))
        modes[name] = ts[1] * len(all_groups) / n * 1e3  # median, scaled to the full workload (ms)
    rss1 = resource.getrusage(resource.RUSAGE_SELF).ru_maxrss
    pairs = flops_mod.allowed_pairs_per_head(L, W, S)
    flops = 14.0 * D * pairs * B * Hq
    scaled = n < len(all_groups)
    return {
        "value": flops / (modes["fwdbwd"] * 1e-3) / 1e12,
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{n} of the {len(all_groups)} KV groups of the workload ({n * G} query heads) per iteration, "
                  f"naive path in {dname} (dense scores, fp32 softmax, autograd backward), warm-up 1 + median of 3 "
                  f"per mode; times {'scaled x' + format(len(all_groups) / n, '.3g') + ' to the full workload (extrapolated)' if scaled else 'of the full workload'}",
        "fwd_ms": round(modes["fwd"], 2),
        "fwdbwd_ms": round(modes["fwdbwd"], 2),
        "bwd_ms": round(modes["bwd"], 2),
        "ms_full_workload_est": modes["fwdbwd"],
        "extrapolated": scaled,
        "max_rss_delta_mb": round((rss1 - rss0) / 1024.0, 1),
        "cpu": cpu_model(),
        "logical_cores": os.cpu_count(),
        "torch_threads": torch.get_num_threads(),
        "torch": torch.__version__,
        "dtype": dname,
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    # 100 warm-up steps: with 20, the GPU's clocks have not settled and the same steps time ~9%
    # slower; 200 timed steps still take well under a second.
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--kernel-iters", type=int, default=50)
    ap.add_argument("--clock-warm-s", type=float, default=0.2,
                    help="seconds of untimed fwd+bwd steps that bring the GPU to its working clocks first")
    ap.add_argument("--cpu-baseline-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-sdpa-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the packed-batch and fp8 entries of the c2 line (for per-kernel profiles of c2 alone)")
    ap.add_argument("--table", action="store_true", help="also time every BASELINE config (stderr)")
    ap.add_argument("--profile-launches", type=int, default=0, metavar="N",
                    help="only launch a 256 MiB copy and each kernel N times (for rocprofv3 --pmc runs)")
    ap.add_argument("--packed-only", action="store_true",
                    help="only time the packed batch (the line's `varlen` entry) and print it (for rocprofv3 kernel traces)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE={world}); this build has no "
              "multi-GPU path: attention shards with zero communication over batch and KV-head groups, so the "
              "per-GPU kernel is what --gpus 1 measures.", file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    fa = _pkg()
    if args.packed_only:
        print(json.dumps(varlen_measure(args.steps, args.warmup)), flush=True)
        return
    cfg = CONFIGS[args.config]
    dev = torch.device("cuda", 0)
    q, k, v, do = make_inputs(cfg, dev)
    if args.profile_launches:
        profile_launches(cfg, q, k, v, do, args.profile_launches)
        return
    acct = kernel_accounting(cfg)
    wl = _mod("flops").Workload(cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["L"], cfg["D"], cfg["W"], cfg["S"])

    # A GPU coming out of idle takes about 200 back-to-back steps (some 30 ms) to reach its working
    # clocks: measured from a cold start, c2 steps time 127 us at first and settle at 110 us.  So
    # the GPU first runs fwd+bwd steps for clock_warm_s before anything is timed (the per-kernel
    # timing, then the W untimed warm-up steps and the K timed ones).
    warm_steps = warm_clocks(fa, cfg, q, k, v, do, args.clock_warm_s)
    kus = time_kernels(cfg, q, k, v, do, iters=args.kernel_iters)
    t = time_steps(fa, cfg, q, k, v, do, args.steps, args.warmup)

    kernels = {}
    for name, us in kus.items():
        a = acct[name]
        ai = a["flops"] / a["bytes"]
        kernels[name] = dict(avg_us=round(us, 3), alg_bytes=a["bytes"], useful_flops=a["flops"],
                             gbs=round(a["bytes"] / us / 1e3, 1), tflops=round(a["flops"] / us / 1e6, 1),
                             bound="hbm" if ai < MFMA_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9) else "mfma")
    dom = max(kernels, key=lambda n: kernels[n]["avg_us"])
    dk = kernels[dom]
    if dk["bound"] == "hbm":
        achieved, peak, unit = dk["gbs"], HBM_PEAK_GBS, "GB/s"
    else:
        achieved, peak, unit = dk["tflops"], MFMA_PEAK_TFLOPS, "TFLOP/s"
    traffic, traffic_src = measured_traffic(args.config, dom)
    # the backward as one unit (the survey's figure: each tensor read or written once, delta fused):
    # its algorithmic bytes or FLOPs over the two backward kernels' summed time
    bwd_us = kernels["bwd_dq"]["avg_us"] + kernels["bwd_dkdv"]["avg_us"]
    bwd_bound = "hbm" if wl.flops("bwd") / wl.bytes("bwd") < MFMA_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9) else "mfma"
    bwd_ach = (wl.bytes("bwd") / bwd_us / 1e3) if bwd_bound == "hbm" else (wl.flops("bwd") / bwd_us / 1e6)
    roofline = {"kernel": dom, "bound": dk["bound"], "achieved": achieved, "peak": peak, "unit": unit,
                "frac": round(achieved / peak, 4), "traffic": traffic, "traffic_source": traffic_src,
                "avg_us": dk["avg_us"], "alg_bytes": dk["alg_bytes"],
                "fused_backward": {"kernels": ["bwd_dq", "bwd_dkdv"], "us": round(bwd_us, 3), "bound": bwd_bound,
                                   "alg_bytes": wl.bytes("bwd"), "useful_flops": wl.flops("bwd"),
                                   "achieved": round(bwd_ach, 1),
                                   "unit": "GB/s" if bwd_bound == "hbm" else "TFLOP/s",
                                   "frac": round(bwd_ach / (HBM_PEAK_GBS if bwd_bound == "hbm" else MFMA_PEAK_TFLOPS), 4)}}

    fb_flops = wl.flops("fwdbwd")
    value = fb_flops / (t["fwdbwd_ms"] * 1e-3) / 1e12
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t["fwdbwd_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic (seeded N(0,1) q, k, v, dO)",
        "config": {"workload": f"{args.config}: {cfg['name']}, fwd+bwd", "batch": cfg["B"], "heads_q": cfg["Hq"],
                   "heads_kv": cfg["Hkv"], "seq_len": cfg["L"], "head_dim": cfg["D"], "window": cfg["W"],
                   "sink": cfg["S"], "parallelism": "single GPU"},
        "fwd_ms": round(t["fwd_ms"], 4),
        "bwd_ms": round(t["bwd_ms"], 4),
        "bwd_event_ms": round(t["bwd_event_ms"], 4),
        "fwdbwd_event_ms": round(t["fwdbwd_event_ms"], 4),
        "fwdbwd_median_ms": round(t["fwdbwd_median_ms"], 4),
        "peak_mem_gb": round(t["peak_mem_gb"], 4),
        "fwdbwd_roofline_frac": round(wl.roofline_seconds("fwdbwd") / (t["fwdbwd_ms"] * 1e-3), 4),
        "modes": mode_figures(wl, t),
        "clock_warm_steps": warm_steps,
        "kernels": kernels,
        "roofline": roofline,
    }
    if not args.no_extras:
        line["graph_step"] = graph_step_measure(fa, cfg, q, k, v, do, args.steps)
    if args.config == "c2" and not args.no_extras:
        line["varlen"] = varlen_measure(args.steps, args.warmup)
        line["long_context"] = long_context_measure()
        line["shard_proxy"] = sp = shard_proxy_measure(args.steps, args.warmup)
        full = fb_flops / (sum(kt["avg_us"] for kt in line["kernels"].values()) * 1e-6) / 1e12
        sp["per_gpu_vs_full"] = round(sp["value"] / full, 3)  # device throughput, share vs full shape
        line["fp8_forward"] = fp8_forward_measure()
        # the README shape, whose autograd step is bound by host work: eager and graph-replayed
        c1 = CONFIGS["c1"]
        q1, k1, v1, do1 = make_inputs(c1, dev)
        warm_clocks(fa, c1, q1, k1, v1, do1, 0.1)
        t1 = time_steps(fa, c1, q1, k1, v1, do1, args.steps, args.warmup)
        line["c1_step"] = {"workload": "c1: " + c1["name"] + ", fwd+bwd", "eager_ms_per_step": round(t1["fwdbwd_ms"], 4),
                           "graph": graph_step_measure(fa, c1, q1, k1, v1, do1, args.steps)}
        del q1, k1, v1, do1
        # the reference's default cases, timed by its protocol (its published numbers are c1's)
        line["reference_cases"] = reference_cases_measure(fa, dev, args.steps, args.warmup)
        line["fp32_path"] = fp32_measure(fa, cfg, dev, 20, 5)
    if not args.no_sdpa_baseline:
        line["sdpa_baseline"] = sdpa_baseline(cfg, q, k, v, do)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(cfg, args.cpu_baseline_seconds)
        # the same path in fp32 (the reference times the config dtype; fp32 is reported beside it)
        f32 = cpu_baseline(cfg, args.cpu_baseline_seconds / 2, fp32=True)
        line["cpu_baseline"]["fp32"] = {k: f32[k] for k in ("value", "unit", "sample", "fwd_ms", "fwdbwd_ms", "bwd_ms",
                                                            "extrapolated", "max_rss_delta_mb")}
    if args.table:
        for name, c in CONFIGS.items():
            qq, kk, vv, dd = make_inputs(c, dev)
            tt = time_steps(fa, c, qq, kk, vv, dd, args.steps, args.warmup)
            w = _mod("flops").Workload(c["B"], c["Hq"], c["Hkv"], c["L"], c["D"], c["W"], c["S"])
            print(json.dumps({"config": name, **{k_: round(v_, 4) for k_, v_ in tt.items()},
                              "tflops": round(w.flops("fwdbwd") / (tt["fwdbwd_ms"] * 1e-3) / 1e12, 2),
                              "roofline_frac": round(w.roofline_seconds("fwdbwd") / (tt["fwdbwd_ms"] * 1e-3), 4)}),
                  file=sys.stderr, flush=True)
            del qq, kk, vv, dd
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
