"""GPU parity of the GPT-OSS integration: learned sink logits (fa_fwd_sinks / fa_bwd_sinks), the
[B, L, H, D] layout, and transformers' GptOssAttention running on the gfx950 kernels.

O, LSE, dQ, dK, dV use the tolerance of test_gpu_parity.py, with the oracle
naive.attention_fwd_bwd_sinks in float32: a = 2e-2 everywhere except the dK/dV rows of positional
sink keys (k < S), where for the small cases the low-precision naive path (transformers' eager
GPT-OSS attention restated, in the input dtype, on the CPU) sets a = max(2e-2, 2 * its error over
those rows).  The sink gradient of head h is a sum over every
row of the head, dsink = -sum P_sink * delta, so its bound scales with the size of that sum:
    |ours - ref| <= 2e-2 * (1 + sum over rows of |P_sink * delta|)
(or twice the naive path's error, if larger).
"""
import math

import pytest
import torch

from conftest import load_mod, load_pkg
from oracle import naive
from test_gpu_parity import BF, FP, assert_close, make_inputs, sink_rows

pytestmark = pytest.mark.gpu


def make_sinks(Hq, seed, scale=2.0, device="cuda"):
    g = torch.Generator().manual_seed(seed + 1000)
    # values exact in bf16, so the low-precision naive path (bf16 sink column) sees them unrounded
    return (scale * torch.randn(Hq, generator=g)).to(torch.bfloat16).float().to(device)


def naive_sinks_reference(q, k, v, sinks, do, W, S, scale):
    """transformers' eager GPT-OSS attention in the inputs' dtype on the CPU (positional sinks, if
    any, through an explicit mask)."""
    qc, kc, vc = (t.detach().cpu().clone().requires_grad_() for t in (q, k, v))
    sc = sinks.detach().cpu().to(q.dtype).clone().requires_grad_()
    G = q.shape[1] // k.shape[1]
    kr, vr = naive.expand_kv(kc, G), naive.expand_kv(vc, G)
    L = q.shape[2]
    s = torch.matmul(qc, kr.transpose(-1, -2).contiguous()) * scale
    s = s.masked_fill(~naive.allowed_mask(L, W, S), float("-inf"))
    col = sc.reshape(1, -1, 1, 1).expand(q.shape[0], -1, L, 1)
    logits = torch.cat([s, col], dim=-1)
    logits = logits - logits.max(dim=-1, keepdim=True).values
    p = torch.softmax(logits, dim=-1)[..., :-1]
    o = torch.matmul(p.to(vc.dtype), vr)
    o.backward(do.cpu())
    return o.detach(), qc.grad, kc.grad, vc.grad, sc.grad


def check_dsinks(got, ref, lse, o_ref, do, sinks, hs, naive_ds=None):
    delta = (do.float() * o_ref).sum(-1)
    terms = (torch.exp(sinks.float().view(1, -1, 1) - lse) * delta).abs().sum(dim=(0, 2))
    for h in hs:
        bound = 2e-2 * (1.0 + float(terms[h]))
        if naive_ds is not None:
            bound = max(bound, 2.0 * abs(float(naive_ds[h]) - float(ref[h])))
        err = abs(float(got[h]) - float(ref[h]))
        assert err <= bound, f"dsinks[{h}]: got {float(got[h]):.6g} ref {float(ref[h]):.6g} (bound {bound:.3g})"


def run_sinks_case(B, Hq, Hkv, L, D, W, S, dtype, seed=0, sink_scale=2.0, sinks=None, heads=None, with_naive=None):
    ops = load_mod("_ops")
    q, k, v, do = make_inputs(B, Hq, Hkv, L, D, dtype, seed)
    if sinks is None:
        sinks = make_sinks(Hq, seed, sink_scale)
    sc = 1.0 / math.sqrt(D)
    o, lse = ops.forward(q, k, v, W, S, sc, sinks=sinks)
    dq, dk, dv, ds = ops.backward(q, k, v, o, lse, do, W, S, sc, sinks=sinks)
    torch.cuda.synchronize()
    assert ds.dtype == torch.float32 and ds.shape == (Hq,)
    ro, rlse, rdq, rdk, rdv, rds = naive.attention_fwd_bwd_sinks(q, k, v, sinks, do, W, S, scale=sc,
                                                                 compute_dtype=torch.float32, row_chunk=2048,
                                                                 heads=heads)
    if with_naive is None:
        with_naive = heads is None and B * Hq * L * L <= (1 << 24)
    nv = naive_sinks_reference(q, k, v, sinks, do, W, S, sc) if with_naive else (None,) * 5
    G = Hq // Hkv
    hs = list(range(Hq)) if heads is None else list(heads)
    sel = lambda t, idx: None if t is None else t[:, idx]
    assert_close("O", o[:, hs], ro[:, hs])
    assert_close("LSE", lse[:, hs], rlse[:, hs])
    assert_close("dQ", dq[:, hs], rdq[:, hs])
    groups = [g for g in range(Hkv) if all(h in hs for h in range(g * G, (g + 1) * G))]
    assert_close("dK", dk[:, groups], rdk[:, groups], sel(nv[2], groups), sink_rows(L, S))
    assert_close("dV", dv[:, groups], rdv[:, groups], sel(nv[3], groups), sink_rows(L, S))
    check_dsinks(ds, rds, rlse, ro, do, sinks, hs, nv[4])
    return o, lse, dq, dk, dv, ds


SINK_CASES = [
    pytest.param(1, 8, 1, 300, 64, 128, 0, BF, id="gpt-oss-sliding-G8"),
    pytest.param(2, 4, 1, 200, 64, 200, 0, BF, id="gpt-oss-full-B2"),
    pytest.param(1, 4, 2, 150, 32, 16, 4, FP, id="learned-plus-positional-D32"),
    pytest.param(1, 4, 2, 160, 128, 40, 0, FP, id="D128-G2"),
    pytest.param(1, 2, 1, 33, 16, 5, 0, BF, id="D16-L33"),
    pytest.param(1, 2, 2, 1, 64, 4, 0, BF, id="L1"),
    pytest.param(1, 16, 16, 100, 64, 1, 0, BF, id="W1-G1"),
]


@pytest.mark.parametrize("B,Hq,Hkv,L,D,W,S,dtype", SINK_CASES)
def test_learned_sinks_parity(gpu, B, Hq, Hkv, L, D, W, S, dtype):
    run_sinks_case(B, Hq, Hkv, L, D, W, S, dtype, seed=L + D)


def _random_sink_cases(n=16, seed=4242):
    """Learned sink logits on shapes drawn from a fixed seed: every head dim, groups 1-8, lengths
    1-600, windows from 1 to past L with and without positional sinks, logits of scale 0.5-8."""
    import random

    rng = random.Random(seed)
    cases = []
    while len(cases) < n:
        D = rng.choice([16, 32, 64, 128])
        Hkv, G, B = rng.choice([1, 2, 4]), rng.choice([1, 2, 3, 8]), rng.choice([1, 2])
        L = rng.choice([rng.randint(1, 64), rng.randint(65, 600)])
        W = rng.choice([1, rng.randint(2, 200), L, L + 7])
        S = rng.choice([0, 0, rng.randint(1, 40)])
        if B * Hkv * G * L * L > (1 << 23):
            continue
        dtype = rng.choice([BF, FP])
        sink_scale = rng.choice([0.5, 2.0, 8.0])
        cases.append(pytest.param(B, Hkv * G, Hkv, L, D, W, S, dtype, sink_scale, len(cases),
                                  id=f"RS{len(cases)}-B{B}-H{Hkv * G}x{Hkv}-L{L}-D{D}-W{W}-S{S}-x{sink_scale}"))
    return cases


@pytest.mark.parametrize("B,Hq,Hkv,L,D,W,S,dtype,sink_scale,seed", _random_sink_cases())
def test_learned_sinks_random_shapes(gpu, B, Hq, Hkv, L, D, W, S, dtype, sink_scale, seed):
    print(f"random sinks case B={B} Hq={Hq} Hkv={Hkv} L={L} D={D} W={W} S={S} {dtype} x{sink_scale}", flush=True)
    run_sinks_case(B, Hq, Hkv, L, D, W, S, dtype, seed=200 + seed, sink_scale=sink_scale)


def test_learned_sinks_extreme_logits(gpu):
    # a dominant sink (most of the mass on the sink), an irrelevant one, and a zero one
    sinks = torch.tensor([8.0, -40.0, 0.0, 3.0], device="cuda")
    run_sinks_case(1, 4, 2, 130, 64, 32, 0, BF, seed=3, sinks=sinks)


def test_learned_sinks_bf16_parameter_and_autograd(gpu, fa):
    q, k, v, do = make_inputs(1, 8, 2, 96, 64, BF, 7)
    sinks = make_sinks(8, 7).to(BF).requires_grad_()
    qq, kk, vv = (t.clone().requires_grad_() for t in (q, k, v))
    o = fa.FlashSWDAWithLearnedSinks.apply(qq, kk, vv, sinks, 32)
    o.backward(do)
    assert sinks.grad.dtype == BF and sinks.grad.shape == (8,)
    ro, _, rdq, rdk, rdv, rds = naive.attention_fwd_bwd_sinks(q, k, v, sinks.detach(), do, 32, 0,
                                                              compute_dtype=torch.float32)
    assert_close("O", o.detach(), ro)
    assert_close("dQ", qq.grad, rdq)
    assert_close("dK", kk.grad, rdk)
    assert_close("dV", vv.grad, rdv)
    assert torch.allclose(sinks.grad.float(), rds, atol=5e-2, rtol=2e-2)


def test_learned_sinks_deterministic(gpu):
    ops = load_mod("_ops")
    q, k, v, do = make_inputs(1, 8, 1, 700, 64, BF, 11)
    sinks = make_sinks(8, 11)
    outs = []
    for _ in range(2):
        o, lse = ops.forward(q, k, v, 128, 0, 0.125, sinks=sinks)
        outs.append((o, lse) + tuple(ops.backward(q, k, v, o, lse, do, 128, 0, 0.125, sinks=sinks)))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_learned_sinks_minus_inf_equals_plain(gpu):
    ops = load_mod("_ops")
    q, k, v, do = make_inputs(1, 4, 2, 200, 64, BF, 5)
    ninf = torch.full((4,), float("-inf"), device="cuda")
    o1, l1 = ops.forward(q, k, v, 64, 4, 0.125)
    o2, l2 = ops.forward(q, k, v, 64, 4, 0.125, sinks=ninf)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    g1 = ops.backward(q, k, v, o1, l1, do, 64, 4, 0.125)
    g2 = ops.backward(q, k, v, o2, l2, do, 64, 4, 0.125, sinks=ninf)
    for a, b in zip(g1, g2[:3]):
        assert torch.equal(a, b)
    assert torch.all(g2[3] == 0)


def test_gpt_oss_layer_full_size_learned_sinks(gpu):
    # c2's shape as a GPT-OSS sliding layer (learned sinks, no positional sinks), on one KV group
    run_sinks_case(1, 64, 8, 4096, 64, 128, 0, BF, seed=2, heads=range(8), with_naive=False)


def test_blhd_layout_reads_and_writes_in_place(gpu, fa):
    B, L, Hq, Hkv, D = 2, 130, 8, 2, 64
    g = torch.Generator().manual_seed(4)
    q = torch.randn(B, L, Hq, D, generator=g).to(BF).cuda().requires_grad_()
    k = torch.randn(B, L, Hkv, D, generator=g).to(BF).cuda().requires_grad_()
    v = torch.randn(B, L, Hkv, D, generator=g).to(BF).cuda().requires_grad_()
    do = torch.randn(B, L, Hq, D, generator=g).to(BF).cuda()
    sinks = make_sinks(Hq, 4).requires_grad_()
    o = fa.attention(q, k, v, window_size=32, sinks=sinks, layout="blhd")
    assert o.shape == (B, L, Hq, D) and o.is_contiguous()
    o.backward(do)
    assert q.grad.is_contiguous() and k.grad.is_contiguous()
    # the same computation on [B, H, L, D] copies gives bitwise the same numbers
    q2, k2, v2 = (t.detach().transpose(1, 2).contiguous().requires_grad_() for t in (q, k, v))
    s2 = sinks.detach().clone().requires_grad_()
    o2 = fa.attention(q2, k2, v2, window_size=32, sinks=s2)
    o2.backward(do.transpose(1, 2))
    assert torch.equal(o.transpose(1, 2), o2)
    assert torch.equal(q.grad.transpose(1, 2), q2.grad)
    assert torch.equal(k.grad.transpose(1, 2), k2.grad)
    assert torch.equal(v.grad.transpose(1, 2), v2.grad)
    assert torch.equal(sinks.grad, s2.grad)


@pytest.mark.parametrize("layer_idx", [0, 1], ids=["sliding", "full"])
def test_transformers_gpt_oss_attention_module(gpu, fa, layer_idx):
    mod = pytest.importorskip("transformers.models.gpt_oss.modeling_gpt_oss")
    from transformers import GptOssConfig

    name = fa.register_transformers("fa_gfx950")
    cfg = dict(hidden_size=256, num_attention_heads=8, num_key_value_heads=2, head_dim=64, sliding_window=24,
               num_hidden_layers=2, layer_types=["sliding_attention", "full_attention"], attention_bias=True,
               vocab_size=128, intermediate_size=64, num_local_experts=4)
    ref_cfg, our_cfg = GptOssConfig(**cfg), GptOssConfig(**cfg)
    ref_cfg._attn_implementation = "eager"
    our_cfg._attn_implementation = name
    torch.manual_seed(0)
    ref = mod.GptOssAttention(ref_cfg, layer_idx).cuda()
    with torch.no_grad():
        for p in ref.parameters():
            p.copy_((0.05 * torch.randn_like(p)).to(BF).float())  # weights exact in bf16
        ref.sinks.copy_(torch.randn(8).to(BF).float())
    ours = mod.GptOssAttention(our_cfg, layer_idx).cuda()
    ours.load_state_dict(ref.state_dict())
    ours = ours.to(BF)
    B, L = 2, 96
    x = torch.randn(B, L, 256, device="cuda").to(BF)
    pos = torch.arange(L, device="cuda").expand(B, L)
    rope = mod.GptOssRotaryEmbedding(ref_cfg).cuda()
    W = ref.sliding_window if ref.sliding_window is not None else L
    add = torch.zeros(L, L, device="cuda").masked_fill(~naive.allowed_mask(L, W, 0, device="cuda"), float("-inf"))
    xr = x.float().requires_grad_()
    yr, _ = ref(xr, rope(xr, pos), add.view(1, 1, L, L))
    xo = x.clone().requires_grad_()
    yo, _ = ours(xo, rope(xo, pos), None)
    g = torch.randn_like(yr)
    yr.backward(g)
    yo.backward(g.to(BF))
    rel = lambda a, b: float((a.detach().float() - b.detach().float()).norm() / b.detach().float().norm())
    assert rel(yo, yr) < 1e-2
    assert rel(xo.grad, xr.grad) < 2e-2
    assert rel(ours.sinks.grad, ref.sinks.grad) < 3e-2
    assert rel(ours.q_proj.weight.grad, ref.q_proj.weight.grad) < 2e-2
    assert rel(ours.k_proj.weight.grad, ref.k_proj.weight.grad) < 2e-2


@pytest.mark.parametrize("layer_idx", [0, 1], ids=["sliding", "full"])
def test_transformers_gpt_oss_attention_padded_batch(gpu, fa, layer_idx):
    """A padded batch -- row 0 right-padded, row 1 left-padded -- through the registered attention
    function, with the 2-D padding mask the flash-attention mask function hands over, equals
    transformers' eager GptOssAttention run on each sequence alone (float32, positions from 0):
    outputs and input gradients on the tokens, and the parameter gradients of the attention path.
    Padded positions come back as zeros and receive no gradient."""
    mod = pytest.importorskip("transformers.models.gpt_oss.modeling_gpt_oss")
    from transformers import GptOssConfig

    name = fa.register_transformers("fa_gfx950")
    cfg = dict(hidden_size=256, num_attention_heads=8, num_key_value_heads=2, head_dim=64, sliding_window=24,
               num_hidden_layers=2, layer_types=["sliding_attention", "full_attention"], attention_bias=True,
               vocab_size=128, intermediate_size=64, num_local_experts=4)
    ref_cfg, our_cfg = GptOssConfig(**cfg), GptOssConfig(**cfg)
    ref_cfg._attn_implementation = "eager"
    our_cfg._attn_implementation = name
    torch.manual_seed(1)
    ref = mod.GptOssAttention(ref_cfg, layer_idx).cuda()
    with torch.no_grad():
        for p in ref.parameters():
            p.copy_((0.05 * torch.randn_like(p)).to(BF).float())
        ref.sinks.copy_(torch.randn(8).to(BF).float())
    ours = mod.GptOssAttention(our_cfg, layer_idx).cuda()
    ours.load_state_dict(ref.state_dict())
    ours = ours.to(BF)
    rope = mod.GptOssRotaryEmbedding(ref_cfg).cuda()
    B, L = 2, 80
    mask = torch.zeros(B, L, dtype=torch.bool, device="cuda")
    mask[0, :60] = True   # right padding
    mask[1, 13:] = True   # left padding
    x = torch.randn(B, L, 256, device="cuda").to(BF)
    g = torch.randn(B, L, 256, device="cuda")
    g[~mask] = 0
    pos = (mask.long().cumsum(-1) - 1).clamp(min=0)

    xo = x.clone().requires_grad_()
    yo, _ = ours(xo, rope(xo, pos), mask)
    yo.backward(g.to(BF))

    yr = torch.zeros(B, L, 256, device="cuda")
    xr_grad = torch.zeros(B, L, 256, device="cuda")
    for b in range(B):
        sel = mask[b]
        n = int(sel.sum())
        xb = x[b:b + 1, sel].float().requires_grad_()
        pb = torch.arange(n, device="cuda").unsqueeze(0)
        W = ref.sliding_window if ref.sliding_window is not None else n
        add = torch.zeros(n, n, device="cuda").masked_fill(~naive.allowed_mask(n, W, 0, device="cuda"), float("-inf"))
        yb, _ = ref(xb, rope(xb, pb), add.view(1, 1, n, n))
        yb.backward(g[b:b + 1, sel])
        yr[b, sel] = yb.detach()[0]
        xr_grad[b, sel] = xb.grad[0]

    rel = lambda a, b: float((a.detach().float() - b.detach().float()).norm() / b.detach().float().norm())
    assert rel(yo[mask], yr[mask]) < 1e-2
    assert rel(xo.grad[mask], xr_grad[mask]) < 2e-2
    assert float(xo.grad[~mask].abs().max()) == 0.0
    assert rel(ours.sinks.grad, ref.sinks.grad) < 3e-2
    assert rel(ours.q_proj.weight.grad, ref.q_proj.weight.grad) < 2e-2
    assert rel(ours.k_proj.weight.grad, ref.k_proj.weight.grad) < 2e-2
    assert rel(ours.v_proj.weight.grad, ref.v_proj.weight.grad) < 2e-2


def _gpt_oss_pair(fa, layer_idx, seed):
    """An eager float32 GptOssAttention and the same weights in bf16 on the registered gfx950
    attention function."""
    mod = pytest.importorskip("transformers.models.gpt_oss.modeling_gpt_oss")
    from transformers import GptOssConfig

    name = fa.register_transformers("fa_gfx950")
    cfg = dict(hidden_size=256, num_attention_heads=8, num_key_value_heads=2, head_dim=64, sliding_window=24,
               num_hidden_layers=2, layer_types=["sliding_attention", "full_attention"], attention_bias=True,
               vocab_size=128, intermediate_size=64, num_local_experts=4)
    ref_cfg, our_cfg = GptOssConfig(**cfg), GptOssConfig(**cfg)
    ref_cfg._attn_implementation = "eager"
    our_cfg._attn_implementation = name
    torch.manual_seed(seed)
    ref = mod.GptOssAttention(ref_cfg, layer_idx).cuda()
    with torch.no_grad():
        for p in ref.parameters():
            p.copy_((0.05 * torch.randn_like(p)).to(BF).float())
        ref.sinks.copy_(torch.randn(8).to(BF).float())
    ours = mod.GptOssAttention(our_cfg, layer_idx).cuda()
    ours.load_state_dict(ref.state_dict())
    return mod, ref, ours.to(BF), mod.GptOssRotaryEmbedding(ref_cfg).cuda()


@pytest.mark.parametrize("layer_idx", [0, 1], ids=["sliding", "full"])
def test_transformers_gpt_oss_packed_position_ids(gpu, fa, layer_idx):
    """Padding-free finetuning: three sequences packed into one row, no mask, position ids that
    restart at each sequence.  Equals the eager module run on each sequence alone -- no token
    attends across a sequence boundary."""
    mod, ref, ours, rope = _gpt_oss_pair(fa, layer_idx, seed=2)
    lens = [40, 17, 35]
    L = sum(lens)
    pos = torch.cat([torch.arange(n) for n in lens]).unsqueeze(0).cuda()
    x = torch.randn(1, L, 256, device="cuda").to(BF)
    g = torch.randn(1, L, 256, device="cuda")
    xo = x.clone().requires_grad_()
    yo, _ = ours(xo, rope(xo, pos), None, position_ids=pos)
    yo.backward(g.to(BF))
    yr = torch.zeros(1, L, 256, device="cuda")
    xr_grad = torch.zeros(1, L, 256, device="cuda")
    lo = 0
    for n in lens:
        xb = x[:, lo:lo + n].float().requires_grad_()
        pb = torch.arange(n, device="cuda").unsqueeze(0)
        W = ref.sliding_window if ref.sliding_window is not None else n
        add = torch.zeros(n, n, device="cuda").masked_fill(~naive.allowed_mask(n, W, 0, device="cuda"), float("-inf"))
        yb, _ = ref(xb, rope(xb, pb), add.view(1, 1, n, n))
        yb.backward(g[:, lo:lo + n])
        yr[:, lo:lo + n] = yb.detach()
        xr_grad[:, lo:lo + n] = xb.grad
        lo += n
    rel = lambda a, b: float((a.detach().float() - b.detach().float()).norm() / b.detach().float().norm())
    assert rel(yo, yr) < 1e-2
    assert rel(xo.grad, xr_grad) < 2e-2
    assert rel(ours.sinks.grad, ref.sinks.grad) < 3e-2
    assert rel(ours.q_proj.weight.grad, ref.q_proj.weight.grad) < 2e-2


def test_padded_batch_later_layers_do_not_synchronise(gpu, fa):
    """The host reads a padded batch's mask once (the first attention layer); the model's other
    layers reuse what it found.  Later layers run with torch's sync debug mode set to "error"
    (any device-to-host synchronisation raises) and give the same result as the first."""
    mod, _, ours, rope = _gpt_oss_pair(fa, 0, seed=3)
    B, L = 2, 80
    mask = torch.zeros(B, L, dtype=torch.bool, device="cuda")
    mask[0, :60] = True
    mask[1, 13:] = True
    pos = (mask.long().cumsum(-1) - 1).clamp(min=0)
    x = torch.randn(B, L, 256, device="cuda").to(BF)
    pe = rope(x, pos)
    y1, _ = ours(x, pe, mask)  # first layer: reads the mask
    torch.cuda.synchronize()
    prev = torch.cuda.get_sync_debug_mode()
    torch.cuda.set_sync_debug_mode("error")
    try:
        outs = [ours(x, pe, mask)[0] for _ in range(3)]  # "later layers": same mask tensor
    finally:
        torch.cuda.set_sync_debug_mode(prev)
    torch.cuda.synchronize()
    for y in outs:
        assert torch.equal(y, y1)
    # and a new batch (another mask tensor) is read again
    mask2 = mask.clone()
    mask2[0, 60:70] = True
    y3, _ = ours(x, pe, mask2)
    assert not torch.equal(y3, y1)
