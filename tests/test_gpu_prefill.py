"""GPU parity of the MFMA causal prefill attention (with the prologue writing the cache first).

Bars: bf16 output within max-abs 2e-2 / mean-abs 2e-3 of the reference's bf16
SDPA (torch on CPU); fp32 output within max-abs 1e-4 of exact fp64 causal
attention over the same bf16 q/K/V (oracle/exact.py causal_attn_fp64), the
fp32 yardstick for this path.  The bf16 output rounds the probabilities to
bf16 before the second matrix product (and its row sums add the rounded
values); the fp32 output feeds them as bf16 high + low parts.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import exact, ref
from solort_amd import ops
from solort_amd import workloads as wl

pytestmark = pytest.mark.gpu
HD = 128
F32_MAX = 1e-4


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _prefill(gpu, T, shape=wl.QWEN3_4B, seed_T=None):
    """Prologue + prefill on the GPU for a seeded prompt; returns (q, kc, vc, out_bf16, out_f32, case)."""
    case = wl.prefill_case(T, layers=1)
    nh, nkv = shape.nh, shape.nkv
    qkv = case.qkv[0]
    if shape is not wl.QWEN3_4B:  # other head counts: draw a prompt of that width
        g = torch.Generator().manual_seed(2000 + T)
        qkv = torch.randn(T, shape.qkv_width, generator=g).to(torch.bfloat16)
    dev = gpu
    kc = torch.zeros(case.max_len, nkv, HD, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    q = torch.empty(T, nh, HD, dtype=torch.bfloat16, device=dev)
    ops.qknorm_rope_kvwrite(qkv.to(dev), case.qn_w[0].to(dev), case.kn_w[0].to(dev), wl.EPS,
                            ops.inv_freq(HD, wl.THETA, dev), None, q, kc, vc, nh, nkv)
    out = torch.empty(T, nh * HD, dtype=torch.bfloat16, device=dev)
    out32 = torch.empty(T, nh * HD, dtype=torch.float32, device=dev)
    ops.prefill_attn(q, kc, vc, shape.scale, out)
    ops.prefill_attn(q, kc, vc, shape.scale, out32)
    torch.cuda.synchronize()
    return q, kc, vc, out, out32, qkv, case


@pytest.mark.parametrize("T", [128, 512, 1024, 1, 17, 100, 1000])
def test_prefill_qwen3_4b(gpu, T):
    sh = wl.QWEN3_4B
    _say(f"[prefill {sh.name} T={T}]")
    q, kc, vc, out, out32, qkv, case = _prefill(gpu, T)
    # reference ops on the CPU: prologue + causal SDPA with repeat_interleave, in bf16
    cos, sin = ops.rope_tables(case.max_len, HD, wl.THETA, gpu)
    c = torch.cat([cos.cpu()[:T]] * 2, -1)
    s = torch.cat([sin.cpu()[:T]] * 2, -1)
    qr, kr, vr = ref.prologue(qkv, case.qn_w[0], case.kn_w[0], wl.EPS, c, s, sh.nh, sh.nkv)
    want = ref.prefill_attn(qr, kr, vr, sh.scale)
    d = (out.float().cpu() - want.float()).abs()
    _say(f"  bf16 vs reference ops: max-abs {d.max().item():.3e} mean-abs {d.mean().item():.3e}")
    assert d.max().item() <= 2e-2 and d.mean().item() <= 2e-3
    # fp32 output against exact attention, per head
    qg = q.float().cpu().numpy()
    kg = kc.float().cpu().numpy()[:T]
    vg = vc.float().cpu().numpy()[:T]
    o32 = out32.cpu().numpy().reshape(T, sh.nh, HD)
    worst, total = 0.0, 0.0
    for h in range(sh.nh):
        kvh = h // sh.group
        e = np.abs(o32[:, h] - exact.causal_attn_fp64(qg[:, h], kg[:, kvh], vg[:, kvh], sh.scale))
        worst = max(worst, float(e.max()))
        total += float(e.sum())
    _say(f"  fp32 vs exact fp64: max-abs {worst:.3e} mean-abs {total / o32.size:.3e}")
    assert worst <= F32_MAX
    # the bf16 output's extra error is the bf16 rounding of p
    d = (out.float() - out32).abs()
    assert d.max().item() <= 2e-2 and d.mean().item() <= 2e-3


def test_prefill_row0_and_last_row_pins(gpu):
    """Row 0 attends only key 0 (output = V[0] per query group); the last row equals single-token decode
    over the same cache at position T-1."""
    sh = wl.QWEN3_4B
    T = 300
    q, kc, vc, out, out32, qkv, case = _prefill(gpu, T)
    o = out32.reshape(T, sh.nh, HD)
    v0 = vc[0].float().repeat_interleave(sh.group, 0)
    assert torch.allclose(o[0], v0, atol=1e-6, rtol=0)
    ws = ops.attn_workspace(1, sh.nh, sh.nkv, 8, gpu)
    dec = torch.empty(1, sh.nh * HD, dtype=torch.float32, device=gpu)
    pos = torch.tensor([T - 1], dtype=torch.long, device=gpu)
    ops.decode_attn(q[T - 1:T].contiguous(), kc, vc, pos, 512, sh.scale, ws, 8, dec)
    torch.cuda.synchronize()
    # both keep ~16 bits of every probability in their fp32 outputs
    assert torch.allclose(o[T - 1], dec.reshape(sh.nh, HD), atol=F32_MAX, rtol=0)


@pytest.mark.parametrize("shape", [wl.QWEN3_0_6B, wl.AttnShape("g1", 8, 8, 1), wl.AttnShape("g8", 16, 2, 1)],
                         ids=["g2", "g1", "g8"])
def test_prefill_other_groups(gpu, shape):
    T = 200
    _say(f"[prefill {shape.name} T={T}]")
    q, kc, vc, out, out32, qkv, case = _prefill(gpu, T, shape)
    qg = q.float().cpu().numpy()
    kg = kc.float().cpu().numpy()[:T]
    vg = vc.float().cpu().numpy()[:T]
    o32 = out32.cpu().numpy().reshape(T, shape.nh, HD)
    for h in range(shape.nh):
        kvh = h // shape.group
        e = np.abs(o32[:, h] - exact.causal_attn_fp64(qg[:, h], kg[:, kvh], vg[:, kvh], shape.scale))
        assert e.max() <= F32_MAX, (h, e.max())


@pytest.mark.parametrize("T,shape", [(1, wl.QWEN3_4B), (17, wl.QWEN3_4B), (128, wl.QWEN3_4B), (333, wl.QWEN3_4B),
                                     (1024, wl.QWEN3_4B), (200, wl.QWEN3_0_6B), (150, wl.AttnShape("g1", 8, 8, 1)),
                                     (131, wl.AttnShape("g8", 16, 2, 1))],
                         ids=["4b-1", "4b-17", "4b-128", "4b-333", "4b-1024", "g2-200", "g1-150", "g8-131"])
def test_prefill_layer_equals_prologue_then_attention(gpu, T, shape):
    """solort_prefill_layer (K/V prologue + attention normalising q itself) writes the same cache
    rows and the same outputs, bit for bit, as solort_qknorm_rope_kvwrite_cs followed by
    solort_prefill_attn on a materialised q, in bf16 and fp32."""
    _say(f"[prefill_layer {shape.name} T={T}]")
    case = wl.prefill_case(T, layers=1)
    nh, nkv = shape.nh, shape.nkv
    g = torch.Generator().manual_seed(3000 + T)
    qkv = (torch.randn(T, (nh + 2 * nkv) * HD, generator=g) * 2).to(torch.bfloat16).to(gpu)
    qn_w, kn_w = case.qn_w[0].to(gpu), case.kn_w[0].to(gpu)
    inv_f = ops.inv_freq(HD, wl.THETA, gpu)
    cs = ops.rope_rows(inv_f, torch.zeros(1, dtype=torch.long, device=gpu), T)
    kc1 = torch.full((case.max_len, nkv, HD), 7.0, dtype=torch.bfloat16, device=gpu)
    vc1 = kc1.clone()
    kc2, vc2 = kc1.clone(), kc1.clone()
    q = torch.empty(T, nh, HD, dtype=torch.bfloat16, device=gpu)
    for dt in (torch.bfloat16, torch.float32):
        o1 = torch.empty(T, nh * HD, dtype=dt, device=gpu)
        o2 = torch.empty_like(o1)
        ops.qknorm_rope_kvwrite_cs(qkv, qn_w, kn_w, wl.EPS, cs, None, q, kc1, vc1, nh, nkv)
        ops.prefill_attn(q, kc1, vc1, shape.scale, o1)
        ops.prefill_layer(qkv, qn_w, kn_w, wl.EPS, cs, kc2, vc2, shape.scale, o2, nh, nkv)
        torch.cuda.synchronize()
        assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
        assert torch.equal(o1, o2), (dt, (o1.float() - o2.float()).abs().max().item())
    assert torch.all(kc2[T:] == 7.0)  # rows past the prompt untouched
