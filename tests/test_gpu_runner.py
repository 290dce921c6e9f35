"""The graph runner: captured decode/verify steps replayed at several positions
equal eager launches of the same kernels and the CPU oracle, replay after
replay, with eager work and synchronisations between replays."""
from __future__ import annotations

import sys

import pytest
import torch

from oracle import ref
from solort_amd import ops
from solort_amd import workloads as wl
from solort_amd.runner import GraphQwen3Attention, verify_bound, verify_splits

pytestmark = pytest.mark.gpu
HD = 128


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _make(gpu, layers=3, max_len=1024, k1=5):
    sh = wl.QWEN3_4B
    g = torch.Generator().manual_seed(77)
    qn = (1 + 0.1 * torch.randn(layers, HD, generator=g)).to(torch.bfloat16)
    kn = (1 + 0.1 * torch.randn(layers, HD, generator=g)).to(torch.bfloat16)
    r = GraphQwen3Attention(sh.nh, sh.nkv, layers, max_len, qn, kn, device=gpu, verify_tokens=k1)
    kc = torch.randn(layers, max_len, sh.nkv, HD, generator=g).to(torch.bfloat16)
    vc = torch.randn(layers, max_len, sh.nkv, HD, generator=g).to(torch.bfloat16)
    r.kc.copy_(kc)
    r.vc.copy_(vc)
    return r, g, sh


def test_bucket_routing_matches_reference_rule(gpu):
    r, _, _ = _make(gpu, layers=1, max_len=1024)
    assert r.buckets == [128, 256, 512, 1024]
    assert [r._bucket_for(p) for p in (0, 127, 128, 500, 1023)] == [128, 128, 256, 512, 1024]
    r2, _, _ = _make(gpu, layers=1, max_len=5000)
    assert r2.buckets == [128, 256, 512, 1024, 2048, 4096, 5000]
    with pytest.raises(RuntimeError):
        r._bucket_for(1024)


def test_decode_graph_replays_match_eager_and_oracle(gpu):
    r, g, sh = _make(gpu)
    eager_kc, eager_vc = r.kc.clone(), r.vc.clone()
    cpu_kc, cpu_vc = r.kc.cpu(), r.vc.cpu()
    cos_t, sin_t = ops.rope_tables(r.max_len, HD, wl.THETA, gpu)
    cos_cpu, sin_cpu = cos_t.cpu(), sin_t.cpu()
    q = torch.empty(1, sh.nh, HD, dtype=torch.bfloat16, device=gpu)
    ws = ops.attn_workspace(1, sh.nh, sh.nkv, 32, gpu)
    # larger buckets before smaller ones exercise one workspace shared by different split counts
    for step, pos in enumerate((5, 100, 127, 128, 300, 777, 1023, 200, 3, 1000)):
        _say(f"[decode replay step={step} pos={pos}]")
        qkv = torch.randn(r.L, 1, r.width, generator=g).to(torch.bfloat16)
        logits = torch.randn(1, wl.VOCAB, generator=g)
        tok = r.decode_argmax(qkv.to(gpu), pos, logits.to(gpu)).clone()
        ctx = r.ctx_dec
        # eager launches of the same kernels on a separate copy of the cache
        bound = r._bucket_for(pos)
        p = torch.tensor([pos], dtype=torch.long, device=gpu)
        out = torch.empty(r.L, 1, sh.nh * HD, dtype=torch.bfloat16, device=gpu)
        for li in range(r.L):
            ops.qknorm_rope_kvwrite(qkv[li].to(gpu), r.qn_w[li], r.kn_w[li], r.eps, r.inv_freq, p, q,
                                    eager_kc[li], eager_vc[li], sh.nh, sh.nkv)
            ops.decode_attn(q, eager_kc[li], eager_vc[li], p, bound, r.scale, ws, 32, out[li])
        torch.cuda.synchronize()
        assert torch.equal(r.kc, eager_kc) and torch.equal(r.vc, eager_vc)
        assert torch.allclose(ctx.float(), out.float(), atol=2e-3, rtol=0)
        assert tok.item() == int(logits.argmax())
        # oracle on CPU for the first layer
        c = torch.cat([cos_cpu[pos:pos + 1]] * 2, -1)
        s = torch.cat([sin_cpu[pos:pos + 1]] * 2, -1)
        qq, kk, vv = ref.prologue(qkv[0], r.qn_w[0].cpu(), r.kn_w[0].cpu(), r.eps, c, s, sh.nh, sh.nkv)
        ref.write_kv(cpu_kc[0], cpu_vc[0], kk, vv, pos)
        want = ref.decode_attn(qq, cpu_kc[0], cpu_vc[0], pos, bound, r.scale)
        d = (ctx[0].float().cpu() - want.float()).abs()
        assert d.max() <= 2e-2 and d.mean() <= 2e-3
        for li in range(1, r.L):  # keep the CPU cache in step for the later positions
            c2, k2, v2 = ref.prologue(qkv[li], r.qn_w[li].cpu(), r.kn_w[li].cpu(), r.eps, c, s, sh.nh, sh.nkv)
            ref.write_kv(cpu_kc[li], cpu_vc[li], k2, v2, pos)
        # eager work between replays
        _ = (torch.randn(1000, 1000, device=gpu) @ torch.randn(1000, 1000, device=gpu)).sum().item()
    assert sorted(r._graphs) == [128, 256, 512, 1024]


def test_verify_graph_replays_match_eager(gpu):
    r, g, sh = _make(gpu, layers=2, max_len=4096, k1=5)
    eager_kc, eager_vc = r.kc.clone(), r.vc.clone()
    q = torch.empty(5, sh.nh, HD, dtype=torch.bfloat16, device=gpu)
    for rep, pos0 in enumerate((2048, 17, 4091, 2048, 100)):
        bound = verify_bound(pos0 + 4, r.buckets)  # 2560, 128, 4096, 2560, 128
        ns = verify_splits(bound, sh.nkv)
        ws = ops.attn_workspace(5, sh.nh, sh.nkv, ns, gpu)
        _say(f"[verify replay pos0={pos0} bound={bound}]")
        qkv = torch.randn(r.L, 5, r.width, generator=g).to(torch.bfloat16)
        logits = torch.randn(5, wl.VOCAB, generator=g)
        draft = logits.argmax(-1)[:4].clone()  # drafts the target agrees with up to a planted mismatch
        if rep < 4:
            draft[rep] = (draft[rep] + 1) % wl.VOCAB
        ctx = r.verify(qkv.to(gpu), pos0, logits.to(gpu), draft.to(gpu))
        p = torch.tensor([pos0], dtype=torch.long, device=gpu)
        out = torch.empty(r.L, 5, sh.nh * HD, dtype=torch.bfloat16, device=gpu)
        for li in range(r.L):
            ops.qknorm_rope_kvwrite(qkv[li].to(gpu), r.qn_w[li], r.kn_w[li], r.eps, r.inv_freq, p, q,
                                    eager_kc[li], eager_vc[li], sh.nh, sh.nkv)
            ops.verify_attn(q, eager_kc[li], eager_vc[li], p, bound, r.scale, ws, ns, out[li])
        torch.cuda.synchronize()
        assert torch.equal(r.kc, eager_kc) and torch.equal(r.vc, eager_vc)
        assert torch.equal(ctx, out)
        assert torch.equal(r.tok_ver.cpu(), logits.argmax(-1))
        # in-graph acceptance (cuda_graph_executor.py:476): the planted mismatch, or all four
        assert tuple(r.acc_ver.cpu().tolist()) == ref.accept_prefix(logits.argmax(-1), draft)
        assert r.acc_ver[0].item() == (rep if rep < 4 else 4)
    assert sorted(r._ver_graphs) == [128, 2560, 4096]


def test_verify_bound_changes_no_bit(gpu):
    """A verify bound below the bucket only drops splits past the live length: with 128-key splits
    the outputs and cache rows over bounds 2560 (the routed one at 2048..2052), 3072 and 4096 are
    bit-identical (an empty split's partial folds in as an exact zero)."""
    r, g, sh = _make(gpu, layers=1, max_len=4096)
    pos0, k1 = 2048, 5
    assert verify_bound(pos0 + k1 - 1, r.buckets) == 2560
    qkv = torch.randn(k1, r.width, generator=g).to(torch.bfloat16).to(gpu)
    p = torch.tensor([pos0], dtype=torch.long, device=gpu)
    cs = ops.rope_rows(r.inv_freq, p, k1)
    outs = []
    for bound in (2560, 3072, 4096):
        _say(f"[verify bound {bound}]")
        ns = verify_splits(bound, sh.nkv)
        assert bound // ns == 128
        kc, vc = r.kc[0].clone(), r.vc[0].clone()
        ws = ops.attn_workspace(k1, sh.nh, sh.nkv, ns, gpu)
        out = torch.empty(k1, sh.nh * HD, dtype=torch.float32, device=gpu)
        ops.decode_layer(qkv, r.qn_w[0], r.kn_w[0], r.eps, cs, p, kc, vc, bound, r.scale, ws, ns, out,
                         sh.nh, sh.nkv)
        torch.cuda.synchronize()
        assert torch.isfinite(out).all()
        outs.append((out, kc, vc))
    for out, kc, vc in outs[1:]:
        assert torch.equal(out, outs[0][0])
        assert torch.equal(kc, outs[0][1]) and torch.equal(vc, outs[0][2])


def test_prefill_graph_then_decode_continues(gpu):
    """Graphed bucketed prefill of a 300-row prompt equals eager launches; a decode step at position 300
    then attends the prefilled rows exactly like decode over an eagerly written cache."""
    r, g, sh = _make(gpu, layers=2, max_len=1024)
    eager_kc, eager_vc = r.kc.clone(), r.vc.clone()
    T = 300
    qkv = torch.randn(r.L, T, r.width, generator=g).to(torch.bfloat16)
    for rep in range(2):  # replays of the same bucket graph
        ctx = r.prefill(qkv.to(gpu)).clone()
    assert sorted(r._pre_graphs) == [512]
    q = torch.empty(512, sh.nh, HD, dtype=torch.bfloat16, device=gpu)
    padded = torch.zeros(r.L, 512, r.width, dtype=torch.bfloat16)
    padded[:, :T] = qkv
    out = torch.empty(r.L, 512, sh.nh * HD, dtype=torch.bfloat16, device=gpu)
    for li in range(r.L):
        ops.qknorm_rope_kvwrite(padded[li].to(gpu), r.qn_w[li], r.kn_w[li], r.eps, r.inv_freq, None, q,
                                eager_kc[li], eager_vc[li], sh.nh, sh.nkv)
        ops.prefill_attn(q, eager_kc[li], eager_vc[li], r.scale, out[li])
    torch.cuda.synchronize()
    assert torch.equal(r.kc, eager_kc) and torch.equal(r.vc, eager_vc)
    assert torch.equal(ctx, out[:, :T])
    # causal: rows < T do not depend on the padding rows (random rows in their place change nothing)
    junk = padded[0].clone()
    junk[T:] = torch.randn(512 - T, r.width, generator=g).to(torch.bfloat16) * 4
    kc2, vc2 = eager_kc.clone(), eager_vc.clone()
    out2 = torch.empty(512, sh.nh * HD, dtype=torch.bfloat16, device=gpu)
    ops.qknorm_rope_kvwrite(junk.to(gpu), r.qn_w[0], r.kn_w[0], r.eps, r.inv_freq, None, q, kc2[0], vc2[0],
                            sh.nh, sh.nkv)
    ops.prefill_attn(q, kc2[0], vc2[0], r.scale, out2)
    torch.cuda.synchronize()
    assert torch.equal(out2[:T], ctx[0])
    assert not torch.equal(out2[T:], out[0, T:])
    # decode continues at position T over the prefilled cache
    qd = torch.randn(r.L, 1, r.width, generator=g).to(torch.bfloat16)
    dctx = r.decode(qd.to(gpu), T).clone()
    ws = ops.attn_workspace(1, sh.nh, sh.nkv, 32, gpu)
    p = torch.tensor([T], dtype=torch.long, device=gpu)
    dout = torch.empty(1, sh.nh * HD, dtype=torch.bfloat16, device=gpu)
    ops.decode_layer(qd[1].to(gpu), r.qn_w[1], r.kn_w[1], r.eps, ops.rope_rows(r.inv_freq, p, 1), p, eager_kc[1],
                     eager_vc[1], 512,
                     r.scale, ws, 32, dout, sh.nh, sh.nkv)
    torch.cuda.synchronize()
    assert torch.allclose(dctx[1].float(), dout.float(), atol=2e-3, rtol=0)
