"""Paged-KV decode (solort_paged_decode_layer) against the contiguous-cache decode layer.

The paged arena is the reference PagedKVCache's per-layer tensor [num_pages, 2, page_size, nkv, hd]
(src/solort/cache/kv_cache.py:71-100) with the sequence's pages scattered by a block table
(:113-145).  The same rows in a contiguous cache give the contiguous kernel's inputs, and the paged
call must reproduce its output and its KV write bit for bit (same bound, same split count): the
arithmetic and the split boundaries are shared, only the row addresses differ.  The contiguous
decode layer is itself held to the reference's attention in test_gpu_kernels.py; one case here is
also checked against the oracle directly.
"""
from __future__ import annotations

import sys

import pytest
import torch

from oracle import exact, ref
from solort_amd import ops
from solort_amd import workloads as wl
from solort_amd.runner import decode_splits

pytestmark = pytest.mark.gpu
HD = 128


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _paged_copy(kc, vc, page_size, gen, extra_pages=5, dev="cuda"):
    """A paged arena holding the rows of kc/vc [bound, nkv, hd] at scattered pages (the rest is
    junk) and the block table (int32, logical page -> physical page)."""
    bound, nkv = kc.shape[0], kc.shape[1]
    n_log = (bound + page_size - 1) // page_size
    num_pages = n_log + extra_pages
    table = torch.randperm(num_pages, generator=gen)[:n_log].to(torch.int32)
    kv = torch.randn(num_pages, 2, page_size, nkv, HD, generator=gen).to(torch.bfloat16)
    slots = torch.tensor(ref.slot_mapping(table.tolist(), list(range(bound)), page_size), dtype=torch.long)
    kv[slots // page_size, 0, slots % page_size] = kc.cpu()  # (a reshape of kv[:, 0] would be a copy)
    kv[slots // page_size, 1, slots % page_size] = vc.cpu()
    return kv.to(dev), table.to(dev), slots


CASES = [  # (workload, live, page_size, n_split or None for the runner's choice)
    (1, 1024, 16, None),    # Qwen3-4B decode at KV 1024, lane-parallel kernel
    (1, 1024, 1, None),     # one row per page
    (1, 128, 64, None),     # live < one... two pages
    (1, 1024, 16, 2),       # 512-key chunks: the MFMA split kernel
    (0, None, 16, None),    # Qwen3-0.6B shape (group 2)
    (4, None, 16, 32),      # speculative verify, 5 tokens at 2048..2052, bucket 4096
    (4, None, 256, 4),      # verify with 1024-key chunks and 256-row pages
]


@pytest.mark.parametrize("index,live,page_size,n_split", CASES,
                         ids=[f"w{c[0]}-live{c[1]}-ps{c[2]}-ns{c[3]}" for c in CASES])
def test_paged_decode_layer_equals_contiguous(gpu, index, live, page_size, n_split):
    case = wl.decode_case(index, live=live, layers=1)
    sh = case.shape
    ns = n_split or decode_splits(case.bound, sh.nkv)
    _say(f"[paged {sh.name} pos={case.pos} nq={case.nq} bound={case.bound} page_size={page_size} n_split={ns}]")
    gen = torch.Generator().manual_seed(500 + index * 7 + page_size)
    kc = case.kc[0][: case.bound].to(gpu)
    vc = case.vc[0][: case.bound].to(gpu)
    kv, table, slots = _paged_copy(kc, vc, page_size, gen, dev=gpu)
    pos = torch.tensor([case.pos], dtype=torch.long, device=gpu)
    qkv = case.qkv[0].to(gpu)
    qn, kn = case.qn_w[0].to(gpu), case.kn_w[0].to(gpu)
    cs = ops.rope_rows(ops.inv_freq(HD, wl.THETA, gpu), pos, case.nq)
    ws_a = ops.attn_workspace(case.nq, sh.nh, sh.nkv, ns, gpu)
    ws_b = ops.attn_workspace(case.nq, sh.nh, sh.nkv, ns, gpu)
    for dt in (torch.bfloat16, torch.float32):
        kc_a, vc_a, kv_b = kc.clone(), vc.clone(), kv.clone()
        out_a = torch.empty(case.nq, sh.nh * HD, dtype=dt, device=gpu)
        out_b = torch.empty_like(out_a)
        ops.decode_layer(qkv, qn, kn, wl.EPS, cs, pos, kc_a, vc_a, case.bound, sh.scale, ws_a, ns, out_a,
                         sh.nh, sh.nkv)
        ops.paged_decode_layer(qkv, qn, kn, wl.EPS, cs, pos, kv_b, table, case.bound, sh.scale, ws_b, ns, out_b,
                               sh.nh, sh.nkv)
        torch.cuda.synchronize()
        k_g, v_g = ref.paged_gather(kv_b.cpu(), slots.tolist())
        assert torch.equal(k_g, kc_a.cpu()) and torch.equal(v_g, vc_a.cpu()), "paged rows differ from the contiguous cache"
        written = set(slots.tolist())
        untouched = torch.ones(kv.shape[0] * page_size, dtype=torch.bool)
        untouched[list(written)] = False
        for half in (0, 1):  # rows outside the sequence's slots are left alone
            flat_b = kv_b[:, half].reshape(-1, sh.nkv, HD).cpu()
            flat_0 = kv[:, half].reshape(-1, sh.nkv, HD).cpu()
            assert torch.equal(flat_b[untouched], flat_0[untouched])
        assert torch.equal(out_a, out_b), f"outputs differ ({dt})"
    _say("  bit-identical to the contiguous cache (bf16 and fp32 outputs, KV rows, untouched pages)")


def test_paged_decode_ignores_table_entries_past_the_live_pages(gpu):
    """Entries past the live pages are read (their rows masked): junk and out-of-range entries (clamped
    into the pool) leave the output unchanged."""
    case = wl.decode_case(1, live=300, layers=1)  # bucket 300: pages 0..18 of 16 rows, live 0..299
    sh = case.shape
    ns = decode_splits(case.bound, sh.nkv)
    gen = torch.Generator().manual_seed(77)
    kv, table, _ = _paged_copy(case.kc[0][: case.bound].to(gpu), case.vc[0][: case.bound].to(gpu), 16, gen,
                               dev=gpu)
    pos = torch.tensor([case.pos - 40], dtype=torch.long, device=gpu)  # live 260: pages 17, 18 are dead
    qkv, qn, kn = case.qkv[0].to(gpu), case.qn_w[0].to(gpu), case.kn_w[0].to(gpu)
    cs = ops.rope_rows(ops.inv_freq(HD, wl.THETA, gpu), pos, 1)
    ws = ops.attn_workspace(1, sh.nh, sh.nkv, ns, gpu)
    outs = []
    for junk in (None, (-3, 10 ** 6)):
        t = table.clone()
        if junk:
            t[17], t[18] = junk
        kvc = kv.clone()
        out = torch.empty(1, sh.nh * HD, dtype=torch.float32, device=gpu)
        ops.paged_decode_layer(qkv, qn, kn, wl.EPS, cs, pos, kvc, t, case.bound, sh.scale, ws, ns, out, sh.nh, sh.nkv)
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])


def test_paged_decode_against_reference_ops(gpu):
    """Directly against the oracle: the gathered rows through the reference's prologue and grouped
    attention (cuda_graph_executor.py:173-184), bf16 bar 2e-2 max-abs / 2e-3 mean-abs."""
    case = wl.decode_case(1, live=700, layers=1)
    sh = case.shape
    ns = decode_splits(case.bound, sh.nkv)
    gen = torch.Generator().manual_seed(78)
    kc0, vc0 = case.kc[0][: case.bound], case.vc[0][: case.bound]
    kv, table, slots = _paged_copy(kc0.to(gpu), vc0.to(gpu), 16, gen, dev=gpu)
    pos = torch.tensor([case.pos], dtype=torch.long, device=gpu)
    cs = ops.rope_rows(ops.inv_freq(HD, wl.THETA, gpu), pos, 1)
    ws = ops.attn_workspace(1, sh.nh, sh.nkv, ns, gpu)
    out = torch.empty(1, sh.nh * HD, dtype=torch.bfloat16, device=gpu)
    ops.paged_decode_layer(case.qkv[0].to(gpu), case.qn_w[0].to(gpu), case.kn_w[0].to(gpu), wl.EPS, cs, pos, kv,
                           table, case.bound, sh.scale, ws, ns, out, sh.nh, sh.nkv)
    torch.cuda.synchronize()
    cos, sin = ref.cos_sin(torch.tensor([case.pos]), ref.inv_freq(HD, wl.THETA), torch.bfloat16)
    q, k, v = ref.prologue(case.qkv[0], case.qn_w[0], case.kn_w[0], wl.EPS, cos, sin, sh.nh, sh.nkv)
    kc_r, vc_r = kc0.clone(), vc0.clone()
    ref.write_kv(kc_r, vc_r, k, v, case.pos)
    want = ref.decode_attn(q, kc_r, vc_r, case.pos, case.bound, sh.scale).float()
    d = (out.float().cpu() - want).abs()
    _say(f"  vs reference ops: max-abs {d.max().item():.3e}, mean-abs {d.mean().item():.3e}")
    assert d.max().item() <= 2e-2 and d.mean().item() <= 2e-3
    # The new K/V row at its slot, bit for bit against the fixed-order prologue (the bar of every KV
    # write: the torch restatement's unspecified sum order can move a K element by one ulp).
    # cos/sin: torch's table on the device (the kernels reproduce it bit for bit; the CPU's cos can
    # differ in the last bit before the bf16 rounding)
    cos_t, sin_t = ops.rope_tables(case.pos + 1, HD, wl.THETA, gpu)
    _, kx, vx = exact.prologue_fixed_order(case.qkv[0].float().numpy(), case.qn_w[0].float().numpy(),
                                           case.kn_w[0].float().numpy(), wl.EPS,
                                           cos_t.cpu()[case.pos:].float().numpy(),
                                           sin_t.cpu()[case.pos:].float().numpy(), sh.nh, sh.nkv)
    k_g, v_g = ref.paged_gather(kv.cpu(), slots.tolist())
    assert torch.equal(k_g[case.pos], torch.from_numpy(kx[0]).to(torch.bfloat16))
    assert torch.equal(v_g[case.pos], torch.from_numpy(vx[0]).to(torch.bfloat16))
    assert (k_g[case.pos].float() - kc_r[case.pos].float()).abs().max().item() <= 2 ** -7 * 4


def test_paged_kv_store_and_gather_match_reference(gpu):
    """solort_paged_kv_store / _gather against the oracle's restatement of store_layer_tokens and
    gather_layer_tokens (kv_cache.py:191-256; pinned on the reference's own test vectors): bit-exact
    arena after the store, the rows back from the gather, rows of other slots untouched, and slots
    outside the pool skipped by the store and read as zeros by the gather."""
    T, nkv, ps, pages = 37, 8, 16, 6
    g = torch.Generator().manual_seed(90)
    table = torch.randperm(pages, generator=g)[:3].tolist()
    slots = ref.slot_mapping(table, list(range(T)), ps)
    k = torch.randn(T, nkv, HD, generator=g).to(torch.bfloat16)
    v = torch.randn(T, nkv, HD, generator=g).to(torch.bfloat16)
    arena = torch.randn(pages, 2, ps, nkv, HD, generator=g).to(torch.bfloat16)
    want = arena.clone()
    ref.paged_store(want, slots, k, v)
    kv = arena.to(gpu)
    sm = torch.tensor(slots, dtype=torch.long, device=gpu)
    ops.paged_kv_store(k.to(gpu), v.to(gpu), sm, kv)
    kg = torch.zeros(T, nkv, HD, dtype=torch.bfloat16, device=gpu)
    vg = torch.zeros_like(kg)
    ops.paged_kv_gather(kv, sm, kg, vg)
    torch.cuda.synchronize()
    assert torch.equal(kv.cpu(), want)
    assert torch.equal(kg.cpu(), k) and torch.equal(vg.cpu(), v)
    bad = torch.tensor([-1, pages * ps, slots[5]], dtype=torch.long, device=gpu)
    kv2 = kv.clone()
    ops.paged_kv_store((k[:3] + 1).to(gpu), (v[:3] + 1).to(gpu), bad, kv2)
    kb, vb = torch.ones(3, nkv, HD, dtype=torch.bfloat16, device=gpu), torch.ones(3, nkv, HD, dtype=torch.bfloat16,
                                                                                  device=gpu)
    ops.paged_kv_gather(kv2, bad, kb, vb)
    torch.cuda.synchronize()
    changed = (kv2 != kv).reshape(pages, 2, ps, -1).any(-1)
    assert changed.sum().item() == 2 and changed[slots[5] // ps, :, slots[5] % ps].all()  # only slot[5], K and V
    assert (kb[:2] == 0).all() and (vb[:2] == 0).all() and torch.equal(kb[2].cpu(), k[2] + 1)


def test_paged_prompt_then_decode_equals_contiguous(gpu):
    """A prompt placed in pages the way the reference's paged path would (solort_prefill_layer into
    contiguous rows, then solort_paged_kv_store through the sequence's slot mapping) followed by
    paged decode steps gives the contiguous path's outputs and cache rows bit for bit."""
    sh = wl.QWEN3_4B
    T, ps, bound, steps = 300, 16, 512, 3
    g = torch.Generator().manual_seed(91)
    ifr = ops.inv_freq(HD, wl.THETA, gpu)
    qn = (1 + 0.1 * torch.randn(HD, generator=g)).to(torch.bfloat16).to(gpu)
    kn = (1 + 0.1 * torch.randn(HD, generator=g)).to(torch.bfloat16).to(gpu)
    qkv = torch.randn(T, sh.qkv_width, generator=g).to(torch.bfloat16).to(gpu)
    kc = torch.zeros(bound, sh.nkv, HD, dtype=torch.bfloat16, device=gpu)
    vc = torch.zeros_like(kc)
    cs = ops.rope_rows(ifr, torch.zeros(1, dtype=torch.long, device=gpu), T)
    ctx = torch.empty(T, sh.nh * HD, dtype=torch.bfloat16, device=gpu)
    ops.prefill_layer(qkv, qn, kn, wl.EPS, cs, kc, vc, sh.scale, ctx, sh.nh, sh.nkv)
    n_log = bound // ps
    table = torch.randperm(n_log + 4, generator=g)[:n_log].to(torch.int32)
    kv = torch.zeros(n_log + 4, 2, ps, sh.nkv, HD, dtype=torch.bfloat16, device=gpu)
    sm = torch.tensor(ref.slot_mapping(table.tolist(), list(range(T)), ps), dtype=torch.long, device=gpu)
    ops.paged_kv_store(kc[:T], vc[:T], sm, kv)
    table = table.to(gpu)
    ns = decode_splits(bound, sh.nkv)
    ws_a = ops.attn_workspace(1, sh.nh, sh.nkv, ns, gpu)
    ws_b = ops.attn_workspace(1, sh.nh, sh.nkv, ns, gpu)
    for i in range(steps):
        pos = torch.tensor([T + i], dtype=torch.long, device=gpu)
        q1 = torch.randn(1, sh.qkv_width, generator=g).to(torch.bfloat16).to(gpu)
        c1 = ops.rope_rows(ifr, pos, 1)
        out_a = torch.empty(1, sh.nh * HD, dtype=torch.float32, device=gpu)
        out_b = torch.empty_like(out_a)
        ops.decode_layer(q1, qn, kn, wl.EPS, c1, pos, kc, vc, bound, sh.scale, ws_a, ns, out_a, sh.nh, sh.nkv)
        ops.paged_decode_layer(q1, qn, kn, wl.EPS, c1, pos, kv, table, bound, sh.scale, ws_b, ns, out_b, sh.nh, sh.nkv)
        torch.cuda.synchronize()
        assert torch.equal(out_a, out_b), i
    sm_all = torch.tensor(ref.slot_mapping(table.cpu().tolist(), list(range(T + steps)), ps), dtype=torch.long,
                          device=gpu)
    kg = torch.empty(T + steps, sh.nkv, HD, dtype=torch.bfloat16, device=gpu)
    vg = torch.empty_like(kg)
    ops.paged_kv_gather(kv, sm_all, kg, vg)
    torch.cuda.synchronize()
    assert torch.equal(kg, kc[:T + steps]) and torch.equal(vg, vc[:T + steps])
