"""GPU parity of the HIP kernels against the CPU oracle, on the seeded workloads.

Bars: KV-cache rows bit-exact with the fixed-order oracle; attention outputs
within max-abs 2e-2 / mean-abs 2e-3 of the reference's bf16 torch ops, and
within 1e-4 (max-abs) when the kernel writes fp32 and is compared with fp64
attention over the same bf16 q/K/V; argmax bit-exact.
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
BF16_MAX, BF16_MEAN, F32_MAX = 2e-2, 2e-3, 1e-4


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _tables(dev, rows):
    """torch's cos/sin table (the oracle's RoPE input; the kernels compute the same values)."""
    cos, sin = ops.rope_tables(rows, HD, wl.THETA, dev)
    return cos, sin


def _ifr(dev):
    return ops.inv_freq(HD, wl.THETA, dev)


def _run_prologue(dev, case, li, kc, vc):
    """Prologue for layer li of a decode case on the GPU; returns q [nq, nh, hd] (device)."""
    sh = case.shape
    q = torch.empty(case.nq, sh.nh, HD, dtype=torch.bfloat16, device=dev)
    pos = torch.tensor([case.pos], dtype=torch.long, device=dev)
    ops.qknorm_rope_kvwrite(case.qkv[li].to(dev), case.qn_w[li].to(dev), case.kn_w[li].to(dev), wl.EPS,
                            _ifr(dev), pos, q, kc, vc, sh.nh, sh.nkv)
    return q, pos


def _oracle_layer(case, li, cos_cpu, sin_cpu):
    """Reference ops (torch CPU, bf16) for one layer: returns (ctx, kc_l, vc_l) after the KV write."""
    sh = case.shape
    pos = torch.arange(case.pos, case.pos + case.nq)
    full_cos = torch.cat([cos_cpu[pos], cos_cpu[pos]], -1)
    full_sin = torch.cat([sin_cpu[pos], sin_cpu[pos]], -1)
    q, k, v = ref.prologue(case.qkv[li], case.qn_w[li], case.kn_w[li], wl.EPS, full_cos, full_sin, sh.nh, sh.nkv)
    kc_l, vc_l = case.kc[li].clone(), case.vc[li].clone()
    ref.write_kv(kc_l, vc_l, k, v, case.pos)
    if case.nq == 1:
        ctx = ref.decode_attn(q, kc_l, vc_l, case.pos, case.bound, sh.scale)
    else:
        ctx = ref.verify_attn(q, kc_l, vc_l, case.pos, sh.scale)
    return ctx, kc_l, vc_l


def _fixed_order_kv(case, li, cos_cpu, sin_cpu):
    sh = case.shape
    pos = np.arange(case.pos, case.pos + case.nq)
    q, k, v = exact.prologue_fixed_order(case.qkv[li].float().numpy(), case.qn_w[li].float().numpy(),
                                         case.kn_w[li].float().numpy(), wl.EPS,
                                         cos_cpu[pos].float().numpy(), sin_cpu[pos].float().numpy(), sh.nh, sh.nkv)
    return q, k, v


def _check_bf16(got: torch.Tensor, want: torch.Tensor, what: str):
    d = (got.float().cpu() - want.float()).abs()
    _say(f"{what}: max-abs {d.max().item():.3e} mean-abs {d.mean().item():.3e}")
    assert d.max().item() <= BF16_MAX and d.mean().item() <= BF16_MEAN, what


def _decode_case_check(gpu, case, n_splits, layers=(0,)):
    dev = gpu
    sh = case.shape
    cos, sin = _tables(dev, case.max_len)
    cos_cpu, sin_cpu = cos.cpu(), sin.cpu()
    for li in layers:
        _say(f"[{sh.name} pos={case.pos} nq={case.nq} bound={case.bound} layer={li}]")
        kc = case.kc[li].to(dev)
        vc = case.vc[li].to(dev)
        q, pos = _run_prologue(dev, case, li, kc, vc)
        torch.cuda.synchronize()
        # KV rows: bit-exact against the fixed-order oracle; other rows untouched
        qx, kx, vx = _fixed_order_kv(case, li, cos_cpu, sin_cpu)
        kc_want = case.kc[li].clone()
        vc_want = case.vc[li].clone()
        kc_want[case.pos:case.pos + case.nq] = torch.from_numpy(kx).to(torch.bfloat16)
        vc_want[case.pos:case.pos + case.nq] = torch.from_numpy(vx).to(torch.bfloat16)
        assert torch.equal(kc.cpu(), kc_want), "K cache differs from the fixed-order oracle"
        assert torch.equal(vc.cpu(), vc_want), "V cache differs"
        assert torch.equal(q.cpu(), torch.from_numpy(qx).to(torch.bfloat16)), "q differs from the fixed-order oracle"
        ctx_ref, kc_ref, _ = _oracle_layer(case, li, cos_cpu, sin_cpu)
        # torch's own sum order may flip a rare bf16 ulp of K relative to the fixed order
        flips = (kc_ref != kc.cpu()).sum().item()
        _say(f"  K elements differing from torch-order restatement: {flips}")
        q64 = q.float().cpu().numpy()
        want64 = exact.causal_decode_fp64(q64, kc.float().cpu().numpy(), vc.float().cpu().numpy(), case.pos,
                                          sh.scale).reshape(case.nq, sh.nh * HD)
        for ns in n_splits:
            ws = ops.attn_workspace(case.nq, sh.nh, sh.nkv, ns, dev)
            out = torch.empty(case.nq, sh.nh * HD, dtype=torch.bfloat16, device=dev)
            out32 = torch.empty(case.nq, sh.nh * HD, dtype=torch.float32, device=dev)
            fn = ops.decode_attn if case.nq == 1 else ops.verify_attn
            fn(q, kc, vc, pos, case.bound, sh.scale, ws, ns, out)
            fn(q, kc, vc, pos, case.bound, sh.scale, ws, ns, out32)
            torch.cuda.synchronize()
            _check_bf16(out, ctx_ref, f"  n_split={ns} bf16 vs reference ops")
            e32 = np.abs(out32.cpu().numpy().astype(np.float64) - want64).max()
            _say(f"  n_split={ns} fp32 vs fp64: max-abs {e32:.3e}")
            assert e32 <= F32_MAX
            assert torch.equal(out, out32.to(torch.bfloat16)), "bf16 output is not the rounded fp32 output"


@pytest.mark.parametrize("live", wl.DECODE_LIVE)
def test_decode_qwen3_4b(gpu, live):
    case = wl.decode_case(1, live=live, layers=2)
    _decode_case_check(gpu, case, n_splits=(1, 7, 32, 64), layers=(0, 1))


def test_decode_qwen3_0_6b(gpu):
    case = wl.decode_case(0, layers=2)
    _decode_case_check(gpu, case, n_splits=(1, 16, 32), layers=(0, 1))


def test_decode_qwen3_8b_32k(gpu):
    case = wl.decode_case(3, layers=1)
    dev = gpu
    sh = case.shape
    kc, vc = case.kc[0].to(dev), case.vc[0].to(dev)
    q, pos = _run_prologue(dev, case, 0, kc, vc)
    torch.cuda.synchronize()
    _say(f"[{sh.name} 32k decode] prologue done")
    q64 = q.float().cpu().numpy()
    kf, vf = kc.float().cpu().numpy(), vc.float().cpu().numpy()
    want64 = exact.causal_decode_fp64(q64, kf, vf, case.pos, sh.scale).reshape(1, -1)
    ctx_ref = ref.decode_attn(q.cpu().transpose(0, 1), kc.cpu(), vc.cpu(), case.pos, case.bound, sh.scale)
    ref_err = np.abs(ctx_ref.float().numpy() - want64)
    _say(f"  reference bf16 ops vs fp64: max-abs {ref_err.max():.3e} mean-abs {ref_err.mean():.3e}")
    for ns in (32, 64, 256, 1024):  # 1024 splits: 32-key chunks (lane-parallel kernel); others MFMA
        ws = ops.attn_workspace(1, sh.nh, sh.nkv, ns, dev)
        out = torch.empty(1, sh.nh * HD, dtype=torch.bfloat16, device=dev)
        out32 = torch.empty(1, sh.nh * HD, dtype=torch.float32, device=dev)
        ops.decode_attn(q, kc, vc, pos, case.bound, sh.scale, ws, ns, out)
        ops.decode_attn(q, kc, vc, pos, case.bound, sh.scale, ws, ns, out32)
        torch.cuda.synchronize()
        e32 = np.abs(out32.cpu().numpy().astype(np.float64) - want64)
        e16 = np.abs(out.float().cpu().numpy() - want64)
        # Distance from the reference's own bf16 ops, on record: with the x8 keys those ops are
        # themselves up to ~7.5e-2 from exact attention, so this is not the bar asserted below.
        dref = np.abs(out.float().cpu().numpy() - ctx_ref.float().numpy())
        _say(f"  n_split={ns}: fp32 vs fp64 max {e32.max():.3e}; bf16 vs fp64 max {e16.max():.3e} "
             f"mean {e16.mean():.3e}; bf16 vs the reference's bf16 ops max {dref.max():.3e} mean {dref.mean():.3e}")
        assert e32.max() <= F32_MAX
        # the kernel's bf16 output is at least as close to exact attention as the reference's bf16 ops
        assert e16.max() <= max(BF16_MAX, ref_err.max()) and e16.mean() <= max(BF16_MEAN, ref_err.mean())


def test_verify_qwen3_4b(gpu):
    case = wl.decode_case(4, layers=1)
    _decode_case_check(gpu, case, n_splits=(1, 16, 64), layers=(0,))


def test_verify_equals_sequential_decode(gpu):
    """Verify of K+1 tokens == K+1 single-token decode calls at pos0..pos0+K over the same cache."""
    case = wl.decode_case(4, layers=1)
    dev = gpu
    sh = case.shape
    kc, vc = case.kc[0].to(dev), case.vc[0].to(dev)
    q, pos = _run_prologue(dev, case, 0, kc, vc)
    ws = ops.attn_workspace(5, sh.nh, sh.nkv, 32, dev)
    out = torch.empty(5, sh.nh * HD, dtype=torch.float32, device=dev)
    ops.verify_attn(q, kc, vc, pos, case.max_len, sh.scale, ws, 32, out)
    ws1 = ops.attn_workspace(1, sh.nh, sh.nkv, 32, dev)
    for t in range(5):
        o1 = torch.empty(1, sh.nh * HD, dtype=torch.float32, device=dev)
        p = torch.tensor([case.pos + t], dtype=torch.long, device=dev)
        ops.decode_attn(q[t:t + 1].contiguous(), kc, vc, p, case.max_len, sh.scale, ws1, 32, o1)
        torch.cuda.synchronize()
        assert torch.allclose(out[t:t + 1], o1, atol=1e-6, rtol=0), t


def test_prologue_prefill_rows_bitexact(gpu):
    """T=1024 prompt rows at positions 0..1023 into an empty cache (prefill KV write)."""
    case = wl.prefill_case(1024, layers=1)
    dev = gpu
    sh = case.shape
    cos, sin = _tables(dev, case.max_len)
    kc = torch.zeros(case.max_len, sh.nkv, HD, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    q = torch.empty(case.T, sh.nh, HD, dtype=torch.bfloat16, device=dev)
    ops.qknorm_rope_kvwrite(case.qkv[0].to(dev), case.qn_w[0].to(dev), case.kn_w[0].to(dev), wl.EPS, _ifr(dev),
                            None, q, kc, vc, sh.nh, sh.nkv)
    torch.cuda.synchronize()
    qx, kx, vx = exact.prologue_fixed_order(case.qkv[0].float().numpy(), case.qn_w[0].float().numpy(),
                                            case.kn_w[0].float().numpy(), wl.EPS, cos.cpu()[:case.T].float().numpy(),
                                            sin.cpu()[:case.T].float().numpy(), sh.nh, sh.nkv)
    assert torch.equal(q.cpu(), torch.from_numpy(qx).to(torch.bfloat16))
    assert torch.equal(kc.cpu()[:case.T], torch.from_numpy(kx).to(torch.bfloat16))
    assert torch.equal(vc.cpu()[:case.T], torch.from_numpy(vx).to(torch.bfloat16))


@pytest.mark.parametrize("T,pos0", [(1024, None), (5, 2048), (1, 32767)])
def test_prologue_with_step_table_equals_in_kernel_cos_sin(gpu, T, pos0):
    """qknorm_rope_kvwrite_cs (cos/sin rows from rope_rows, once per step) writes the same q, K and V
    bits as qknorm_rope_kvwrite (cos/sin evaluated in the kernel)."""
    dev = gpu
    sh = wl.QWEN3_4B
    g = torch.Generator().manual_seed(77 + T)
    qkv = torch.randn(T, sh.qkv_width, generator=g).to(torch.bfloat16).to(dev)
    qn = (1 + 0.1 * torch.randn(HD, generator=g)).to(torch.bfloat16).to(dev)
    kn = (1 + 0.1 * torch.randn(HD, generator=g)).to(torch.bfloat16).to(dev)
    max_len = 32768
    p0 = 0 if pos0 is None else pos0
    pos = torch.tensor([p0], dtype=torch.long, device=dev)
    outs = []
    for use_table in (False, True):
        kc = torch.zeros(max_len, sh.nkv, HD, dtype=torch.bfloat16, device=dev)
        vc = torch.zeros_like(kc)
        q = torch.empty(T, sh.nh, HD, dtype=torch.bfloat16, device=dev)
        pos_arg = None if pos0 is None else pos
        if use_table:
            cs = ops.rope_rows(_ifr(dev), pos, T)
            ops.qknorm_rope_kvwrite_cs(qkv, qn, kn, wl.EPS, cs, pos_arg, q, kc, vc, sh.nh, sh.nkv)
        else:
            ops.qknorm_rope_kvwrite(qkv, qn, kn, wl.EPS, _ifr(dev), pos_arg, q, kc, vc, sh.nh, sh.nkv)
        torch.cuda.synchronize()
        outs.append((q.cpu(), kc[p0:p0 + T].cpu(), vc[p0:p0 + T].cpu()))
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_prologue_skips_out_of_range_positions(gpu):
    dev = gpu
    kc = torch.full((64, 8, HD), 7.0, dtype=torch.bfloat16, device=dev)
    vc = kc.clone()
    qkv = torch.randn(2, 48 * HD, device=dev).to(torch.bfloat16)
    w = torch.ones(HD, dtype=torch.bfloat16, device=dev)
    q = torch.empty(2, 32, HD, dtype=torch.bfloat16, device=dev)
    pos = torch.tensor([63], dtype=torch.long, device=dev)  # token 1 lands at 64: outside the cache
    ops.qknorm_rope_kvwrite(qkv, w, w, wl.EPS, _ifr(dev), pos, q, kc, vc, 32, 8)
    torch.cuda.synchronize()
    assert torch.all(kc[:63] == 7.0) and torch.all(vc[:63] == 7.0)
    assert not torch.all(kc[63] == 7.0)


# ------------------------------------------------------------------ argmax

def _argmax_check(dev, x: torch.Tensor, ws: torch.Tensor | None = None):
    ws = ops.argmax_workspace(x.shape[0], dev) if ws is None else ws
    out = torch.empty(x.shape[0], dtype=torch.long, device=dev)
    xd = x.to(dev)
    for _ in range(2):  # the workspace must be ready again after each call
        ops.argmax_rows(xd, out, ws)
        torch.cuda.synchronize()
        want = exact.argmax_first(x.float().numpy())
        assert np.array_equal(out.cpu().numpy(), want)
    assert ops.argmax_failures(ws, x.shape[0]) == 0


def _argmax_hard_rows() -> torch.Tensor:
    x = torch.full((4, 151936), -5.0)
    x[0, [151935, 70000, 2048, 2047]] = 3.0        # ties straddling block boundaries
    x[1, 123456] = float("nan")
    x[1, 99999] = float("inf")
    x[1, 140000] = float("nan")                     # first NaN wins
    x[2] = -0.0
    x[2, 5] = 0.0                                   # -0 == +0: index 0 wins
    x[3] = float("-inf")                            # all -inf: index 0
    return x


def test_argmax_planted_ties(gpu):
    case = wl.decode_case(4, layers=1)
    _say("[argmax bf16 5x151936 planted ties]")
    _argmax_check(gpu, case.logits)
    _argmax_check(gpu, case.logits.float())


@pytest.mark.parametrize("rows,vocab", [(1, 151936), (3, 1000), (2, 8), (4, 2049), (1, 1)])
def test_argmax_shapes(gpu, rows, vocab):
    g = torch.Generator().manual_seed(rows * 7919 + vocab)
    x = torch.randn(rows, vocab, generator=g)
    _argmax_check(gpu, x.to(torch.bfloat16))
    _argmax_check(gpu, x)


def test_argmax_ties_across_blocks_nan_and_zero(gpu):
    x = _argmax_hard_rows()
    _argmax_check(gpu, x)
    _argmax_check(gpu, x.to(torch.bfloat16))


def test_argmax_two_launch_fallback(gpu):
    """The second-launch reduction (used where the workgroup placement is unverified), forced by
    the host switch, gives the one-launch indices on the planted-tie and NaN cases; one workspace
    alternates between the two modes (each mode advances the same per-row epochs) and serves graph
    replays in the fallback mode."""
    assert ops.argmax_mode(-1) == 1, "solort_init did not enable the one-launch argmax"
    case = wl.decode_case(4, layers=1)
    hard = _argmax_hard_rows()
    ws = ops.argmax_workspace(5, gpu)
    try:
        for mode in (0, 1, 0):
            assert ops.argmax_mode(mode) == mode
            _say(f"[argmax mode {mode}: planted ties, NaN, -0, -inf]")
            _argmax_check(gpu, case.logits, ws)
            _argmax_check(gpu, case.logits.float(), ws)
            _argmax_check(gpu, hard, ws)
            _argmax_check(gpu, hard.to(torch.bfloat16), ws)
        ops.argmax_mode(0)
        a = case.logits.to(gpu)
        oa = torch.empty(a.shape[0], dtype=torch.long, device=gpu)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            ops.argmax_rows(a, oa, ws)
        want = exact.argmax_first(case.logits.float().numpy())
        for r in range(3):
            oa.fill_(-7)
            graph.replay()
            torch.cuda.synchronize()
            assert np.array_equal(oa.cpu().numpy(), want), f"replay {r}"
            _argmax_check(gpu, hard, ws)  # eager work between replays
    finally:
        ops.argmax_mode(1)
    assert ops.argmax_failures(ws, 5) == 0


def test_argmax_workspace_across_shapes_and_graph_replays(gpu):
    """One workspace over calls whose rows are cut into different numbers of chunks (each launch
    tags its slots with the row's next epoch, so slots left by a longer row earlier are never
    read), then a graph of two argmax launches replayed with eager calls in between."""
    g = torch.Generator().manual_seed(11)
    xs = [torch.randn(5, 151936, generator=g), torch.randn(5, 8, generator=g), torch.randn(3, 20000, generator=g),
          torch.randn(5, 151936, generator=g).to(torch.bfloat16), torch.randn(1, 3000, generator=g)]
    ws = ops.argmax_workspace(5, gpu)
    for rep in range(3):
        for x in xs:
            out = torch.empty(x.shape[0], dtype=torch.long, device=gpu)
            ops.argmax_rows(x.to(gpu), out, ws)
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy(), exact.argmax_first(x.float().numpy())), (rep, tuple(x.shape))
    a, b = xs[0].to(gpu), xs[3].to(gpu)
    oa = torch.empty(5, dtype=torch.long, device=gpu)
    ob = torch.empty(5, dtype=torch.long, device=gpu)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.argmax_rows(a, oa, ws)
        ops.argmax_rows(b, ob, ws)
    wa, wb = exact.argmax_first(xs[0].float().numpy()), exact.argmax_first(xs[3].float().numpy())
    for r in range(4):
        oa.zero_()
        ob.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(oa.cpu().numpy(), wa) and np.array_equal(ob.cpu().numpy(), wb), f"replay {r}"
        out = torch.empty(3, dtype=torch.long, device=gpu)
        ops.argmax_rows(xs[2].to(gpu), out, ws)  # eager work between replays
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), exact.argmax_first(xs[2].numpy()))


def test_argmax_failure_path_stays_in_the_row(gpu):
    """The host-forced failure mode (solort_argmax_mode(2): a row's reducing block stops polling at
    once) writes, for every row, the index of the best key that block saw: its own chunk's, the
    row's last, so x[r, idx] is the maximum of x[r, idx:]; each call counts one failure per row.
    Back in the default mode the same workspace gives the exact indices and counts nothing more."""
    g = torch.Generator().manual_seed(17)
    x = torch.randn(5, 151936, generator=g)
    ws = ops.argmax_workspace(5, gpu)
    out = torch.empty(5, dtype=torch.long, device=gpu)
    xd = x.to(gpu)
    try:
        assert ops.argmax_mode(2) == 2
        for call in (1, 2):
            ops.argmax_rows(xd, out, ws)
            torch.cuda.synchronize()
            idx = out.cpu().numpy()
            _say(f"[argmax failure mode, call {call}] indices {idx.tolist()}")
            assert ((idx >= 0) & (idx < x.shape[1])).all()
            assert ops.argmax_failures(ws, 5) == 5 * call
            for r in range(5):
                assert x[r, idx[r]] == x[r, idx[r]:].max()
    finally:
        ops.argmax_mode(1)
    ops.argmax_rows(xd, out, ws)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), exact.argmax_first(x.numpy()))
    assert ops.argmax_failures(ws, 5) == 10


def test_argmax_strided_rows(gpu):
    g = torch.Generator().manual_seed(5)
    big = torch.randn(3, 1003, generator=g)
    x = big[:, 1:1000]  # unaligned start and odd stride: scalar path
    ws = ops.argmax_workspace(3, gpu)
    out = torch.empty(3, dtype=torch.long, device=gpu)
    ops.argmax_rows(big.to(gpu)[:, 1:1000], out, ws)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), exact.argmax_first(x.numpy()))


# ------------------------------------------------------------------ fused layer

@pytest.mark.parametrize("index,live,n_split", [(1, 128, 4), (1, 256, 8), (1, 512, 16), (1, 1024, 32),
                                                (1, 1024, 64), (1, 1024, 7), (0, None, 32), (3, None, 256),
                                                (4, None, 64)])
def test_decode_layer_equals_prologue_then_attention(gpu, index, live, n_split):
    """The fused launch writes the same KV bits and produces the same output bits as the two-launch path."""
    case = wl.decode_case(index, live=live, layers=1)
    dev = gpu
    sh = case.shape
    _say(f"[fused {sh.name} pos={case.pos} nq={case.nq} bound={case.bound} n_split={n_split}]")
    ifr = _ifr(dev)
    kc_a, vc_a = case.kc[0].to(dev), case.vc[0].to(dev)
    kc_b, vc_b = kc_a.clone(), vc_a.clone()
    pos = torch.tensor([case.pos], dtype=torch.long, device=dev)
    qkv = case.qkv[0].to(dev)
    qn, kn = case.qn_w[0].to(dev), case.kn_w[0].to(dev)
    q = torch.empty(case.nq, sh.nh, HD, dtype=torch.bfloat16, device=dev)
    ws = ops.attn_workspace(case.nq, sh.nh, sh.nkv, n_split, dev)
    for dt in (torch.bfloat16, torch.float32):
        out_a = torch.empty(case.nq, sh.nh * HD, dtype=dt, device=dev)
        out_b = torch.empty_like(out_a)
        ops.qknorm_rope_kvwrite(qkv, qn, kn, wl.EPS, ifr, pos, q, kc_a, vc_a, sh.nh, sh.nkv)
        fn = ops.decode_attn if case.nq == 1 else ops.verify_attn
        fn(q, kc_a, vc_a, pos, case.bound, sh.scale, ws, n_split, out_a)
        ops.decode_layer(qkv, qn, kn, wl.EPS, ops.rope_rows(ifr, pos, case.nq), pos, kc_b, vc_b, case.bound,
                         sh.scale, ws, n_split, out_b,
                         sh.nh, sh.nkv)
        torch.cuda.synchronize()
        assert torch.equal(kc_a, kc_b) and torch.equal(vc_a, vc_b), "KV rows differ"
        assert torch.equal(out_a, out_b), f"outputs differ ({dt})"


def test_decode_layer_repeated_calls_reuse_workspace(gpu):
    """Ten back-to-back fused launches over different layers share one workspace and each matches
    the launch four calls earlier on the same layer."""
    case = wl.decode_case(1, live=1024, layers=4)
    dev = gpu
    sh = case.shape
    ifr = _ifr(dev)
    pos = torch.tensor([case.pos], dtype=torch.long, device=dev)
    kc, vc = case.kc.to(dev), case.vc.to(dev)
    ws = ops.attn_workspace(1, sh.nh, sh.nkv, 32, dev)
    outs = torch.empty(10, 1, sh.nh * HD, dtype=torch.float32, device=dev)
    cs = ops.rope_rows(ifr, pos, 1)
    for i in range(10):
        li = i % 4
        ops.decode_layer(case.qkv[li].to(dev), case.qn_w[li].to(dev), case.kn_w[li].to(dev), wl.EPS, cs, pos,
                         kc[li], vc[li], case.bound, sh.scale, ws, 32, outs[i], sh.nh, sh.nkv)
    torch.cuda.synchronize()
    for i in range(4, 10):
        assert torch.equal(outs[i], outs[i - 4])


@pytest.mark.parametrize("index,live,n_split", [(1, 1024, 32), (1, 256, 8), (4, None, 32)])
def test_decode_layer_head_major_cache_equals_token_major(gpu, index, live, n_split):
    """A head-major cache ([nkv][rows][128] storage with rows >= 8192: head stride >= 2^20 elements,
    past the 16-bit stride fields of the packed-argument kernels, so the launch takes the general
    one) gives the same KV bits and output bits as the token-major [max_len][nkv][128] cache, for the
    lane kernel (one token) and the MFMA kernel (verify, 5 tokens)."""
    case = wl.decode_case(index, live=live, layers=1)
    dev = gpu
    sh = case.shape
    _say(f"[head-major {sh.name} pos={case.pos} nq={case.nq} bound={case.bound} n_split={n_split}]")
    ifr = _ifr(dev)
    pos = torch.tensor([case.pos], dtype=torch.long, device=dev)
    qkv = case.qkv[0].to(dev)
    qn, kn = case.qn_w[0].to(dev), case.kn_w[0].to(dev)
    kc_t, vc_t = case.kc[0].to(dev), case.vc[0].to(dev)
    rows = max(8192, 2 * case.max_len)
    k_store = torch.zeros(sh.nkv, rows, HD, dtype=torch.bfloat16, device=dev)
    v_store = torch.zeros_like(k_store)
    k_store[:, :case.max_len] = kc_t.permute(1, 0, 2)
    v_store[:, :case.max_len] = vc_t.permute(1, 0, 2)
    kc_h = k_store[:, :case.max_len].permute(1, 0, 2)
    vc_h = v_store[:, :case.max_len].permute(1, 0, 2)
    assert kc_h.stride() == (HD, rows * HD, 1)
    ws = ops.attn_workspace(case.nq, sh.nh, sh.nkv, n_split, dev)
    cs = ops.rope_rows(ifr, pos, case.nq)
    for dt in (torch.bfloat16, torch.float32):
        out_t = torch.empty(case.nq, sh.nh * HD, dtype=dt, device=dev)
        out_h = torch.empty_like(out_t)
        ops.decode_layer(qkv, qn, kn, wl.EPS, cs, pos, kc_t, vc_t, case.bound, sh.scale, ws, n_split, out_t,
                         sh.nh, sh.nkv)
        ops.decode_layer(qkv, qn, kn, wl.EPS, cs, pos, kc_h, vc_h, case.bound, sh.scale, ws, n_split, out_h,
                         sh.nh, sh.nkv)
        torch.cuda.synchronize()
        assert torch.equal(out_t, out_h), f"outputs differ ({dt})"
        assert torch.equal(kc_t, kc_h) and torch.equal(vc_t, vc_h), "KV rows differ"


@pytest.mark.parametrize("index,live,n_split", [(1, 1024, 32), (4, None, 32)])
def test_decode_layer_padded_qkv_rows_equal_packed(gpu, index, live, n_split):
    """qkv rows with a padded row stride (the general MFMA kernel: its packed variant assumes packed
    rows) give the same KV bits and output bits as packed rows."""
    case = wl.decode_case(index, live=live, layers=1)
    dev = gpu
    sh = case.shape
    _say(f"[padded qkv {sh.name} pos={case.pos} nq={case.nq} bound={case.bound} n_split={n_split}]")
    ifr = _ifr(dev)
    pos = torch.tensor([case.pos], dtype=torch.long, device=dev)
    qkv = case.qkv[0].to(dev)
    store = torch.zeros(case.nq, sh.qkv_width + 64, dtype=torch.bfloat16, device=dev)
    store[:, :sh.qkv_width] = qkv
    qkv_p = store[:, :sh.qkv_width]
    assert qkv_p.stride(0) == sh.qkv_width + 64
    qn, kn = case.qn_w[0].to(dev), case.kn_w[0].to(dev)
    kc_a, vc_a = case.kc[0].to(dev), case.vc[0].to(dev)
    kc_b, vc_b = kc_a.clone(), vc_a.clone()
    ws = ops.attn_workspace(case.nq, sh.nh, sh.nkv, n_split, dev)
    cs = ops.rope_rows(ifr, pos, case.nq)
    for dt in (torch.bfloat16, torch.float32):
        out_a = torch.empty(case.nq, sh.nh * HD, dtype=dt, device=dev)
        out_b = torch.empty_like(out_a)
        ops.decode_layer(qkv, qn, kn, wl.EPS, cs, pos, kc_a, vc_a, case.bound, sh.scale, ws, n_split, out_a,
                         sh.nh, sh.nkv)
        ops.decode_layer(qkv_p, qn, kn, wl.EPS, cs, pos, kc_b, vc_b, case.bound, sh.scale, ws, n_split, out_b,
                         sh.nh, sh.nkv)
        torch.cuda.synchronize()
        assert torch.equal(out_a, out_b), f"outputs differ ({dt})"
        assert torch.equal(kc_a, kc_b) and torch.equal(vc_a, vc_b), "KV rows differ"


@pytest.mark.parametrize("group,nq", [(1, 1), (8, 1), (1, 5), (8, 4)])
def test_decode_layer_query_groups_1_and_8(gpu, group, nq):
    """Query groups 1 and 8 (the split kernels serve 1, 2, 4 and 8; the Qwen3 shapes use 2 and 4):
    the fused layer equals the two-launch path bit for bit (KV rows and output) and the
    reference's bf16 ops within the bf16 bar, for one new token (lane kernel) and for several
    (MFMA kernel)."""
    dev = gpu
    nkv, max_len, bound, n_split, pos0 = 4, 512, 512, 16, 300
    nh = nkv * group
    width = (nh + 2 * nkv) * HD
    scale = HD ** -0.5
    g = torch.Generator().manual_seed(4000 + 10 * group + nq)
    kc0 = torch.zeros(max_len, nkv, HD)
    vc0 = torch.zeros(max_len, nkv, HD)
    kc0[:pos0] = torch.randn(pos0, nkv, HD, generator=g)
    vc0[:pos0] = torch.randn(pos0, nkv, HD, generator=g)
    kc0, vc0 = kc0.to(torch.bfloat16), vc0.to(torch.bfloat16)
    qkv_c = torch.randn(nq, width, generator=g).to(torch.bfloat16)
    qn_c = (1 + 0.1 * torch.randn(HD, generator=g)).to(torch.bfloat16)
    kn_c = (1 + 0.1 * torch.randn(HD, generator=g)).to(torch.bfloat16)
    _say(f"[group {group} nh={nh} nkv={nkv} nq={nq} pos0={pos0} bound={bound} n_split={n_split}]")
    ifr = _ifr(dev)
    pos = torch.tensor([pos0], dtype=torch.long, device=dev)
    qkv, qn, kn = qkv_c.to(dev), qn_c.to(dev), kn_c.to(dev)
    kc_a, vc_a = kc0.to(dev), vc0.to(dev)
    kc_b, vc_b = kc_a.clone(), vc_a.clone()
    q = torch.empty(nq, nh, HD, dtype=torch.bfloat16, device=dev)
    ws = ops.attn_workspace(nq, nh, nkv, n_split, dev)
    out_a = torch.empty(nq, nh * HD, dtype=torch.bfloat16, device=dev)
    out_b = torch.empty_like(out_a)
    ops.qknorm_rope_kvwrite(qkv, qn, kn, wl.EPS, ifr, pos, q, kc_a, vc_a, nh, nkv)
    (ops.decode_attn if nq == 1 else ops.verify_attn)(q, kc_a, vc_a, pos, bound, scale, ws, n_split, out_a)
    ops.decode_layer(qkv, qn, kn, wl.EPS, ops.rope_rows(ifr, pos, nq), pos, kc_b, vc_b, bound, scale, ws, n_split,
                     out_b, nh, nkv)
    torch.cuda.synchronize()
    assert torch.equal(kc_a, kc_b) and torch.equal(vc_a, vc_b), "KV rows differ"
    assert torch.equal(out_a, out_b), "outputs differ"
    cos, sin = _tables(dev, max_len)
    rows = torch.arange(pos0, pos0 + nq)
    c, sn = cos.cpu()[rows], sin.cpu()[rows]
    qr, kr, vr = ref.prologue(qkv_c, qn_c, kn_c, wl.EPS, torch.cat([c, c], -1), torch.cat([sn, sn], -1), nh, nkv)
    kc_r, vc_r = kc0.clone(), vc0.clone()
    ref.write_kv(kc_r, vc_r, kr, vr, pos0)
    if nq == 1:
        want = ref.decode_attn(qr, kc_r, vc_r, pos0, bound, scale)
    else:
        want = ref.verify_attn(qr, kc_r, vc_r, pos0, scale)
    _check_bf16(out_b, want, f"  group {group} nq={nq} bf16 vs reference ops")


def test_device_rope_table_equals_torch_table(gpu):
    """The library's cos/sin kernel reproduces torch's table (the reference's expression) bit for bit
    for every position of the longest cache served (32768)."""
    rows = 32768
    cos_t, sin_t = ops.rope_tables(rows, HD, wl.THETA, gpu)
    cos_k, sin_k = ops.rope_tables_device(_ifr(gpu), rows)
    torch.cuda.synchronize()
    dc = (cos_k.view(torch.int16) != cos_t.view(torch.int16)).sum().item()
    ds = (sin_k.view(torch.int16) != sin_t.view(torch.int16)).sum().item()
    _say(f"[rope table] differing cos {dc}, sin {ds} of {rows * 64}")
    assert dc == 0 and ds == 0


def test_accept_prefix_equals_reference_expression(gpu):
    """solort_accept_prefix against cuda_graph_executor.py:476 (restated in oracle/ref.py) on planted
    mismatch positions, k up to 1000 (several 64-pair scans)."""
    g = torch.Generator().manual_seed(32)
    out = torch.zeros(2, dtype=torch.long, device=gpu)
    n = 0
    for k in (1, 4, 63, 64, 65, 200, 1000):
        for miss in sorted({0, 1 % k, k // 2, k - 1, k}):
            draft = torch.randint(0, 151936, (k,), generator=g)
            tg = torch.cat([draft.clone(), torch.randint(0, 151936, (1,), generator=g)])
            if miss < k:
                tg[miss] = (draft[miss] + 7) % 151936
            out.fill_(-5)
            ops.accept_prefix(tg.to(gpu), draft.to(gpu), out)
            torch.cuda.synchronize()
            assert tuple(out.cpu().tolist()) == ref.accept_prefix(tg, draft), (k, miss)
            n += 1
    _say(f"  accept_prefix: {n} cases equal")
