"""Single-launch split combine: the placement it relies on, and equality with the two-launch combine.

For long key chunks (the MFMA split kernel), the last split of each KV head to finish merges the
head's partials inside the split kernel; the partials meet in the L2 of the XCD all of the head's
splits run on.  These tests check the workgroup -> XCD placement on this device, and that both
combine modes give the same bits (outputs and cache rows) for query groups 1, 2, 4 and 8, two new
tokens, 16 KV heads and mostly empty splits, over many consecutive calls (each call's last split
must leave the tickets at zero for the next) and over graph replays.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from solort_amd import _lib, ops
from solort_amd import workloads as wl

pytestmark = pytest.mark.gpu

HD = 128


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture
def lib(gpu):
    lib = _lib.load()
    yield lib
    lib.solort_combine_mode(1)


def test_workgroups_round_robin_over_xcds(lib, gpu):
    n = 4096
    out = torch.zeros(2 * n, dtype=torch.int32, device=gpu)
    _lib.check(lib.solort_probe_placement(out.data_ptr(), n, torch.cuda.current_stream().cuda_stream),
               "probe_placement")
    torch.cuda.synchronize()
    xcc = out.view(n, 2)[:, 0].cpu()
    _say(f"XCD of workgroups 0..15: {xcc[:16].tolist()}; distinct XCDs {sorted(set(xcc.tolist()))}")
    assert torch.equal(xcc, xcc[torch.arange(n) % 8]), "workgroup b does not share the XCD of b % 8"
    assert lib.solort_combine_mode(-1) == 1, "solort_init did not enable the single-launch combine"


def test_read_probe_reads_every_byte(lib, gpu):
    g = torch.Generator().manual_seed(5)
    data = torch.randint(-2**31, 2**31 - 1, (1 << 20,), generator=g, dtype=torch.int64).to(torch.int32)
    want = int(np.bitwise_xor.reduce(data.numpy().view(np.uint32)))  # xor of every 32-bit word
    src = data.to(gpu)
    for n_wg, inflight in ((256, 1), (512, 2), (37, 4)):
        sink = torch.zeros(n_wg, dtype=torch.int32, device=gpu)
        _lib.check(lib.solort_probe_read(src.data_ptr(), src.numel() * 4, n_wg, inflight, sink.data_ptr(),
                                         torch.cuda.current_stream().cuda_stream), "probe_read")
        torch.cuda.synchronize()
        got = int(np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32)))
        assert got == want, (n_wg, inflight)


# (name, nh, nkv, max_len, bound, pos, n_split, nq): long chunks (at least 512 keys per split, the
# MFMA split kernel), where the combine runs in the split kernel's launch
CASES = [
    ("8B KV 32768", 32, 8, 32768, 32768, 32767, 32, 1),
    ("4B KV 16384, 16 splits", 32, 8, 16384, 16384, 12000, 16, 1),
    ("4B early position, most splits empty", 32, 8, 16384, 16384, 700, 16, 1),
    ("group 2 (0.6B shape)", 16, 8, 8192, 8192, 5000, 8, 1),
    ("group 1, chunk 512", 8, 8, 4096, 4096, 4000, 8, 1),
    ("group 8", 64, 8, 8192, 8192, 7777, 16, 1),
    ("2 tokens, group 4", 32, 8, 8192, 8192, 6000, 16, 2),
    ("16 KV heads", 64, 16, 8192, 8192, 6500, 8, 1),
]


def _inputs(nh, nkv, max_len, nq, seed):
    g = torch.Generator().manual_seed(seed)
    kc = torch.randn(max_len, nkv, HD, generator=g).to(torch.bfloat16)
    vc = torch.randn(max_len, nkv, HD, generator=g).to(torch.bfloat16)
    qkv = torch.randn(nq, (nh + 2 * nkv) * HD, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(2, HD, generator=g)).to(torch.bfloat16)
    return kc, vc, qkv, w


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_single_launch_equals_two_launch(lib, gpu, case):
    name, nh, nkv, max_len, bound, pos, ns, nq = case
    _say(f"[{name}] nh={nh} nkv={nkv} bound={bound} pos={pos} n_split={ns} nq={nq}")
    kc0, vc0, qkv, w = _inputs(nh, nkv, max_len, nq, 900 + nh + nkv + nq)
    qkv, w = qkv.to(gpu), w.to(gpu)
    posb = torch.tensor([pos], dtype=torch.long, device=gpu)
    cs = ops.rope_rows(ops.inv_freq(HD, wl.THETA, gpu), posb, nq)
    res = {}
    for mode in (0, 1):
        assert lib.solort_combine_mode(mode) == mode
        ws = ops.attn_workspace(nq, nh, nkv, ns, gpu)
        outs = []
        for dt in (torch.bfloat16, torch.float32):
            kc, vc = kc0.to(gpu), vc0.to(gpu)
            out = torch.empty(nq, nh * HD, dtype=dt, device=gpu)
            ops.decode_layer(qkv, w[0], w[1], wl.EPS, cs, posb, kc, vc, bound, HD ** -0.5, ws, ns, out, nh, nkv)
            torch.cuda.synchronize()
            outs.append((out.cpu(), kc[pos:pos + nq].cpu(), vc[pos:pos + nq].cpu()))
        res[mode] = outs
        assert not torch.isnan(outs[1][0]).any()
    for a, b in zip(res[0], res[1]):
        for x, y in zip(a, b):
            assert torch.equal(x, y), name


def test_single_launch_repeated_calls_and_graph_replays(lib, gpu):
    """Consecutive calls at moving positions (each call's last split must clear the tickets), then
    one graph of 12 calls replayed with eager work between the replays: every result equals the
    two-launch combine's."""
    nh, nkv, max_len, ns = 32, 8, 8192, 16
    kc0, vc0, qkv, w = _inputs(nh, nkv, max_len, 1, 4242)
    qkv, w = qkv.to(gpu), w.to(gpu)
    inv = ops.inv_freq(HD, wl.THETA, gpu)
    positions = list(range(5000, 8192, 97))

    def run(mode):
        lib.solort_combine_mode(mode)
        ws = ops.attn_workspace(1, nh, nkv, ns, gpu)
        kc, vc = kc0.to(gpu), vc0.to(gpu)
        outs = []
        for p in positions:
            posb = torch.tensor([p], dtype=torch.long, device=gpu)
            out = torch.empty(1, nh * HD, dtype=torch.bfloat16, device=gpu)
            ops.decode_layer(qkv, w[0], w[1], wl.EPS, ops.rope_rows(inv, posb, 1), posb, kc, vc, max_len,
                             HD ** -0.5, ws, ns, out, nh, nkv)
            outs.append(out)
        torch.cuda.synchronize()
        return torch.stack([o.cpu() for o in outs]), kc.cpu(), vc.cpu()

    two, one = run(0), run(1)
    for x, y in zip(two, one):
        assert torch.equal(x, y)

    # graph: 12 layers' calls on distinct caches, replayed 5 times
    lib.solort_combine_mode(1)
    layers = 12
    kcs = [kc0.to(gpu) for _ in range(layers)]
    vcs = [vc0.to(gpu) for _ in range(layers)]
    posb = torch.tensor([8000], dtype=torch.long, device=gpu)
    cs = ops.rope_rows(inv, posb, 1)
    ws = ops.attn_workspace(1, nh, nkv, ns, gpu)
    outs = torch.zeros(layers, 1, nh * HD, dtype=torch.bfloat16, device=gpu)

    def step():
        for li in range(layers):
            ops.decode_layer(qkv, w[0], w[1], wl.EPS, cs, posb, kcs[li], vcs[li], max_len, HD ** -0.5, ws, ns,
                             outs[li], nh, nkv)

    step()
    torch.cuda.synchronize()
    eager = outs.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for r in range(5):
        outs.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(outs, eager), f"replay {r}"
        step()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(outs, eager)
    lib.solort_combine_mode(0)
    step()
    torch.cuda.synchronize()
    assert torch.equal(outs, eager), "two-launch combine differs"
