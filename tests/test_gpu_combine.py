"""In-launch split merge: the placement it relies on, and equality with the two-launch combine.

With more than one split, each split stores its partial tagged with this launch's value of the
KV head's counter; the last min(n_split, rows) splits of each head poll for the tags and merge
one row each, in the XCD's L2 that all of the head's splits share.  These tests check the
workgroup -> XCD placement on this device, and that both combine modes give the same bits
(outputs and cache rows) for both split kernels (short chunks of one token, long chunks and
several tokens), query groups 1 to 8, fewer splits than rows, split counts that are not
multiples of 8, empty splits and 16 KV heads; over many consecutive calls (each call must
advance the counters so that no partial of an earlier call is taken for a fresh one), over
calls of different shapes sharing one workspace, and over graph replays.
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
    assert lib.solort_combine_mode(-1) == 1, "solort_init did not enable the in-launch merge"


def test_read_probe_reads_every_byte(lib, gpu):
    g = torch.Generator().manual_seed(5)
    data = torch.randint(-2**31, 2**31 - 1, (1 << 20,), generator=g, dtype=torch.int64).to(torch.int32)
    want = int(np.bitwise_xor.reduce(data.numpy().view(np.uint32)))  # xor of every 32-bit word
    src = data.to(gpu)
    for n_wg, inflight in ((256, 1), (512, 2), (37, 4), (300, 2 | 16), (64, 4 | 16)):  # +16: non-temporal loads
        sink = torch.zeros(n_wg, dtype=torch.int32, device=gpu)
        _lib.check(lib.solort_probe_read(src.data_ptr(), src.numel() * 4, n_wg, inflight, sink.data_ptr(),
                                         torch.cuda.current_stream().cuda_stream), "probe_read")
        torch.cuda.synchronize()
        got = int(np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32)))
        assert got == want, (n_wg, inflight)


def test_read_heads_probe_reads_every_byte_once(lib, gpu):
    g = torch.Generator().manual_seed(6)
    for rows, nkv, n_split, d in ((1024, 8, 8, 1), (4096, 8, 32, 2), (512, 2, 1, 1), (384, 4, 3, 2), (1024, 8, 2, 2),
                                  (768, 2, 2, 2)):
        kv = torch.randint(-2**31, 2**31 - 1, (2, rows * nkv * 64), generator=g, dtype=torch.int64).to(torch.int32)
        want = int(np.bitwise_xor.reduce(kv.numpy().view(np.uint32).ravel()))  # xor of every word of k and v
        k, v = kv[0].to(gpu), kv[1].to(gpu)
        sink = torch.zeros(nkv * n_split, dtype=torch.int32, device=gpu)
        _lib.check(lib.solort_probe_read_heads(k.data_ptr(), v.data_ptr(), rows, nkv, n_split, d, sink.data_ptr(),
                                               torch.cuda.current_stream().cuda_stream), "probe_read_heads")
        torch.cuda.synchronize()
        got = int(np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32)))
        assert got == want, (rows, nkv, n_split, d)


# (name, nh, nkv, max_len, bound, pos, n_split, nq)
CASES = [
    ("8B KV 32768", 32, 8, 32768, 32768, 32767, 32, 1),
    ("4B KV 16384, 16 splits", 32, 8, 16384, 16384, 12000, 16, 1),
    ("4B early position, most splits empty", 32, 8, 16384, 16384, 700, 16, 1),
    ("group 2 (0.6B shape)", 16, 8, 8192, 8192, 5000, 8, 1),
    ("group 1, chunk 512", 8, 8, 4096, 4096, 4000, 8, 1),
    ("group 8", 64, 8, 8192, 8192, 7777, 16, 1),
    ("2 tokens, group 4", 32, 8, 8192, 8192, 6000, 16, 2),
    ("16 KV heads", 64, 16, 8192, 8192, 6500, 8, 1),
    # short chunks (the lane-parallel split kernel)
    ("8B KV 1024, 32 splits", 32, 8, 1024, 1024, 1000, 32, 1),
    ("8B KV 1024, 64 splits of 16 keys", 32, 8, 1024, 1024, 1023, 64, 1),
    ("0.6B KV 1024, 513 keys", 16, 8, 1024, 1024, 512, 32, 1),
    ("group 8, 64 splits", 64, 8, 2048, 2048, 2047, 64, 1),
    ("group 1, 12 splits", 8, 8, 384, 384, 300, 12, 1),
    ("2 splits for 4 rows", 32, 8, 64, 64, 40, 2, 1),
    ("20 splits, 4 empty", 32, 8, 1024, 1000, 999, 20, 1),
    ("16 KV heads, short chunks", 64, 16, 1024, 1024, 777, 32, 1),
    # verify: 5 tokens, 20 rows per KV head (both modes combine in a second launch)
    ("verify, 32 splits", 32, 8, 4096, 4096, 2048, 32, 5),
    ("verify, 8 splits for 20 rows", 32, 8, 4096, 4096, 3000, 8, 5),
]


def _inputs(nh, nkv, max_len, nq, seed):
    g = torch.Generator().manual_seed(seed)
    kc = torch.randn(max_len, nkv, HD, generator=g).to(torch.bfloat16)
    vc = torch.randn(max_len, nkv, HD, generator=g).to(torch.bfloat16)
    qkv = torch.randn(nq, (nh + 2 * nkv) * HD, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(2, HD, generator=g)).to(torch.bfloat16)
    return kc, vc, qkv, w


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_in_launch_merge_equals_two_launch(lib, gpu, case):
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


@pytest.mark.parametrize("max_len,ns,first", [(8192, 16, 5000), (1024, 32, 600)], ids=["long chunks", "short chunks"])
def test_in_launch_merge_repeated_calls_and_graph_replays(lib, gpu, max_len, ns, first):
    """Consecutive calls at moving positions (each call must advance the counters), then one graph
    of 12 calls replayed with eager work between the replays: every result equals the two-launch
    combine's."""
    nh, nkv = 32, 8
    _say(f"[repeated calls] max_len={max_len} n_split={ns}")
    kc0, vc0, qkv, w = _inputs(nh, nkv, max_len, 1, 4242)
    qkv, w = qkv.to(gpu), w.to(gpu)
    inv = ops.inv_freq(HD, wl.THETA, gpu)
    positions = list(range(first, max_len, (max_len - first) // 33 + 1))

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
    posb = torch.tensor([max_len - 7], dtype=torch.long, device=gpu)
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


def test_shapes_sharing_one_workspace(lib, gpu):
    """Calls of different shapes (rows per head, split counts, KV heads) in turn on one workspace:
    a partial left by one shape lies where another shape polls, and must never pass for fresh.
    Every result equals the two-launch combine's on a workspace of its own."""
    # (nq, nh, nkv, max_len, pos, n_split)
    shapes = [(1, 32, 8, 1024, 1000, 32), (5, 32, 8, 4096, 3000, 32), (1, 64, 16, 1024, 900, 16),
              (1, 16, 8, 2048, 2000, 64), (2, 32, 8, 8192, 6000, 16), (1, 8, 8, 384, 300, 12)]
    inv = ops.inv_freq(HD, wl.THETA, gpu)
    data = []
    for i, (nq, nh, nkv, max_len, pos, ns) in enumerate(shapes):
        kc, vc, qkv, w = _inputs(nh, nkv, max_len, nq, 77 + i)
        posb = torch.tensor([pos], dtype=torch.long, device=gpu)
        data.append((kc, vc, qkv.to(gpu), w.to(gpu), posb, ops.rope_rows(inv, posb, nq)))

    def call(i, ws):
        nq, nh, nkv, max_len, pos, ns = shapes[i]
        kc0, vc0, qkv, w, posb, cs = data[i]
        kc, vc = kc0.to(gpu), vc0.to(gpu)
        out = torch.empty(nq, nh * HD, dtype=torch.bfloat16, device=gpu)
        ops.decode_layer(qkv, w[0], w[1], wl.EPS, cs, posb, kc, vc, max_len, HD ** -0.5, ws, ns, out, nh, nkv)
        return out

    lib.solort_combine_mode(0)
    want = []
    for i, (nq, nh, nkv, max_len, pos, ns) in enumerate(shapes):
        want.append(call(i, ops.attn_workspace(nq, nh, nkv, ns, gpu)).cpu())
    lib.solort_combine_mode(1)
    need = max(lib.solort_attn_workspace_bytes(nq, nh, nkv, HD, ns) for nq, nh, nkv, _, _, ns in shapes)
    ws = torch.zeros(need, dtype=torch.uint8, device=gpu)
    order = [0, 1, 2, 3, 4, 5, 1, 0, 3, 2, 5, 4, 0, 0, 1, 1, 2, 3, 4, 5, 0]
    for n, i in enumerate(order):
        _say(f"[shared workspace] call {n}: shape {shapes[i]}")
        got = call(i, ws)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), want[i]), (n, shapes[i])
