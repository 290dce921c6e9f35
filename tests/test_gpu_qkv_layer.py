"""The qkv product and attention block in one launch (solort_decode_qkv_layer) against the product
as its own launch followed by solort_decode_layer: the same output and cache bits, on the shapes the
fused kernel serves and on shapes that take the two-launch path."""
import pytest
import torch

from solort_amd import ops
from solort_amd import workloads as wl

pytestmark = pytest.mark.gpu
HD = 128


def _say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


# (name, nh, nkv, hidden, max_len, bound, pos, n_split)
CASES = [
    ("4B KV 1024, 32-key splits", 32, 8, 2560, 1024, 1024, 1023, 32),
    ("4B KV 2048, 64-key splits", 32, 8, 2560, 2048, 2048, 1500, 32),
    ("4B early position", 32, 8, 2560, 1024, 1024, 5, 32),
    ("4B position 0", 32, 8, 2560, 1024, 1024, 0, 32),
    ("0.6B KV 1024", 16, 8, 1024, 1024, 1024, 700, 32),
    ("8B KV 1024", 32, 8, 4096, 1024, 1024, 1000, 32),
    ("4B KV 512, 16-key splits", 32, 8, 2560, 512, 512, 300, 32),
    ("4B KV 4096, 128-key splits (MFMA kernel)", 32, 8, 2560, 4096, 4096, 4000, 32),
    ("4B KV 8192, early position (256-key splits: two launches)", 32, 8, 2560, 8192, 8192, 100, 32),
    ("0.6B KV 4096 (MFMA kernel)", 16, 8, 1024, 4096, 4096, 3000, 32),
    ("8B KV 32768, 1024-key splits (two launches)", 32, 8, 4096, 32768, 32768, 32767, 32),
    ("4B KV 512, 16 splits (two launches)", 32, 8, 2560, 512, 512, 300, 16),
    ("hidden 2048 (two launches)", 32, 8, 2048, 1024, 1024, 800, 32),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_qkv_layer_equals_product_then_layer(gpu, case):
    name, nh, nkv, hidden, max_len, bound, pos, n_split = case
    _say(f"[qkv layer: {name}]")
    g = torch.Generator().manual_seed(900 + pos)
    width = (nh + 2 * nkv) * HD
    scale = HD ** -0.5
    wqkv = (torch.randn(width, hidden, generator=g) * hidden ** -0.5).to(torch.bfloat16).to(gpu)
    in_w = (1.0 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16).to(gpu)
    qn_w = (1.0 + 0.1 * torch.randn(HD, generator=g)).to(torch.bfloat16).to(gpu)
    kn_w = (1.0 + 0.1 * torch.randn(HD, generator=g)).to(torch.bfloat16).to(gpu)
    kc = torch.randn(max_len, nkv, HD, generator=g).to(torch.bfloat16).to(gpu)
    vc = torch.randn(max_len, nkv, HD, generator=g).to(torch.bfloat16).to(gpu)
    kc2, vc2 = kc.clone(), vc.clone()
    posb = torch.tensor([pos], dtype=torch.long, device=gpu)
    cs = ops.rope_rows(ops.inv_freq(HD, wl.THETA, gpu), posb, 1)
    ws_ref = ops.attn_workspace(1, nh, nkv, n_split, gpu)
    ws = ops.decode_qkv_workspace(nh, nkv, n_split, gpu)
    qkv = torch.empty(1, width, dtype=torch.bfloat16, device=gpu)
    scratch = torch.empty(width, dtype=torch.bfloat16, device=gpu)
    for call in range(3):  # consecutive calls: the handed-over rows carry each launch's tag
        x = torch.randn(hidden, generator=g).to(torch.bfloat16).to(gpu)
        want = torch.empty(1, nh * HD, dtype=torch.bfloat16, device=gpu)
        got = torch.empty_like(want)
        ops.gemv(wqkv, x, qkv.view(-1), in_w, wl.EPS)
        ops.decode_layer(qkv, qn_w, kn_w, wl.EPS, cs, posb, kc, vc, bound, scale, ws_ref, n_split, want, nh, nkv)
        ops.decode_qkv_layer(x, in_w, wl.EPS, wqkv, qn_w, kn_w, wl.EPS, cs, posb, kc2, vc2, bound, scale, ws,
                             n_split, scratch, got, nh, nkv)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all(), (name, call)
        assert torch.equal(got, want), (name, call, (got.float() - want.float()).abs().max().item())
        assert torch.equal(kc2, kc) and torch.equal(vc2, vc), (name, call)


def test_qkv_layer_strided_weight_rows(gpu):
    """wqkv rows padded past hidden (row stride hidden + 64): the entry point takes the two-launch
    path, with the same output and cache bits as the product followed by the attention block."""
    nh, nkv, hidden, bound, pos = 32, 8, 2560, 1024, 1000
    _say("[qkv layer: padded weight rows]")
    g = torch.Generator().manual_seed(91)
    width = (nh + 2 * nkv) * HD
    wfull = (torch.randn(width, hidden + 64, generator=g) * hidden ** -0.5).to(torch.bfloat16).to(gpu)
    wqkv = wfull[:, :hidden]
    assert wqkv.stride(0) == hidden + 64
    in_w = (1.0 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16).to(gpu)
    qn_w = (1.0 + 0.1 * torch.randn(HD, generator=g)).to(torch.bfloat16).to(gpu)
    kn_w = (1.0 + 0.1 * torch.randn(HD, generator=g)).to(torch.bfloat16).to(gpu)
    kc = torch.randn(bound, nkv, HD, generator=g).to(torch.bfloat16).to(gpu)
    vc = torch.randn(bound, nkv, HD, generator=g).to(torch.bfloat16).to(gpu)
    kc2, vc2 = kc.clone(), vc.clone()
    posb = torch.tensor([pos], dtype=torch.long, device=gpu)
    cs = ops.rope_rows(ops.inv_freq(HD, wl.THETA, gpu), posb, 1)
    ws = ops.decode_qkv_workspace(nh, nkv, 32, gpu)
    ws_ref = ops.attn_workspace(1, nh, nkv, 32, gpu)
    qkv = torch.empty(1, width, dtype=torch.bfloat16, device=gpu)
    scratch = torch.empty(width, dtype=torch.bfloat16, device=gpu)
    for call in range(3):
        x = torch.randn(hidden, generator=g).to(torch.bfloat16).to(gpu)
        want = torch.empty(1, nh * HD, dtype=torch.bfloat16, device=gpu)
        got = torch.empty_like(want)
        ops.gemv(wqkv, x, qkv.view(-1), in_w, wl.EPS)
        ops.decode_layer(qkv, qn_w, kn_w, wl.EPS, cs, posb, kc, vc, bound, HD ** -0.5, ws_ref, 32, want, nh, nkv)
        ops.decode_qkv_layer(x, in_w, wl.EPS, wqkv, qn_w, kn_w, wl.EPS, cs, posb, kc2, vc2, bound, HD ** -0.5, ws,
                             32, scratch, got, nh, nkv)
        torch.cuda.synchronize()
        assert torch.equal(got, want), call
        assert torch.equal(kc2, kc) and torch.equal(vc2, vc), call
        assert torch.equal(scratch, qkv.view(-1)), call  # the product went through qkv_out


def test_qkv_layer_graph_replays(gpu):
    """A graph of 36 calls over distinct layer caches and weights, replayed several times with eager
    work between the replays, against the two-launch path."""
    nh, nkv, hidden, L, bound, pos = 32, 8, 2560, 36, 1024, 900
    _say("[qkv layer: graph of 36 layers]")
    g = torch.Generator().manual_seed(77)
    width = (nh + 2 * nkv) * HD
    wq = [(torch.randn(width, hidden, generator=g) * hidden ** -0.5).to(torch.bfloat16).to(gpu) for _ in range(4)]
    in_w = (1.0 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16).to(gpu)
    qn_w = (1.0 + 0.1 * torch.randn(HD, generator=g)).to(torch.bfloat16).to(gpu)
    kn_w = (1.0 + 0.1 * torch.randn(HD, generator=g)).to(torch.bfloat16).to(gpu)
    kc = torch.randn(L, bound, nkv, HD, generator=g).to(torch.bfloat16).to(gpu)
    vc = torch.randn(L, bound, nkv, HD, generator=g).to(torch.bfloat16).to(gpu)
    posb = torch.tensor([pos], dtype=torch.long, device=gpu)
    cs = ops.rope_rows(ops.inv_freq(HD, wl.THETA, gpu), posb, 1)
    ws = ops.decode_qkv_workspace(nh, nkv, 32, gpu)
    ws_ref = ops.attn_workspace(1, nh, nkv, 32, gpu)
    xs = torch.randn(L, hidden, generator=g).to(torch.bfloat16).to(gpu)
    out = torch.empty(L, 1, nh * HD, dtype=torch.bfloat16, device=gpu)
    scratch = torch.empty(width, dtype=torch.bfloat16, device=gpu)
    kc2, vc2 = kc.clone(), vc.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for li in range(L):
            ops.decode_qkv_layer(xs[li], in_w, wl.EPS, wq[li % 4], qn_w, kn_w, wl.EPS, cs, posb, kc2[li], vc2[li],
                                 bound, HD ** -0.5, ws, 32, scratch, out[li], nh, nkv)
    qkv = torch.empty(1, width, dtype=torch.bfloat16, device=gpu)
    want = torch.empty_like(out)
    for li in range(L):
        ops.gemv(wq[li % 4], xs[li], qkv.view(-1), in_w, wl.EPS)
        ops.decode_layer(qkv, qn_w, kn_w, wl.EPS, cs, posb, kc[li], vc[li], bound, HD ** -0.5, ws_ref, 32, want[li],
                         nh, nkv)
    for rep in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), rep
        assert torch.equal(kc2, kc) and torch.equal(vc2, vc), rep
