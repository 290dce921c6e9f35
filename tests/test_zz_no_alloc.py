"""The allocation-free decode layer (solort_decode_layer_noalloc), called through the C ABI.

It must give solort_decode_layer's bits (output and the new K/V rows) with the partials in the
library's fixed scratch array: on two calls in a row, the second with a smaller input (the array
keeps the first call's contents: counters and partials), for both split kernels, with the splits
merged in the same launch (up to 8 query rows per KV head) or by the combine kernel (the 5-token
verify).  A request above the array's size is refused before any launch.
"""
from __future__ import annotations

import ctypes
import sys

import pytest
import torch

from solort_amd import _lib, ops
from solort_amd import workloads as wl

pytestmark = pytest.mark.gpu
HD = 128
EINVAL = -22


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _case(nh, nkv, max_len, nq, seed):
    g = torch.Generator().manual_seed(seed)
    kc = torch.randn(max_len, nkv, HD, generator=g).to(torch.bfloat16)
    vc = torch.randn(max_len, nkv, HD, generator=g).to(torch.bfloat16)
    qkv = torch.randn(nq, (nh + 2 * nkv) * HD, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(2, HD, generator=g)).to(torch.bfloat16)
    return kc, vc, qkv, w


def _call_both(gpu, lib, nh, nkv, max_len, bound, pos, ns, nq, dtype, seed):
    """One call of each entry point on identical inputs; returns ((out, K rows, V rows) x 2)."""
    kc0, vc0, qkv, w = _case(nh, nkv, max_len, nq, seed)
    qkv, w = qkv.to(gpu), w.to(gpu)
    posb = torch.tensor([pos], dtype=torch.long, device=gpu)
    cs = ops.rope_rows(ops.inv_freq(HD, wl.THETA, gpu), posb, nq)
    dt = 1 if dtype == torch.float32 else 0
    stream = torch.cuda.current_stream().cuda_stream
    res = []
    for noalloc in (False, True):
        kc, vc = kc0.to(gpu), vc0.to(gpu)
        out = torch.full((nq, nh * HD), float("nan"), dtype=dtype, device=gpu)
        common = (qkv.data_ptr(), qkv.stride(0), nq, nh, nkv, HD, w[0].data_ptr(), w[1].data_ptr(), wl.EPS,
                  cs.data_ptr(), posb.data_ptr(), kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1), max_len,
                  bound, HD ** -0.5)
        if noalloc:
            rc = lib.solort_decode_layer_noalloc(*common, ns, out.data_ptr(), dt, stream)
        else:
            ws = ops.attn_workspace(nq, nh, nkv, ns, gpu)
            rc = lib.solort_decode_layer(*common, ws.data_ptr(), ns, out.data_ptr(), dt, stream)
        _lib.check(rc, "decode_layer_noalloc" if noalloc else "decode_layer")
        torch.cuda.synchronize()
        res.append((out.cpu(), kc[pos:pos + nq].cpu(), vc[pos:pos + nq].cpu()))
    return res


# (name, nh, nkv, max_len, bound, pos, n_split, nq): first call, then a smaller one
PAIRS = [
    (("Qwen3-8B KV 32768", 32, 8, 32768, 32768, 32767, 32, 1),
     ("KV 8192, 16 splits", 32, 8, 8192, 8192, 5000, 16, 1)),
    (("Qwen3-4B verify, 5 tokens over 4096", 32, 8, 4096, 4096, 2048, 32, 5),
     ("Qwen3-4B decode KV 1024", 32, 8, 1024, 1024, 1023, 32, 1)),
    (("Qwen3-4B decode KV 1024", 32, 8, 1024, 1024, 1023, 32, 1),
     ("Qwen3-0.6B decode KV 512", 16, 8, 1024, 1024, 512, 16, 1)),
]


@pytest.mark.parametrize("pair", PAIRS, ids=[f"{a[0]} then {b[0]}" for a, b in PAIRS])
def test_noalloc_equals_decode_layer_twice(gpu, pair):
    lib = _lib.load()
    for i, (name, nh, nkv, max_len, bound, pos, ns, nq) in enumerate(pair):
        for dtype in (torch.bfloat16, torch.float32):
            _say(f"[call {i + 1}: {name}, {dtype}]")
            (o1, k1, v1), (o2, k2, v2) = _call_both(gpu, lib, nh, nkv, max_len, bound, pos, ns, nq, dtype, 77 + i)
            assert not torch.isnan(o2).any()
            assert torch.equal(o1, o2), name
            assert torch.equal(k1, k2) and torch.equal(v1, v2), name


def _scratch_bytes() -> int:
    """SOLORT_NOALLOC_SCRATCH_BYTES as include/solort_hip.h defines it."""
    import re
    from pathlib import Path
    text = (Path(__file__).resolve().parents[1] / "include" / "solort_hip.h").read_text()
    m = re.search(r"#define SOLORT_NOALLOC_SCRATCH_BYTES\s+\(?\s*(\d+)u?\s*(?:<<\s*(\d+))?", text)
    assert m, "SOLORT_NOALLOC_SCRATCH_BYTES not found in include/solort_hip.h"
    return int(m.group(1)) << int(m.group(2) or 0)


def test_noalloc_refuses_requests_above_the_scratch(gpu):
    lib = _lib.load()
    p = ctypes.c_void_p(16 * 1024)  # never dereferenced
    nh, nkv, nq, ns = 64, 8, 4, 1024  # 8 heads x 1024 splits x 32 rows x 1040 B
    need = lib.solort_attn_workspace_bytes(nq, nh, nkv, HD, ns)
    assert need > _scratch_bytes()
    # The caches, the position and the output are NULL: were the size check ever to pass, the
    # argument checks would still refuse the call before any launch.
    rc = lib.solort_decode_layer_noalloc(p, (nh + 2 * nkv) * HD, nq, nh, nkv, HD, p, p, 1e-6, p, None, None, None,
                                         1024, 128, 65536, 65536, 0.088, ns, None, 0, None)
    assert rc == EINVAL
    assert "scratch" in lib.solort_last_error().decode()
