"""Decode and verify at the edges of the position range: the first token (one live key), the split
kernels' chunk boundaries (16, 32, 33 keys), a bucket's last slot and the cache's last slot.

Bars as in test_gpu_kernels: the written K/V rows bit for bit against the fixed-order prologue
(oracle/exact.py) fed the device cos/sin table, fp32 outputs within 1e-4 of fp64 attention over the
same bf16 cache (oracle/exact.py causal_decode_fp64), bf16 outputs the rounded fp32 ones.  With one
live key the output is that key's V row exactly (softmax of one score is 1).
"""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import exact
from solort_amd import ops
from solort_amd import workloads as wl
from solort_amd.runner import decode_splits, verify_splits

pytestmark = pytest.mark.gpu
HD = 128


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _check(gpu, pos0, nq, bound, max_len, n_split, seed):
    sh = wl.QWEN3_4B
    g = torch.Generator().manual_seed(seed)
    kc = torch.randn(max_len, sh.nkv, HD, generator=g).to(torch.bfloat16)
    vc = torch.randn(max_len, sh.nkv, HD, generator=g).to(torch.bfloat16)
    qkv = torch.randn(nq, sh.qkv_width, generator=g).to(torch.bfloat16)
    qn = (1 + 0.1 * torch.randn(HD, generator=g)).to(torch.bfloat16)
    kn = (1 + 0.1 * torch.randn(HD, generator=g)).to(torch.bfloat16)
    kd, vd = kc.to(gpu), vc.to(gpu)
    pos = torch.tensor([pos0], dtype=torch.long, device=gpu)
    cs = ops.rope_rows(ops.inv_freq(HD, wl.THETA, gpu), pos, nq)
    ws = ops.attn_workspace(nq, sh.nh, sh.nkv, n_split, gpu)
    out32 = torch.empty(nq, sh.nh * HD, dtype=torch.float32, device=gpu)
    out16 = torch.empty(nq, sh.nh * HD, dtype=torch.bfloat16, device=gpu)
    ops.decode_layer(qkv.to(gpu), qn.to(gpu), kn.to(gpu), wl.EPS, cs, pos, kd, vd, bound, sh.scale, ws, n_split,
                     out32, sh.nh, sh.nkv)
    kd2, vd2 = kc.to(gpu), vc.to(gpu)
    ops.decode_layer(qkv.to(gpu), qn.to(gpu), kn.to(gpu), wl.EPS, cs, pos, kd2, vd2, bound, sh.scale, ws, n_split,
                     out16, sh.nh, sh.nkv)
    cos_t, sin_t = ops.rope_tables(pos0 + nq, HD, wl.THETA, gpu)
    torch.cuda.synchronize()
    q, k, v = exact.prologue_fixed_order(qkv.float().numpy(), qn.float().numpy(), kn.float().numpy(), wl.EPS,
                                         cos_t.cpu()[pos0:].float().numpy(), sin_t.cpu()[pos0:].float().numpy(),
                                         sh.nh, sh.nkv)
    kw, vw = kc.clone(), vc.clone()
    kw[pos0:pos0 + nq] = torch.from_numpy(k).to(torch.bfloat16)
    vw[pos0:pos0 + nq] = torch.from_numpy(v).to(torch.bfloat16)
    assert torch.equal(kd.cpu(), kw) and torch.equal(vd.cpu(), vw), "KV rows differ from the fixed-order oracle"
    qb = torch.from_numpy(q).to(torch.bfloat16).float().numpy()
    want = exact.causal_decode_fp64(qb, kw.float().numpy(), vw.float().numpy(), pos0, sh.scale).reshape(nq, -1)
    err = np.abs(out32.cpu().numpy().astype(np.float64) - want).max()
    _say(f"  pos0={pos0} nq={nq} bound={bound} n_split={n_split}: fp32 vs fp64 {err:.2e}")
    assert err <= 1e-4
    assert torch.equal(out16, out32.to(torch.bfloat16))
    if pos0 == 0 and nq == 1:  # one live key: every head of a group returns its KV head's V row 0
        v0 = vw[0].float().repeat_interleave(sh.group, 0).reshape(1, -1)
        assert torch.equal(out32.cpu(), v0)


@pytest.mark.parametrize("pos0", [0, 1, 15, 16, 31, 32, 33, 127, 128, 255, 1023])
def test_decode_positions(gpu, pos0):
    bound = next(b for b in (128, 256, 512, 1024) if b > pos0)
    _check(gpu, pos0, 1, bound, 1024, decode_splits(bound, 8), 700 + pos0)


@pytest.mark.parametrize("pos0,bound,max_len", [(0, 128, 128), (3, 128, 128), (123, 128, 128), (4091, 4096, 4096)],
                         ids=["start", "start+3", "bucket-end", "cache-end"])
def test_verify_positions(gpu, pos0, bound, max_len):
    _check(gpu, pos0, 5, bound, max_len, verify_splits(bound, 8), 800 + pos0)


def test_decode_single_split_long_chunk(gpu):
    """One split over a whole 4096-key bucket (the MFMA split kernel with 128 tiles, no combine)."""
    _check(gpu, 4000, 1, 4096, 4096, 1, 901)
