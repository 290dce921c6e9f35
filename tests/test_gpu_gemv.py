"""GPU parity of the decode-step GEMVs (solort_gemv) with their fused RMSNorm, residual and SwiGLU.

Bar (floating point): every output within four bf16 ulps (2^-6 relative) plus 2e-3 of the fp64 value
of the same computation on the same bf16 inputs, and mean relative error <= 2e-3.  The kernel's fp32
sums run in a different order than a BLAS, so a result can land one rounding away; a wrong row,
scale, norm or epilogue shows up as errors of order one.  Compared also with the torch restatement
of the reference's ops (oracle/ref.py).  Shapes: Qwen3-4B's fused QKV, o_proj, gate_up and down,
the lm_head, and ragged small ones.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ref
from solort_amd import ops

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _close(got: torch.Tensor, want: np.ndarray, what: str) -> None:
    got = got.float().cpu().numpy().astype(np.float64).reshape(want.shape)
    err = np.abs(got - want)
    rel = err / (np.abs(want) + 1e-3)
    _say(f"  {what}: max-abs {err.max():.3e}, mean rel {rel.mean():.3e}, worst ulp-scaled "
         f"{(err / (np.abs(want) * 2 ** -8 + 1e-6)).max():.2f}")
    assert (err <= np.abs(want) * 2 ** -6 + 2e-3).all(), what
    assert rel.mean() <= 2e-3, what


def _data(n_rows, k, seed):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(n_rows, k, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(k, generator=g).to(torch.bfloat16)
    nw = (torch.randn(k, generator=g) * 0.1 + 1).to(torch.bfloat16)
    return w, x, nw


@pytest.mark.parametrize("n,k,norm", [(6144, 2560, True), (151936, 2560, True), (7, 24, False), (1000, 136, True),
                                      (2560, 4096, False)], ids=["qkv", "lm_head", "tiny", "odd", "plain"])
def test_gemv_plain(gpu, n, k, norm):
    _say(f"[gemv plain n={n} k={k} norm={norm}]")
    w, x, nw = _data(n, k, 40 + n % 97)
    out = torch.empty(n, dtype=torch.bfloat16, device=gpu)
    ops.gemv(w.to(gpu), x.to(gpu), out, nw.to(gpu) if norm else None, 1e-6)
    torch.cuda.synchronize()
    xin = ref.rmsnorm(x.view(1, k), nw, 1e-6).view(k) if norm else x
    _close(out, w.double().numpy() @ xin.double().numpy(), "vs fp64 of the same bf16 input")
    _close(out, ref.linear(xin.view(1, k), w).float().numpy().reshape(n).astype(np.float64), "vs torch ops")


@pytest.mark.parametrize("n,k", [(2560, 4096), (2560, 9728), (33, 520)], ids=["o_proj", "down", "small"])
def test_gemv_residual_in_place(gpu, n, k):
    _say(f"[gemv residual n={n} k={k}]")
    w, x, _ = _data(n, k, 50 + k % 97)
    g = torch.Generator().manual_seed(51)
    res = torch.randn(n, generator=g).to(torch.bfloat16)
    buf = res.to(gpu).clone()
    ops.gemv(w.to(gpu), x.to(gpu), buf, res=buf, mode=ops.GEMV_RESID)  # x = x + W ctx, in place
    torch.cuda.synchronize()
    lin = ref.linear(x.view(1, k), w).view(n)
    want = (res.double() + lin.double()).numpy()
    _close(buf, want, "vs fp64 of res + bf16(W x)")
    _close(buf, (res + lin).float().numpy().astype(np.float64), "vs torch ops")


@pytest.mark.parametrize("inter,k", [(9728, 2560), (100, 264)], ids=["gate_up", "small"])
def test_gemv_swiglu(gpu, inter, k):
    _say(f"[gemv swiglu inter={inter} k={k}]")
    w, x, nw = _data(2 * inter, k, 60 + inter % 97)
    out = torch.empty(inter, dtype=torch.bfloat16, device=gpu)
    ops.gemv(w.to(gpu), x.to(gpu), out, nw.to(gpu), 1e-6, mode=ops.GEMV_SWIGLU, inter=inter)
    torch.cuda.synchronize()
    h2 = ref.rmsnorm(x.view(1, k), nw, 1e-6)
    gate, up = ref.linear(h2, w).split(inter, dim=-1)
    want = (F.silu(gate) * up).view(inter)
    g64, u64 = gate.double().view(inter).numpy(), up.double().view(inter).numpy()
    _close(out, g64 / (1 + np.exp(-g64)) * u64, "vs fp64 silu(g) * u of the bf16 g, u")
    _close(out, want.float().numpy().astype(np.float64), "vs torch ops")


def test_decode_mlp_block_chain(gpu):
    """o_proj + residual, post-norm + gate_up + SwiGLU, down + residual: the reference's layer tail."""
    K, I = 2560, 9728
    g = torch.Generator().manual_seed(70)
    x = torch.randn(K, generator=g).to(torch.bfloat16)
    ctx = torch.randn(4096, generator=g).to(torch.bfloat16)
    wo = (torch.randn(K, 4096, generator=g) * 0.02).to(torch.bfloat16)
    ln = (torch.randn(K, generator=g) * 0.1 + 1).to(torch.bfloat16)
    wgu = (torch.randn(2 * I, K, generator=g) * 0.02).to(torch.bfloat16)
    wd = (torch.randn(K, I, generator=g) * 0.02).to(torch.bfloat16)
    xd, act = x.to(gpu), torch.empty(I, dtype=torch.bfloat16, device=gpu)
    ops.gemv(wo.to(gpu), ctx.to(gpu), xd, res=xd, mode=ops.GEMV_RESID)
    ops.gemv(wgu.to(gpu), xd, act, ln.to(gpu), 1e-6, mode=ops.GEMV_SWIGLU, inter=I)
    ops.gemv(wd.to(gpu), act, xd, res=xd, mode=ops.GEMV_RESID)
    torch.cuda.synchronize()
    want = ref.decode_mlp_block(x.view(1, K), ctx.view(1, 4096), wo, ln, wgu, wd, 1e-6).view(K)
    err = (xd.float().cpu() - want.float()).abs()
    _say(f"  chain vs torch ops: max-abs {err.max().item():.3e} mean-abs {err.mean().item():.3e}")
    assert err.max().item() <= 5e-2 and err.mean().item() <= 2e-3


@pytest.mark.parametrize("n,k,norm", [(151936, 2560, True), (151936, 4096, False), (4099, 136, True), (1, 8, False)],
                         ids=["lm_head_4b", "lm_head_8b", "odd", "one"])
def test_gemv_argmax_equals_gemv_then_argmax(gpu, n, k, norm):
    """The fused lm_head + argmax: logits bit-identical to solort_gemv's, index bit-identical to
    solort_argmax_rows over them and equal to the first maximum of those logits, including exact ties
    planted by duplicating the winning row at a lower and a higher index, and a NaN row (NaN ranks
    highest, the first NaN wins).  The workspaces are reused across all calls."""
    _say(f"[gemv_argmax n={n} k={k} norm={norm}]")
    w, x, nw = _data(n, k, 70 + n % 89)
    w, x, nw = w.to(gpu), x.to(gpu), nw.to(gpu) if norm else None
    ws = ops.argmax_workspace(1, gpu)
    gws = ops.gemv_argmax_workspace(n, gpu)
    want_logits = torch.empty(n, dtype=torch.bfloat16, device=gpu)
    got_logits = torch.empty(n, dtype=torch.bfloat16, device=gpu)
    idx, idx2, idx_ref = (torch.full((1,), -1, dtype=torch.long, device=gpu) for _ in range(3))

    def check(what):
        ops.gemv(w, x, want_logits, nw, 1e-6)
        ops.argmax_rows(want_logits.view(1, n), idx_ref, ws)
        ops.gemv_argmax(w, x, idx, gws, nw, 1e-6, logits=got_logits)
        ops.gemv_argmax(w, x, idx2, gws, nw, 1e-6)  # without the logits
        torch.cuda.synchronize()
        first = int(torch.argmax(want_logits.float()).item())
        _say(f"  {what}: index {idx.item()} (argmax_rows {idx_ref.item()}, first max {first})")
        assert torch.equal(got_logits.view(torch.int16), want_logits.view(torch.int16)), what  # bits (NaN too)
        assert idx.item() == idx_ref.item() == idx2.item() == first, what

    check("random")
    if n < 3:
        return
    j = int(idx.item())
    lo, hi = (j // 2, min(n - 1, j + 1 + (n - j) // 2)) if j > 0 else (0, min(n - 1, 1 + n // 2))
    w[lo].copy_(w[j])
    w[hi].copy_(w[j])
    check(f"tie planted at {lo} and {hi}")
    w[hi, 3] = float("nan")
    w[min(n - 1, hi + 1), 0] = float("nan")
    check(f"NaN rows {hi} and {min(n - 1, hi + 1)}")


def test_greedy_advance_after_gemv_argmax(gpu):
    """solort_gemv_argmax with no out_idx leaves the keys; solort_greedy_advance turns them into the
    next input token (equal to the argmax of the logits), records it at tokens[step] while step is
    below the list's length, advances step and pos, and copies the token's embedding row into x."""
    n, k, hidden = 4099, 136, 64
    w, x, nw = _data(n, k, 91)
    w, x, nw = w.to(gpu), x.to(gpu), nw.to(gpu)
    embed = torch.randn(n, hidden, device=gpu).to(torch.bfloat16)
    gws = ops.gemv_argmax_workspace(n, gpu)
    logits = torch.empty(n, dtype=torch.bfloat16, device=gpu)
    xo = torch.zeros(hidden, dtype=torch.bfloat16, device=gpu)
    tok = torch.full((1,), -1, dtype=torch.long, device=gpu)
    tokens = torch.full((4,), -1, dtype=torch.long, device=gpu)
    step = torch.tensor([3], dtype=torch.long, device=gpu)
    pos = torch.tensor([17], dtype=torch.long, device=gpu)
    first = None
    for call in range(2):
        ops.gemv_argmax(w, x, None, gws, nw, 1e-6, logits=logits)
        ops.greedy_advance(gws, n, embed, xo, tok, tokens, step, pos)
        torch.cuda.synchronize()
        t = int(torch.argmax(logits.float()).item())
        _say(f"  call {call}: token {tok.item()} (first max {t}), tokens {tokens.tolist()}, step {step.item()}, "
             f"pos {pos.item()}")
        assert tok.item() == t and torch.equal(xo, embed[t])
        assert step.item() == 4 + call and pos.item() == 18 + call
        first = t if first is None else first
        assert tokens.tolist() == [-1, -1, -1, first]  # the second call's step 4 is past the list
        x = (x.float() * -1.5).to(torch.bfloat16)  # another argmax for the second call


def test_greedy_advance_never_embeds_a_row_outside_the_table(gpu):
    """Keys that name no vocabulary row (a workspace no solort_gemv_argmax call filled: all zero
    here, which decodes to index 2^32 - 1) are recorded as token -1, the error the host checks, while
    row 0 is embedded and step and pos still advance: no row outside the table is read."""
    n, hidden = 4099, 64
    embed = torch.randn(n, hidden, device=gpu).to(torch.bfloat16)
    gws = ops.gemv_argmax_workspace(n, gpu).zero_()
    xo = torch.zeros(hidden, dtype=torch.bfloat16, device=gpu)
    tok = torch.full((1,), 5, dtype=torch.long, device=gpu)
    tokens = torch.full((2,), 7, dtype=torch.long, device=gpu)
    step = torch.tensor([1], dtype=torch.long, device=gpu)
    pos = torch.tensor([30], dtype=torch.long, device=gpu)
    ops.greedy_advance(gws, n, embed, xo, tok, tokens, step, pos)
    torch.cuda.synchronize()
    assert tokens.tolist() == [7, -1] and tok.item() == 0 and torch.equal(xo, embed[0])
    assert step.item() == 2 and pos.item() == 31
    with pytest.raises(RuntimeError, match="outside the vocabulary"):
        ops.check_tokens(tokens.tolist(), n, "greedy decode")
