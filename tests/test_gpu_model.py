"""Whole-model greedy decode (solort_amd/model.py) on a small seeded Qwen3-shaped model.

Parity: per step, the logits against the CPU restatement of cuda_graph_executor.py:163-190
(oracle/ref.py decode_model_step) fed the same tokens: max-abs <= 6e-2 and mean-abs <= 4e-3 on
logits of spread ~1 (bf16 rounding in a different accumulation order at every one of the ~10 matrix
products and norms on the way), and the greedy token equal to the reference's argmax whenever the
reference's top-two margin exceeds twice the max-abs bar.  The argmax itself is bit-exact (its own
tests).  Graph replays equal eager launches bit for bit.
"""
from __future__ import annotations

import sys

import pytest
import torch

from oracle import ref
from solort_amd.model import GraphQwen3Decode, ModelShape, RandomQwen3

pytestmark = pytest.mark.gpu
TINY = ModelShape("tiny", hidden=512, inter=1024, nh=4, nkv=2, layers=2, vocab=4096, tie_embeddings=True)
# untied: a random tied model greedily repeats its input token (the embedding row scores itself), an
# untied one walks through varied tokens
TINY_UNTIED = ModelShape("tiny-untied", hidden=512, inter=1024, nh=8, nkv=2, layers=3, vocab=4096,
                         tie_embeddings=False)


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _model(gpu, p0, shape=TINY, max_len=256, seed=81):
    w = RandomQwen3(shape, gpu, seed=seed)
    m = GraphQwen3Decode(w, max_len)
    g = torch.Generator(device=gpu).manual_seed(seed + 1)
    kv = (shape.layers, p0, shape.nkv, 128)
    m.kc[:, :p0].copy_(torch.randn(kv, generator=g, device=gpu).to(torch.bfloat16))
    m.vc[:, :p0].copy_(torch.randn(kv, generator=g, device=gpu).to(torch.bfloat16))
    return w, m


def test_decode_graph_replays_equal_eager_steps(gpu):
    p0, n = 120, 12  # crosses the 128 bucket boundary
    _, m = _model(gpu, p0, TINY_UNTIED)
    _, e = _model(gpu, p0, TINY_UNTIED)
    toks = m.generate(7, p0, n)
    e.start(7, p0)
    for i in range(n):
        e._step(e.bucket_for(p0 + i))
    torch.cuda.synchronize()
    assert toks == e.tokens[:n].tolist()
    assert torch.equal(m.kc, e.kc) and torch.equal(m.vc, e.vc)
    assert sorted(m._graphs) == [128, 256]
    assert len(set(toks)) > 1
    # the separate-ops tail (lm_head, argmax, token copy, counter adds, embedding gather) agrees
    w, u = _model(gpu, p0, TINY_UNTIED)
    u2 = GraphQwen3Decode(w, 256, fused_tail=False)
    u2.kc.copy_(u.kc)
    u2.vc.copy_(u.vc)
    assert u2.generate(7, p0, n) == toks and torch.equal(u2.kc, m.kc)
    _say(f"  tokens {toks}")


@pytest.mark.parametrize("shape", [TINY, TINY_UNTIED], ids=lambda s: s.name)
def test_decode_steps_match_reference_ops(gpu, shape):
    """Each step's logits against two CPU evaluations of cuda_graph_executor.py:163-190 fed the same
    tokens: the reference's bf16 arithmetic, and the same weights and cache in fp32 (no intermediate
    rounding).  The device runs bf16 with its own accumulation orders, so it is held to the bf16
    reference's own distance from the fp32 model: mean-abs within 1.5x and max-abs within 2x of it
    (plus 2e-3), and mean-abs under 5% of the logits' spread (a wiring mistake moves the logits by
    about the spread)."""
    p0, n = 60, 6
    w, m = _model(gpu, p0, shape)
    bf = {k: (v.cpu() if torch.is_tensor(v) else [t.cpu() for t in v]) for k, v in vars(w).items() if k != "shape"}
    f32 = {k: (v.float() if torch.is_tensor(v) else [t.float() for t in v]) for k, v in bf.items()}
    kc, vc = m.kc.cpu(), m.vc.cpu()
    kc32, vc32 = kc.float(), vc.float()
    tok = 7
    m.start(tok, p0)
    for i in range(n):
        pos = p0 + i
        bound = m.bucket_for(pos)
        m.graph(bound).replay()
        torch.cuda.synchronize()
        got = m.logits.view(-1).float().cpu()
        want = ref.decode_model_step(bf, tok, pos, kc, vc, bound, shape.nh, shape.nkv).float()
        exact = ref.decode_model_step(f32, tok, pos, kc32, vc32, bound, shape.nh, shape.nkv)
        dg, dr = (got - exact).abs(), (want - exact).abs()
        _say(f"  step {i} pos {pos}: to fp32 model  device mean {dg.mean().item():.3e} max {dg.max().item():.3e}"
             f" | bf16 reference mean {dr.mean().item():.3e} max {dr.max().item():.3e} | spread {exact.std().item():.3f}")
        assert dg.mean().item() <= 1.5 * dr.mean().item() + 2e-3
        assert dg.max().item() <= 2.0 * dr.max().item() + 2e-3
        assert dg.mean().item() <= 0.05 * exact.std().item()
        nxt = int(m.tok.item())
        assert nxt == int(torch.argmax(got).item())  # the device argmax of its own logits
        assert m.tokens[i].item() == nxt and m.step.item() == i + 1 and m.pos.item() == pos + 1
        assert torch.equal(m.x.view(-1), w.embed[nxt])  # the next step's input row
        top2 = torch.topk(exact, 2).values
        if (top2[0] - top2[1]).item() > 2 * dg.max().item():
            assert nxt == int(torch.argmax(exact).item()), i
        _say(f"    token {nxt}")
        tok = nxt  # every path continues from the device's token
    kd = (m.kc.float().cpu() - kc32).abs().max().item()
    kr = (kc.float() - kc32).abs().max().item()
    _say(f"  K rows written: device {kd:.3e}, bf16 reference {kr:.3e} from the fp32 model")
    assert kd <= 2.0 * kr + 2e-3
