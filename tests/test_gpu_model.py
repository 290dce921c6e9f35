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
from solort_amd.runner import decode_qkv_splits, decode_splits

pytestmark = pytest.mark.gpu
TINY = ModelShape("tiny", hidden=512, inter=1024, nh=4, nkv=2, layers=2, vocab=4096, tie_embeddings=True)
# untied: a random tied model greedily repeats its input token (the embedding row scores itself), an
# untied one walks through varied tokens
TINY_UNTIED = ModelShape("tiny-untied", hidden=512, inter=1024, nh=8, nkv=2, layers=3, vocab=4096,
                         tie_embeddings=False)
# a query group of 8 (as Qwen3-32B's 64 query heads over 8 KV heads), one KV head
TINY_G8 = ModelShape("tiny-g8", hidden=512, inter=1024, nh=8, nkv=1, layers=2, vocab=4096, tie_embeddings=False)
# the Qwen3-4B widths (hidden, intermediate, heads, vocabulary, tied embedding) with two layers
QWEN3_4B_2L = ModelShape("qwen3-4b-2layers", hidden=2560, inter=9728, nh=32, nkv=8, layers=2, vocab=151936,
                         tie_embeddings=True)


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


@pytest.mark.parametrize("p0", [400, 1000, 1500, 3000], ids=["bucket512", "bucket1024", "bucket2048", "bucket4096"])
def test_qkv_in_attention_launch_equals_own_launch(gpu, p0):
    """The Qwen3-4B layer shapes (hidden 2560, 32 q / 8 kv heads, 2 layers) in the buckets where the
    QKV product runs inside the attention launch: the same tokens as the step with the product as
    its own launch, and the same cache bits where both run the attention with the same split count
    (at 512 keys the fused launch runs 32 splits of 16 keys, the attention on its own 16 of 32, so
    the merge adds the partials in another order)."""
    n = 6
    w, m = _model(gpu, p0, QWEN3_4B_2L, max_len=4096)
    u = GraphQwen3Decode(w, 4096, fused_qkv=False)
    u.kc.copy_(m.kc)
    u.vc.copy_(m.vc)
    toks = m.generate(5, p0, n)
    assert u.generate(5, p0, n) == toks
    bound = m.bucket_for(p0)
    if decode_qkv_splits(bound, QWEN3_4B_2L.nkv) == decode_splits(bound, QWEN3_4B_2L.nkv):
        assert torch.equal(u.kc, m.kc) and torch.equal(u.vc, m.vc)
    _say(f"  tokens {toks}")


@pytest.mark.parametrize("shape", [TINY, TINY_UNTIED, TINY_G8, QWEN3_4B_2L], ids=lambda s: s.name)
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


@pytest.mark.parametrize("plen,max_len,shape", [(37, 256, TINY_UNTIED), (300, 512, TINY_UNTIED), (300, 512, TINY_G8)],
                         ids=["bucket64", "bucket512-fused", "g8-bucket512-fused"])
def test_prompt_prefill_then_decode_match_reference_ops(gpu, plen, max_len, shape):
    """Prompt prefill (cuda_graph_executor.py:104-161: library GEMMs around solort_prefill_layer or
    the prologue + solort_prefill_attn) and the decode steps after it, against the CPU evaluations of
    the same model in bf16 and fp32.  The first token's logits and the KV rows of the prompt are
    held to the bf16 reference's own distance from the fp32 model (as the decode steps are); the
    first token is the device argmax of its logits and becomes the decode input at position plen;
    three teacher-forced decode steps follow on each side's own cache."""
    w = RandomQwen3(shape, gpu, seed=83)
    m = GraphQwen3Decode(w, max_len)
    g = torch.Generator().manual_seed(84)
    ids = torch.randint(0, shape.vocab, (plen,), generator=g).tolist()
    bf = {k: (v.cpu() if torch.is_tensor(v) else [t.cpu() for t in v]) for k, v in vars(w).items() if k != "shape"}
    f32 = {k: (v.float() if torch.is_tensor(v) else [t.float() for t in v]) for k, v in bf.items()}
    kv_shape = (shape.layers, max_len, shape.nkv, 128)
    kc, vc = torch.zeros(kv_shape, dtype=torch.bfloat16), torch.zeros(kv_shape, dtype=torch.bfloat16)
    kc32, vc32 = torch.zeros(kv_shape), torch.zeros(kv_shape)
    m.prefill(ids)
    torch.cuda.synchronize()
    got = m.logits.view(-1).float().cpu()
    want = ref.prefill_model(bf, ids, kc, vc, shape.nh, shape.nkv).float()
    exact = ref.prefill_model(f32, ids, kc32, vc32, shape.nh, shape.nkv)
    dg, dr = (got - exact).abs(), (want - exact).abs()
    _say(f"  prefill T={plen}: to fp32 model device mean {dg.mean().item():.3e} max {dg.max().item():.3e} | "
         f"bf16 reference mean {dr.mean().item():.3e} max {dr.max().item():.3e}")
    assert dg.mean().item() <= 1.5 * dr.mean().item() + 2e-3 and dg.max().item() <= 2.0 * dr.max().item() + 2e-3
    kd = (m.kc[:, :plen].float().cpu() - kc32[:, :plen]).abs().max().item()
    kr = (kc[:, :plen].float() - kc32[:, :plen]).abs().max().item()
    _say(f"  prompt K rows: device {kd:.3e}, bf16 reference {kr:.3e} from the fp32 model")
    assert kd <= 2.0 * kr + 2e-3
    tok = int(m.tok.item())
    assert tok == int(torch.argmax(got).item()) and m.tokens[0].item() == tok
    assert m.pos.item() == plen and m.step.item() == 1 and torch.equal(m.x.view(-1), w.embed[tok])
    for i in range(3):  # decode after the prompt, teacher-forced with the device's tokens
        pos = plen + i
        m.graph(m.bucket_for(pos)).replay()
        torch.cuda.synchronize()
        got = m.logits.view(-1).float().cpu()
        want = ref.decode_model_step(bf, tok, pos, kc, vc, m.bucket_for(pos), shape.nh, shape.nkv).float()
        exact = ref.decode_model_step(f32, tok, pos, kc32, vc32, m.bucket_for(pos), shape.nh, shape.nkv)
        dg, dr = (got - exact).abs(), (want - exact).abs()
        _say(f"  decode pos {pos}: device mean {dg.mean().item():.3e} | bf16 reference mean {dr.mean().item():.3e}")
        assert dg.mean().item() <= 1.5 * dr.mean().item() + 2e-3 and dg.max().item() <= 2.0 * dr.max().item() + 2e-3
        tok = int(m.tok.item())
        assert m.tokens[i + 1].item() == tok


def test_generate_from_prompt_is_prefill_then_decode_replays(gpu):
    """generate_from_prompt = prefill + n-1 decode replays, with either step tail (identical tokens),
    and a second prompt on the same runner (captured graphs reused) repeats the first result."""
    w = RandomQwen3(TINY_UNTIED, gpu, seed=85)
    ids = list(range(3, 60, 2))
    a = GraphQwen3Decode(w, 256).generate_from_prompt(ids, 10)
    m = GraphQwen3Decode(w, 256, fused_tail=False)
    b = m.generate_from_prompt(ids, 10)
    c = m.generate_from_prompt(ids, 10)
    _say(f"  tokens {a}")
    assert a == b == c and len(set(a)) > 1


def test_argmax_failure_raises_at_the_sync(gpu):
    """A failed argmax reduction never passes silently: with the separate-ops tail and the argmax in
    its host-forced failure mode (solort_argmax_mode(2)) the greedy decode raises at its one
    synchronisation, and every token it recorded lies in the vocabulary; the fused tail, which does
    not use that reduction, decodes as before."""
    from solort_amd import ops
    p0, n = 60, 4
    w, fused = _model(gpu, p0, TINY_UNTIED)
    sep = GraphQwen3Decode(w, 256, fused_tail=False)
    sep.kc.copy_(fused.kc)
    sep.vc.copy_(fused.vc)
    want = fused.generate(7, p0, n)
    try:
        assert ops.argmax_mode(2) == 2
        with pytest.raises(RuntimeError, match="argmax reduction failed"):
            sep.generate(7, p0, n)
        assert all(0 <= t < TINY_UNTIED.vocab for t in sep.tokens[:n].tolist())
        fused.kc.copy_(sep.kc)
        fused.vc.copy_(sep.vc)
        assert fused.generate(7, p0, n) == want
    finally:
        ops.argmax_mode(1)


@pytest.mark.parametrize("p0,max_len,bounds", [(90, 256, [128]), (2040, 4096, [2048, 2560])],
                         ids=["bucket-128", "bounds-2048-2560"])
def test_verify_graph_matches_reference_ops(gpu, p0, max_len, bounds):
    """The whole-model verify graph (cuda_graph_executor.py:245-268 with the argmax and acceptance of
    :475-481): its logits against the CPU evaluations in bf16 and fp32 (the decode steps' bar), its
    argmax tokens the argmax of its logits, and acc_ver the first-mismatch rule applied on the host.
    From 2040 the three rounds end at 2044, 2049 and 2054: verify bounds 2048 (bucket 2048) and
    2560 (bucket 4096 cut at a multiple of 512)."""
    shape = TINY_UNTIED
    _say(f"[verify graph at {p0}, max_len {max_len}]")
    w, m = _model(gpu, p0, shape, max_len=max_len)
    bf = {k: (v.cpu() if torch.is_tensor(v) else [t.cpu() for t in v]) for k, v in vars(w).items() if k != "shape"}
    f32 = {k: (v.float() if torch.is_tensor(v) else [t.float() for t in v]) for k, v in bf.items()}
    kc, vc = m.kc.cpu(), m.vc.cpu()
    kc32, vc32 = kc.float(), vc.float()
    g = torch.Generator().manual_seed(87)
    for rnd in range(3):
        toks = torch.randint(0, shape.vocab, (m.k1,), generator=g).tolist()
        pos0 = p0 + rnd * m.k1
        m.vtok.copy_(torch.tensor(toks, device=gpu))
        logits = m.verify(pos0).float().cpu()
        torch.cuda.synchronize()
        want = ref.verify_model(bf, toks, pos0, kc, vc, shape.nh, shape.nkv).float()
        exact = ref.verify_model(f32, toks, pos0, kc32, vc32, shape.nh, shape.nkv)
        dg, dr = (logits - exact).abs(), (want - exact).abs()
        _say(f"  verify at {pos0}: device mean {dg.mean().item():.3e} max {dg.max().item():.3e} | "
             f"bf16 reference mean {dr.mean().item():.3e} max {dr.max().item():.3e}")
        assert dg.mean().item() <= 1.5 * dr.mean().item() + 2e-3 and dg.max().item() <= 2.0 * dr.max().item() + 2e-3
        tg = m.tok_ver.tolist()
        assert tg == logits.argmax(-1).tolist()
        a, nxt = ref.accept_prefix(torch.tensor(tg), torch.tensor(toks[1:]))
        assert m.acc_ver.tolist() == [a, nxt]
    kd = (m.kc[:, : p0 + 3 * m.k1].float().cpu() - kc32[:, : p0 + 3 * m.k1]).abs().max().item()
    kr = (kc[:, : p0 + 3 * m.k1].float() - kc32[:, : p0 + 3 * m.k1]).abs().max().item()
    assert kd <= 2.0 * kr + 2e-3
    assert sorted(m._ver_graphs) == bounds


@pytest.mark.parametrize("draft_seed", [None, 99], ids=["draft-same-weights", "draft-other-weights"])
def test_speculative_generation(gpu, draft_seed):
    """Greedy speculative rounds (cuda_graph_executor.py:463-482) after a prompt prefill: every
    emitted token is the fp32 model's argmax at its position (teacher-forced on the CPU with the
    emitted tokens) wherever that argmax leads the runner-up by more than 0.05, the target cache
    rows hold the emitted sequence's K rows, and a draft with the target's weights has most of its
    drafts accepted while a draft with other weights has almost none."""
    shape = TINY_UNTIED
    w = RandomQwen3(shape, gpu, seed=86)
    target = GraphQwen3Decode(w, 256)
    draft = GraphQwen3Decode(w if draft_seed is None else RandomQwen3(shape, gpu, seed=draft_seed), 256)
    ids = torch.randint(0, shape.vocab, (20,), generator=torch.Generator().manual_seed(88)).tolist()
    n = 24
    toks, accepted = target.generate_speculative(draft, ids, n)
    _say(f"  tokens {toks}\n  accepted per round {accepted}")
    bf = {k: (v.cpu() if torch.is_tensor(v) else [t.cpu() for t in v]) for k, v in vars(w).items() if k != "shape"}
    f32 = {k: (v.float() if torch.is_tensor(v) else [t.float() for t in v]) for k, v in bf.items()}
    kc32 = torch.zeros(shape.layers, 256, shape.nkv, 128)
    vc32 = torch.zeros_like(kc32)
    lg = ref.prefill_model(f32, ids, kc32, vc32, shape.nh, shape.nkv)
    checked = 0
    for i in range(n):
        top2 = torch.topk(lg, 2).values
        if (top2[0] - top2[1]).item() > 0.05:
            assert toks[i] == int(lg.argmax().item()), i
            checked += 1
        if i + 1 < n:
            lg = ref.decode_model_step(f32, toks[i], len(ids) + i, kc32, vc32, target.bucket_for(len(ids) + i),
                                       shape.nh, shape.nkv)
    P = len(ids) + n - 1
    kd = (target.kc[:, :P].float().cpu() - kc32[:, :P]).abs().max().item()
    _say(f"  {checked} of {n} tokens checked against the fp32 argmax; cache K rows to fp32 {kd:.3e}")
    assert checked >= n // 2 and kd <= 6e-2
    k = target.k1 - 1
    if draft_seed is None:
        assert sum(accepted) >= 0.6 * k * len(accepted)
    else:
        assert sum(accepted) <= 0.2 * k * len(accepted)


# the Qwen3-0.6B shape as a draft for a target at the Qwen3-4B widths: different hidden size, heads,
# layer count and query group, the same 151,936-token vocabulary (untied: the lm_head is its own matrix)
DRAFT_0_6B = ModelShape("qwen3-0.6b-draft", hidden=1024, inter=3072, nh=16, nkv=8, layers=28, vocab=151936,
                        tie_embeddings=False)
TARGET_4B_2L = ModelShape("qwen3-4b-widths-2l", hidden=2560, inter=9728, nh=32, nkv=8, layers=2, vocab=151936,
                          tie_embeddings=False)


def test_speculative_cross_shape_draft(gpu):
    """A 0.6B-shape draft (28 layers, hidden 1024, 16/8 heads) proposing for a target at the Qwen3-4B
    widths (2 layers, hidden 2560, 32/8 heads), as cuda_graph_executor.py:408-424, :463-482 pair a
    0.6B draft with a 4B target.  Every round's accepted count and appended token equal the reference
    rule (:476-481) applied to that round's drafts and the target's verify argmaxes; the emitted tokens
    equal the target-only greedy run, except that they may part at a position whose fp32 top-2 margin
    is under 0.05 (there the verify and decode paths' roundings may legitimately pick different
    tokens), after which the two runs continue different sequences; the draft's
    cache holds the emitted sequence, as a fresh draft prefilled with it does.  With independent
    random weights the draft almost never agrees, so rounds reject; the accepting rounds are the next
    test's."""
    wt = RandomQwen3(TARGET_4B_2L, gpu, seed=91)
    wd = RandomQwen3(DRAFT_0_6B, gpu, seed=92)
    target = GraphQwen3Decode(wt, 256)
    draft = GraphQwen3Decode(wd, 256)
    ids = torch.randint(0, 151936, (20,), generator=torch.Generator().manual_seed(93)).tolist()
    n = 24
    plen, k = len(ids), target.k1 - 1
    target.prefill(ids)
    draft.prefill(ids)
    out = [int(target.tok.item())]
    rounds = []
    while len(out) < n:
        got = target.speculative_round(draft, out[-1], plen + len(out) - 1)
        drafts = target.vtok[1:].tolist()
        tg = target.tok_ver.tolist()
        a, nxt = target.acc_ver.tolist()
        assert [a, nxt] == list(ref.accept_prefix(torch.tensor(tg), torch.tensor(drafts)))
        assert got == drafts[:a] + [nxt]
        rounds.append(a)
        out += got
    out = out[:n]
    _say(f"  tokens {out}\n  accepted per round {rounds}")

    greedy = GraphQwen3Decode(wt, 256).generate_from_prompt(ids, n)
    same = next((i for i in range(n) if out[i] != greedy[i]), n)
    if same < n:  # a divergence is allowed only where the fp32 model's top-2 margin is thin
        bf = {kk: (v.cpu() if torch.is_tensor(v) else [t.cpu() for t in v]) for kk, v in vars(wt).items()
              if kk != "shape"}
        f32 = {kk: (v.float() if torch.is_tensor(v) else [t.float() for t in v]) for kk, v in bf.items()}
        kc32 = torch.zeros(TARGET_4B_2L.layers, 256, TARGET_4B_2L.nkv, 128)
        vc32 = torch.zeros_like(kc32)
        lg = ref.prefill_model(f32, ids, kc32, vc32, TARGET_4B_2L.nh, TARGET_4B_2L.nkv)
        for i in range(same):
            lg = ref.decode_model_step(f32, greedy[i], plen + i, kc32, vc32, target.bucket_for(plen + i),
                                       TARGET_4B_2L.nh, TARGET_4B_2L.nkv)
        top2 = torch.topk(lg, 2).values
        margin = (top2[0] - top2[1]).item()
        _say(f"  first divergence from the target-only greedy run at token {same}, fp32 margin {margin:.3e}")
        assert margin < 0.05
    _say(f"  target-only greedy {greedy}; equal for the first {same} tokens")

    fresh = GraphQwen3Decode(wd, 256)
    fresh.prefill(ids + out[:n - 1])
    P = plen + n - 1
    d = (draft.kc[:, :P].float() - fresh.kc[:, :P].float()).abs()
    _say(f"  draft cache vs a fresh draft prefilled with the emitted tokens: max-abs {d.max().item():.3e} "
         f"mean-abs {d.mean().item():.3e}")
    # 28 layers of bf16 rounding in two accumulation orders (decode GEMVs against prefill GEMMs) leave
    # a few ulps; a row of another token would differ by ~1 on average
    assert d.mean().item() <= 1e-2 and d.max().item() <= 0.25
    assert sum(rounds) <= 0.2 * k * len(rounds)


def _bigram(w: RandomQwen3, skip_every: int = 0) -> None:
    """Turns random weights into a bigram model with a known greedy rule: o_proj and down are zero, so
    the residual stream stays embed[t] and the logits are lm_head @ rmsnorm(embed[t]); lm_head row v
    is embed row v - 1, so the self term (|embed[t]|^2 / rms, about 0.05 * hidden) leads every other
    logit by dozens of its spread and the next token is t + 1.  With skip_every = m, row v also gets
    1.5 x embed row v - 2 when (v - 2) % m == 0: then a token t with t % m == 0 is followed by t + 2."""
    for t in w.wo + w.wd:
        t.zero_()
    e = w.embed.float()
    lm = e.roll(1, dims=0)
    if skip_every:
        v = torch.arange(e.shape[0], device=e.device)
        lm += 1.5 * ((v - 2) % skip_every == 0).float()[:, None] * e.roll(2, dims=0)
    w.lm_head = lm.to(torch.bfloat16)


def test_speculative_cross_shape_partial_acceptance(gpu):
    """The same cross-shape pair as bigram models with known greedy rules: the target always emits
    t + 1, the 0.6B-shape draft emits t + 2 after a multiple of 7 and t + 1 otherwise.  Then every
    round's drafts, accepted count and appended token follow exactly from the reference's acceptance
    rule (cuda_graph_executor.py:463-482), rounds accept 0 to all 4 drafts, and the emitted tokens are
    the target's own greedy sequence."""
    wt = RandomQwen3(TARGET_4B_2L, gpu, seed=94)
    wd = RandomQwen3(DRAFT_0_6B, gpu, seed=95)
    _bigram(wt)
    _bigram(wd, skip_every=7)
    target = GraphQwen3Decode(wt, 256)
    draft = GraphQwen3Decode(wd, 256)
    ids = [1000 + 7 * i for i in range(20)]
    n = 40
    plen, k = len(ids), target.k1 - 1
    target.prefill(ids)
    draft.prefill(ids)
    out = [int(target.tok.item())]
    assert out[0] == ids[-1] + 1
    rounds = []
    f = lambda u: u + 2 if u % 7 == 0 else u + 1  # noqa: E731  (the draft's rule)
    while len(out) < n:
        last = out[-1]
        got = target.speculative_round(draft, last, plen + len(out) - 1)
        drafts = [f(last)]
        for _ in range(k - 1):
            drafts.append(f(drafts[-1]))
        tg = [last + 1] + [d + 1 for d in drafts]
        a = next((j for j in range(k) if drafts[j] != tg[j]), k)
        assert target.vtok[1:].tolist() == drafts
        assert target.tok_ver.tolist() == tg
        assert target.acc_ver.tolist() == [a, tg[a]]
        assert got == drafts[:a] + [tg[a]]
        rounds.append(a)
        out += got
    _say(f"  accepted per round {rounds}")
    assert out == list(range(ids[-1] + 1, ids[-1] + 1 + len(out)))
    # the first token after the prompt (1134) is a multiple of 7 (nothing accepted); after that the
    # rounds alternate between all k drafts and one
    assert 0 in rounds and k in rounds and any(0 < a < k for a in rounds)
