"""Greedy decode of a whole Qwen3-shaped model on one MI355X: the attention block of this package and
the decode-step GEMVs around it, one hipGraph replay per token.

Follows src/solort/model/cuda_graph_executor.py: the layer loop of _decode_forward (:163-190) with
the fused QKV and gate/up weights of :54-63, the embedding row (:165), final norm and lm_head
(:189-190), greedy argmax (:206) and the bucket routing (:192-193).  There is no checkpoint offline,
so the weights are seeded random tensors of the real shapes; every launch and byte moved is what
the real model would cost.

Per token (graph of one bucket): cos/sin rows -> per layer
  solort_gemv (RMSNorm + QKV) -> solort_decode_layer (q/k norm + RoPE + KV write + split-KV
  attention) -> solort_gemv (o_proj + residual) -> solort_gemv (RMSNorm + gate_up + SwiGLU) ->
  solort_gemv (down + residual)
-> solort_gemv_argmax (final RMSNorm + lm_head, each workgroup keeping the argmax key of its
logits) -> solort_greedy_advance (the token becomes the next input and is recorded, position and
count advance, and the token's embedding row becomes the next step's x).  K replays give K tokens
with one host synchronisation, as the reference's chunked greedy decode does (:362-374).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import ops
from .runner import (DECODE_BUCKETS, FUSED_PREFILL_MIN, HD, PREFILL_BUCKETS, decode_qkv_splits, decode_splits,
                     verify_bound, verify_splits)


@dataclass(frozen=True)
class ModelShape:
    name: str
    hidden: int
    inter: int
    nh: int
    nkv: int
    layers: int
    vocab: int
    tie_embeddings: bool

    @property
    def qkv_width(self) -> int:
        return (self.nh + 2 * self.nkv) * HD


QWEN3_0_6B = ModelShape("Qwen3-0.6B", 1024, 3072, 16, 8, 28, 151936, True)
QWEN3_4B = ModelShape("Qwen3-4B", 2560, 9728, 32, 8, 36, 151936, True)
QWEN3_8B = ModelShape("Qwen3-8B", 4096, 12288, 32, 8, 36, 151936, False)


class RandomQwen3:
    """Seeded random weights of a Qwen3 shape on the device (bf16): matrices N(0, 0.02), the
    embedding N(0, 0.05), norm weights N(1, 0.1)."""

    def __init__(self, shape: ModelShape, device: torch.device | str = "cuda", seed: int = 1007) -> None:
        self.shape = s = shape
        dev = torch.device(device)
        g = torch.Generator(device=dev).manual_seed(seed)

        def rnd(*dims, std=0.02, mean=0.0):
            return (torch.randn(*dims, generator=g, device=dev) * std + mean).to(torch.bfloat16)

        L, H, I = s.layers, s.hidden, s.inter
        self.embed = rnd(s.vocab, H, std=0.05)
        self.in_ln = rnd(L, H, std=0.1, mean=1.0)
        self.post_ln = rnd(L, H, std=0.1, mean=1.0)
        self.qn = rnd(L, HD, std=0.1, mean=1.0)
        self.kn = rnd(L, HD, std=0.1, mean=1.0)
        self.wqkv = [rnd(s.qkv_width, H) for _ in range(L)]   # cat(q_proj, k_proj, v_proj) (:57)
        self.wo = [rnd(H, s.nh * HD) for _ in range(L)]
        self.wgu = [rnd(2 * I, H) for _ in range(L)]          # cat(gate_proj, up_proj) (:58)
        self.wd = [rnd(H, I) for _ in range(L)]
        self.final_norm = rnd(H, std=0.1, mean=1.0)
        self.lm_head = self.embed if s.tie_embeddings else rnd(s.vocab, H)


def _rmsnorm_rows(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """cuda_graph_executor.py:25-28 over the rows of a prompt, as the reference's torch ops on the
    device: fp32 upcast, x * rsqrt(mean(x^2) + eps), times w in fp32, cast back."""
    xf = x.float()
    return ((xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps)) * w.float()).to(x.dtype)


class GraphQwen3Decode:
    """Greedy decode over a runner-owned bf16 KV cache, one captured graph per KV bucket."""

    def __init__(self, weights: RandomQwen3, max_len: int, eps: float = 1e-6, theta: float = 1e6,
                 max_tokens: int = 4096, fused_tail: bool = True, spec_k: int = 4, fused_qkv: bool = True) -> None:
        """fused_tail: the argmax folded into the lm_head launch and the token bookkeeping plus the
        next embedding row in one launch (solort_gemv_argmax + solort_greedy_advance); False runs
        the same step as the reference's separate ops (lm_head, argmax, token copy, counter adds,
        embedding gather).  fused_qkv: each layer's qkv product and attention block through
        solort_decode_qkv_layer (one launch where its shapes allow); False runs solort_gemv and
        solort_decode_layer.  All combinations give the same tokens bit for bit.  spec_k: draft
        tokens per speculative round (the verify graph scores spec_k + 1 tokens)."""
        self.w = weights
        self.fused_tail = bool(fused_tail)
        self.fused_qkv = bool(fused_qkv)
        # Measurement hook (bench.py): a decode graph captured with this False leaves the attention
        # call out of every layer, so the difference in step time is the attention's cost inside
        # the step.  Its tokens are not the model's.
        self.attention_in_step = True
        s = self.s = weights.shape
        self.dev = weights.embed.device
        self.max_len, self.eps, self.scale = int(max_len), float(eps), HD ** -0.5
        kv = (s.layers, self.max_len, s.nkv, HD)
        self.kc = torch.zeros(kv, dtype=torch.bfloat16, device=self.dev)
        self.vc = torch.zeros(kv, dtype=torch.bfloat16, device=self.dev)
        self.buckets = sorted({b for b in DECODE_BUCKETS if b < self.max_len} | {self.max_len})
        self.inv_freq = ops.inv_freq(HD, theta, self.dev)
        bf = dict(dtype=torch.bfloat16, device=self.dev)
        self.tok = torch.zeros(1, dtype=torch.long, device=self.dev)   # input token, then the argmax
        self.pos = torch.zeros(1, dtype=torch.long, device=self.dev)
        self.step = torch.zeros(1, dtype=torch.long, device=self.dev)  # tokens recorded so far
        self.tokens = torch.zeros(max_tokens, dtype=torch.long, device=self.dev)
        self.x = torch.zeros(1, s.hidden, **bf)                          # the residual stream
        self.qkv = torch.zeros(1, s.qkv_width, **bf)
        self.ctx = torch.zeros(1, s.nh * HD, **bf)
        self.act = torch.zeros(s.inter, **bf)
        self.logits = torch.zeros(1, s.vocab, **bf)
        self.cs = torch.zeros(2, 1, HD // 2, **bf)
        self.ws = ops.decode_qkv_workspace(
            s.nh, s.nkv, max(max(decode_splits(b, s.nkv), decode_qkv_splits(b, s.nkv)) for b in self.buckets), self.dev)
        self.ws_arg = ops.gemv_argmax_workspace(s.vocab, self.dev) if fused_tail else ops.argmax_workspace(1, self.dev)
        self._graphs: dict[int, torch.cuda.CUDAGraph] = {}
        # prefill (cuda_graph_executor.py:83-85, :104-161): one graph per prompt bucket over the padded
        # token buffer; the graph returns the last layer's hidden rows
        self.pre_buckets = sorted(b for b in PREFILL_BUCKETS if b <= self.max_len)
        pmax = max(self.pre_buckets)
        self.pre_tok = torch.zeros(pmax, dtype=torch.long, device=self.dev)
        self.cs_pre = torch.zeros(2 * pmax * (HD // 2), **bf)
        self.q_pre = torch.zeros(min(pmax, FUSED_PREFILL_MIN), s.nh, HD, **bf)
        self.ctx_pre = torch.zeros(pmax, s.nh * HD, **bf)
        self.zero_pos = torch.zeros(1, dtype=torch.long, device=self.dev)
        self._pre_graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self._pre_hidden: dict[int, torch.Tensor] = {}
        # speculative verify (cuda_graph_executor.py:245-289, :463-482): spec_k + 1 tokens per
        # graph, bucketed by key range like decode; acceptance on the device
        self.k1 = int(spec_k) + 1
        self.vtok = torch.zeros(self.k1, dtype=torch.long, device=self.dev)  # the input token, then the drafts
        self.vpos0 = torch.zeros(1, dtype=torch.long, device=self.dev)
        self.cs_ver = torch.zeros(2, self.k1, HD // 2, **bf)
        self.ctx_ver = torch.zeros(self.k1, s.nh * HD, **bf)
        self.tok_ver = torch.zeros(self.k1, dtype=torch.long, device=self.dev)
        self.acc_ver = torch.zeros(2, dtype=torch.long, device=self.dev)
        self.ws_ver = ops.attn_workspace(self.k1, s.nh, s.nkv, max(verify_splits(b, s.nkv) for b in self.buckets), self.dev)
        self.ws_argv = ops.argmax_workspace(self.k1, self.dev)
        self._ver_graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self._ver_logits: dict[int, torch.Tensor] = {}

    def start(self, token: int, pos: int) -> None:
        """The first input: token at position pos (rows 0..pos-1 of the cache hold the context)."""
        self.tok.fill_(int(token))
        self.pos.fill_(int(pos))
        self.step.zero_()
        torch.index_select(self.w.embed, 0, self.tok, out=self.x)     # :165 for the first step

    def _step(self, bound: int) -> None:
        """One token: cuda_graph_executor.py:163-190 from the x the previous step (or start) left,
        then argmax (:206), the token bookkeeping of :241-242 and :372, and the next step's :165."""
        s, w = self.s, self.w
        ns = decode_splits(bound, s.nkv)
        nsq = decode_qkv_splits(bound, s.nkv)
        if not self.fused_tail:
            torch.index_select(w.embed, 0, self.tok, out=self.x)                                       # :165
        ops.rope_rows(self.inv_freq, self.pos, 1, self.cs)             # :164, once per step
        x = self.x.view(s.hidden)
        for li in range(s.layers):
            if self.fused_qkv and self.attention_in_step:                                             # :170-184
                ops.decode_qkv_layer(x, w.in_ln[li], self.eps, w.wqkv[li], w.qn[li], w.kn[li], self.eps, self.cs,
                                     self.pos, self.kc[li], self.vc[li], bound, self.scale, self.ws, nsq,
                                     self.qkv.view(-1), self.ctx, s.nh, s.nkv)
            else:
                ops.gemv(w.wqkv[li], x, self.qkv.view(-1), w.in_ln[li], self.eps)                      # :170-171
                if self.attention_in_step:
                    ops.decode_layer(self.qkv, w.qn[li], w.kn[li], self.eps, self.cs, self.pos, self.kc[li],
                                     self.vc[li], bound, self.scale, self.ws, ns, self.ctx, s.nh, s.nkv)  # :172-184
            ops.gemv(w.wo[li], self.ctx.view(-1), x, res=x, mode=ops.GEMV_RESID)                       # :185
            ops.gemv(w.wgu[li], x, self.act, w.post_ln[li], self.eps, mode=ops.GEMV_SWIGLU,
                     inter=s.inter)                                                                    # :186-187
            ops.gemv(w.wd[li], self.act, x, res=x, mode=ops.GEMV_RESID)                                # :188
        if self.fused_tail:
            ops.gemv_argmax(w.lm_head, x, None, self.ws_arg, w.final_norm, self.eps,
                            logits=self.logits.view(-1))                                               # :189-190, :206
            ops.greedy_advance(self.ws_arg, s.vocab, w.embed, x, self.tok, self.tokens, self.step, self.pos)
        else:
            ops.gemv(w.lm_head, x, self.logits.view(-1), w.final_norm, self.eps)                      # :189-190
            ops.argmax_rows(self.logits, self.tok, self.ws_arg)                                        # :206
            self.tokens.index_copy_(0, self.step, self.tok)                                            # :372
            self.step.add_(1)
            self.pos.add_(1)                                                                           # :242

    def bucket_for(self, pos: int) -> int:
        """cuda_graph_executor.py:192-193: the first bucket strictly above the position."""
        for b in self.buckets:
            if b > pos:
                return b
        raise RuntimeError(f"decode position {pos} exceeds max_len {self.max_len}")

    def graph(self, bound: int) -> torch.cuda.CUDAGraph:
        if bound not in self._graphs:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._step(bound)
            self._graphs[bound] = g
        return self._graphs[bound]

    def _prefill_forward(self, bound: int) -> torch.Tensor:
        """cuda_graph_executor.py:104-135 over pre_tok[:bound] at positions 0..bound-1: the T-row
        products as library GEMMs (hipBLASLt), the attention block (with the KV write of rows
        0..bound-1) as solort_prefill_layer, or for short buckets the prologue then
        solort_prefill_attn.  Returns the last layer's hidden rows [bound, hidden] (the final norm
        is applied to the one row the lm_head reads)."""
        s, w = self.s, self.w
        cs = self.cs_pre[: 2 * bound * (HD // 2)].view(2, bound, HD // 2)
        ops.rope_rows(self.inv_freq, self.zero_pos, bound, cs)                  # :111
        x = w.embed.index_select(0, self.pre_tok[:bound])                       # :112
        ctx = self.ctx_pre[:bound]
        for li in range(s.layers):
            qkv = F.linear(_rmsnorm_rows(x, w.in_ln[li], self.eps), w.wqkv[li])  # :114-115
            if bound >= FUSED_PREFILL_MIN:                                       # :116-130
                ops.prefill_layer(qkv, w.qn[li], w.kn[li], self.eps, cs, self.kc[li], self.vc[li], self.scale, ctx,
                                  s.nh, s.nkv)
            else:
                ops.qknorm_rope_kvwrite_cs(qkv, w.qn[li], w.kn[li], self.eps, cs, None, self.q_pre[:bound],
                                           self.kc[li], self.vc[li], s.nh, s.nkv)
                ops.prefill_attn(self.q_pre[:bound], self.kc[li], self.vc[li], self.scale, ctx)
            x = x + F.linear(ctx, w.wo[li])                                      # :131
            gate, up = F.linear(_rmsnorm_rows(x, w.post_ln[li], self.eps), w.wgu[li]).split(s.inter, dim=-1)
            x = x + F.linear(F.silu(gate) * up, w.wd[li])                        # :132-134
        return x

    def prefill(self, ids: torch.Tensor | list[int]) -> None:
        """Graphed bucketed prefill (cuda_graph_executor.py:149-161) of a prompt of plen tokens: pads
        it with token 0 to the first prompt bucket >= plen, replays that bucket's graph (cache rows
        0..bucket-1 written; decode never reads the padding rows), then runs the final norm + lm_head +
        greedy argmax on row plen-1 (the reference runs its lm_head eagerly for that one row, :161)
        and leaves the first generated token as the next decode input at position plen, recorded
        as tokens[0]."""
        ids = torch.as_tensor(ids, dtype=torch.long).view(-1)
        plen = int(ids.numel())
        bound = next((b for b in self.pre_buckets if b >= plen), None)
        if bound is None or plen < 1:
            raise RuntimeError(f"prompt length {plen} outside the prefill buckets {self.pre_buckets}")
        self.pre_tok[:plen].copy_(ids.to(self.dev))
        self.pre_tok[plen:bound].zero_()
        if bound not in self._pre_graphs:
            self._prefill_forward(bound)  # eager once: the GEMM library initialises outside the capture
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self._pre_hidden[bound] = self._prefill_forward(bound)
            self._pre_graphs[bound] = graph
        self._pre_graphs[bound].replay()
        s, w = self.s, self.w
        last = self._pre_hidden[bound][plen - 1]
        self.pos.fill_(plen - 1)
        self.step.zero_()
        if self.fused_tail:
            ops.gemv_argmax(w.lm_head, last, None, self.ws_arg, w.final_norm, self.eps, logits=self.logits.view(-1))
            ops.greedy_advance(self.ws_arg, s.vocab, w.embed, self.x.view(-1), self.tok, self.tokens, self.step,
                               self.pos)
        else:
            ops.gemv(w.lm_head, last, self.logits.view(-1), w.final_norm, self.eps)
            ops.argmax_rows(self.logits, self.tok, self.ws_arg)
            self.tokens.index_copy_(0, self.step, self.tok)
            self.step.add_(1)
            self.pos.add_(1)

    def generate_from_prompt(self, ids: torch.Tensor | list[int], n: int) -> list[int]:
        """Greedy continuation of a prompt: prefill, then n - 1 decode replays (one host
        synchronisation); returns the n generated tokens."""
        plen = len(ids)
        if n < 1 or n > self.tokens.numel() or plen + n > self.max_len:
            raise RuntimeError(f"cannot generate {n} tokens after a {plen}-token prompt (max_len {self.max_len})")
        self.prefill(ids)
        for i in range(n - 1):
            self.graph(self.bucket_for(plen + i)).replay()
        return self._read_tokens(n)

    def _verify_forward(self, bound: int) -> torch.Tensor:
        """cuda_graph_executor.py:245-268 for the k1 tokens in vtok at vpos0..vpos0+k1-1: library GEMMs
        on the k1 rows around solort_decode_layer (nq = k1: prologue, KV write, causal attention over
        the bucket), the logits [k1, V], their argmax (:475) and the accepted-prefix rule (:476-481)
        into acc_ver = [a, tg[a]]."""
        s, w = self.s, self.w
        ops.rope_rows(self.inv_freq, self.vpos0, self.k1, self.cs_ver)          # :248
        x = w.embed.index_select(0, self.vtok)                                  # :249
        for li in range(s.layers):
            qkv = F.linear(_rmsnorm_rows(x, w.in_ln[li], self.eps), w.wqkv[li])  # :252-253
            ops.decode_layer(qkv, w.qn[li], w.kn[li], self.eps, self.cs_ver, self.vpos0, self.kc[li], self.vc[li],
                             bound, self.scale, self.ws_ver, verify_splits(bound, s.nkv), self.ctx_ver, s.nh, s.nkv)
            x = x + F.linear(self.ctx_ver, w.wo[li])                            # :264
            gate, up = F.linear(_rmsnorm_rows(x, w.post_ln[li], self.eps), w.wgu[li]).split(s.inter, dim=-1)
            x = x + F.linear(F.silu(gate) * up, w.wd[li])                       # :265-267
        logits = F.linear(_rmsnorm_rows(x, w.final_norm, self.eps), w.lm_head)   # :268
        ops.argmax_rows(logits, self.tok_ver, self.ws_argv)
        if self.k1 > 1:
            ops.accept_prefix(self.tok_ver, self.vtok[1:], self.acc_ver)
        return logits

    def verify(self, pos0: int) -> torch.Tensor:
        """Replays the verify graph of the bound holding positions pos0..pos0+k1-1 (verify_bound)
        over the tokens already in vtok; tok_ver then holds the k1 argmax tokens and acc_ver
        [a, tg[a]].  Returns the logits [k1, V] (the graph's buffer)."""
        if not 0 <= pos0 <= self.max_len - self.k1:
            raise RuntimeError(f"verify positions {pos0}..{pos0 + self.k1 - 1} exceed max_len {self.max_len}")
        bound = verify_bound(pos0 + self.k1 - 1, self.buckets)
        self.vpos0.fill_(int(pos0))
        if bound not in self._ver_graphs:
            self._verify_forward(bound)  # eager once: the GEMM library initialises outside the capture
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self._ver_logits[bound] = self._verify_forward(bound)
            self._ver_graphs[bound] = graph
        self._ver_graphs[bound].replay()
        return self._ver_logits[bound]

    def speculative_round(self, draft: "GraphQwen3Decode", last_token: int, pos: int) -> list[int]:
        """One exact greedy speculative round, cuda_graph_executor.py:463-482: the draft model decodes
        k = k1 - 1 tokens from last_token at pos (its own graphs and cache), this model scores
        [last_token, drafts] at pos..pos+k in one verify replay, and the accepted drafts plus the
        token after them are returned (one host synchronisation).  With every draft accepted the
        draft also decodes its last draft at pos+k, so its cache stays whole (:479)."""
        k = self.k1 - 1
        if draft.k1 != self.k1 or draft.max_len < pos + k + 1:
            raise RuntimeError("draft model does not match the verify width or is too short")
        draft.start(last_token, pos)
        for i in range(k):
            draft.graph(draft.bucket_for(pos + i)).replay()
        self.vtok[0].fill_(int(last_token))
        self.vtok[1:].copy_(draft.tokens[:k])
        self.verify(pos)
        got = torch.cat([self.acc_ver, self.vtok[1:]]).tolist()  # the one synchronisation
        a, nxt, drafts = got[0], got[1], got[2:]
        ops.check_tokens([nxt] + drafts, self.s.vocab, "speculative round")
        if ops.argmax_failures(self.ws_argv, self.k1):
            raise RuntimeError("speculative round: an argmax reduction failed (see solort_argmax_rows)")
        if a == k:
            draft.start(drafts[k - 1], pos + k)
            draft.graph(draft.bucket_for(pos + k)).replay()
        return drafts[:a] + [nxt]

    def generate_speculative(self, draft: "GraphQwen3Decode", ids: list[int], n: int) -> tuple[list[int], list[int]]:
        """Greedy continuation of a prompt by speculative rounds: both models prefill the prompt,
        then rounds run until n tokens are out (the last round's extra tokens are dropped).
        Returns the tokens and the accepted-draft count of every round."""
        plen = len(ids)
        if plen + n + self.k1 > min(self.max_len, draft.max_len):
            raise RuntimeError(f"{plen} + {n} tokens and a round of {self.k1} exceed max_len")
        self.prefill(ids)
        draft.prefill(ids)
        out = ops.check_tokens([int(self.tok.item())], self.s.vocab, "prefill")
        accepted = []
        while len(out) < n:
            toks = self.speculative_round(draft, out[-1], plen + len(out) - 1)
            accepted.append(len(toks) - 1)
            out += toks
        return out[:n], accepted

    def generate(self, first_token: int, pos: int, n: int) -> list[int]:
        """Greedy tokens after `first_token` at position `pos` (rows 0..pos-1 of the cache hold the
        context): n graph replays, one synchronisation."""
        if n < 1 or n > self.tokens.numel() or pos + n > self.max_len:
            raise RuntimeError(f"cannot generate {n} tokens from position {pos} (max_len {self.max_len})")
        self.start(first_token, pos)
        for i in range(n):
            self.graph(self.bucket_for(pos + i)).replay()
        return self._read_tokens(n)

    def _read_tokens(self, n: int) -> list[int]:
        """The first n recorded tokens (one synchronisation), checked: every token in the vocabulary
        and, with the separate-ops tail, no argmax reduction failed."""
        toks = ops.check_tokens(self.tokens[:n].tolist(), self.s.vocab, "greedy decode")
        if not self.fused_tail and ops.argmax_failures(self.ws_arg, 1):
            raise RuntimeError("greedy decode: an argmax reduction failed (see solort_argmax_rows)")
        return toks
