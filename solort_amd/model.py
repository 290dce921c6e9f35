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

from . import ops
from .runner import DECODE_BUCKETS, HD, decode_splits


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


class GraphQwen3Decode:
    """Greedy decode over a runner-owned bf16 KV cache, one captured graph per KV bucket."""

    def __init__(self, weights: RandomQwen3, max_len: int, eps: float = 1e-6, theta: float = 1e6,
                 max_tokens: int = 4096, fused_tail: bool = True) -> None:
        """fused_tail: the argmax folded into the lm_head launch and the token bookkeeping plus the
        next embedding row in one launch (solort_gemv_argmax + solort_greedy_advance); False runs
        the same step as the reference's separate ops (lm_head, argmax, token copy, counter adds,
        embedding gather).  Both give the same tokens bit for bit."""
        self.w = weights
        self.fused_tail = bool(fused_tail)
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
        self.ws = ops.attn_workspace(1, s.nh, s.nkv, max(decode_splits(b, s.nkv) for b in self.buckets), self.dev)
        self.ws_arg = ops.gemv_argmax_workspace(s.vocab, self.dev) if fused_tail else ops.argmax_workspace(1, self.dev)
        self._graphs: dict[int, torch.cuda.CUDAGraph] = {}

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
        if not self.fused_tail:
            torch.index_select(w.embed, 0, self.tok, out=self.x)                                       # :165
        ops.rope_rows(self.inv_freq, self.pos, 1, self.cs)             # :164, once per step
        x = self.x.view(s.hidden)
        for li in range(s.layers):
            ops.gemv(w.wqkv[li], x, self.qkv.view(-1), w.in_ln[li], self.eps)                          # :170-171
            ops.decode_layer(self.qkv, w.qn[li], w.kn[li], self.eps, self.cs, self.pos, self.kc[li],
                             self.vc[li], bound, self.scale, self.ws, ns, self.ctx, s.nh, s.nkv)       # :172-184
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

    def generate(self, first_token: int, pos: int, n: int) -> list[int]:
        """Greedy tokens after `first_token` at position `pos` (rows 0..pos-1 of the cache hold the
        context): n graph replays, one synchronisation."""
        if n < 1 or n > self.tokens.numel() or pos + n > self.max_len:
            raise RuntimeError(f"cannot generate {n} tokens from position {pos} (max_len {self.max_len})")
        self.start(first_token, pos)
        for i in range(n):
            self.graph(self.bucket_for(pos + i)).replay()
        return self.tokens[:n].tolist()
