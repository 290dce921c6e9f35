"""Seeded synthetic inputs for the benchmark and parity workloads (CPU tensors).

Everything is drawn on the CPU from ``torch.Generator().manual_seed(seed)`` in
fp32, in a fixed order (cache K, cache V, raw qkv, norm weights, logits), then
cast, so every machine sees identical bits.  Shapes are the Qwen3 attention
shapes (head_dim 128, RMSNorm eps 1e-6, RoPE theta 1e6); there are no model
weights beyond the two per-layer q/k norm vectors, drawn N(1, 0.1).

Workloads (seed = 1000 + index):
  0  Qwen3-0.6B decode: 16 q / 8 kv heads, 28 layers, cache max 1024 with rows
     0..511 filled, new token at position 512 (513 live keys, bucket 1024).
  1  Qwen3-4B decode sweep: 32 q / 8 kv heads, 36 layers, cache max 1024;
     live length L in {128, 256, 512, 1024}: rows 0..L-2 filled, new token at L-1.
  2  Qwen3-4B causal prefill: T in {128, 512, 1024} prompt rows into an empty
     cache of max 1024, positions 0..T-1.
  3  Qwen3-8B long decode: 32 q / 8 kv heads, cache max 32768, rows 0..32766
     filled, new token at 32767; per layer 1% of key rows (seeded randperm) x8.
  4  Qwen3-4B speculative verify: 5 queries at 2048..2052 over rows 0..2047,
     cache max 4096; then logits [5, 151936] ~ N(0, 3) in bf16 with 10 planted
     exact ties per row (one in the first 1K, one in the last 1K) at
     bf16(rowmax + 1).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

HD = 128
EPS = 1e-6
THETA = 1e6
VOCAB = 151936


@dataclass(frozen=True)
class AttnShape:
    name: str
    nh: int
    nkv: int
    layers: int

    @property
    def group(self) -> int:
        return self.nh // self.nkv

    @property
    def qkv_width(self) -> int:
        return (self.nh + 2 * self.nkv) * HD

    @property
    def scale(self) -> float:
        return HD ** -0.5


QWEN3_0_6B = AttnShape("Qwen3-0.6B", 16, 8, 28)
QWEN3_4B = AttnShape("Qwen3-4B", 32, 8, 36)
QWEN3_8B = AttnShape("Qwen3-8B", 32, 8, 36)

DECODE_LIVE = (128, 256, 512, 1024)
PREFILL_T = (128, 512, 1024)


@dataclass
class DecodeCase:
    shape: AttnShape
    max_len: int
    pos: int            # position of the first new token
    nq: int             # new tokens (1 decode, K+1 verify)
    bound: int          # static key bound (the bucket)
    kc: torch.Tensor    # [layers, max_len, nkv, hd]
    vc: torch.Tensor
    qkv: torch.Tensor   # [layers, nq, (nh+2nkv)*hd]
    qn_w: torch.Tensor  # [layers, hd]
    kn_w: torch.Tensor
    logits: torch.Tensor | None = None


def _norm_weights(g: torch.Generator, layers: int) -> tuple[torch.Tensor, torch.Tensor]:
    qn = 1.0 + 0.1 * torch.randn(layers, HD, generator=g)
    kn = 1.0 + 0.1 * torch.randn(layers, HD, generator=g)
    return qn, kn


def _cache(g: torch.Generator, layers: int, max_len: int, nkv: int, filled: int,
           heavy_frac: float = 0.0) -> tuple[torch.Tensor, torch.Tensor]:
    kc = torch.zeros(layers, max_len, nkv, HD)
    vc = torch.zeros(layers, max_len, nkv, HD)
    if filled > 0:
        kc[:, :filled] = torch.randn(layers, filled, nkv, HD, generator=g)
        if heavy_frac > 0:
            n_heavy = int(round(heavy_frac * max_len))
            for li in range(layers):
                rows = torch.randperm(max_len, generator=g)[:n_heavy]
                rows = rows[rows < filled]
                kc[li, rows] *= 8.0
        vc[:, :filled] = torch.randn(layers, filled, nkv, HD, generator=g)
    return kc, vc


def decode_case(index: int, live: int | None = None, layers: int | None = None,
                dtype: torch.dtype = torch.bfloat16) -> DecodeCase:
    """Workload 0, 1, 3 or 4 (attention part) as CPU tensors in `dtype`."""
    g = torch.Generator().manual_seed(1000 + index)
    if index == 0:
        shape, max_len, pos, nq, bound, heavy = QWEN3_0_6B, 1024, 512, 1, 1024, 0.0
    elif index == 1:
        live = 1024 if live is None else int(live)
        shape, max_len, pos, nq, bound, heavy = QWEN3_4B, 1024, live - 1, 1, live, 0.0
    elif index == 3:
        shape, max_len, pos, nq, bound, heavy = QWEN3_8B, 32768, 32767, 1, 32768, 0.01
    elif index == 4:
        shape, max_len, pos, nq, bound, heavy = QWEN3_4B, 4096, 2048, 5, 4096, 0.0
    else:
        raise ValueError(f"workload {index} is not a decode workload")
    L = shape.layers if layers is None else int(layers)
    kc, vc = _cache(g, L, max_len, shape.nkv, pos, heavy)
    qkv = torch.randn(L, nq, shape.qkv_width, generator=g)
    qn, kn = _norm_weights(g, L)
    logits = None
    if index == 4:
        logits = planted_logits(g, nq, VOCAB)
    cast = (lambda t: t.to(dtype))
    return DecodeCase(shape, max_len, pos, nq, bound, cast(kc), cast(vc), cast(qkv), cast(qn), cast(kn),
                      logits)


@dataclass
class PrefillCase:
    shape: AttnShape
    max_len: int
    T: int
    qkv: torch.Tensor   # [layers, T, (nh+2nkv)*hd]
    qn_w: torch.Tensor
    kn_w: torch.Tensor


def prefill_case(T: int, layers: int | None = None, dtype: torch.dtype = torch.bfloat16) -> PrefillCase:
    """Workload 2 at prompt length T (the cache starts empty, max 1024)."""
    g = torch.Generator().manual_seed(1002)
    shape = QWEN3_4B
    L = shape.layers if layers is None else int(layers)
    qkv = torch.randn(L, T, shape.qkv_width, generator=g)
    qn, kn = _norm_weights(g, L)
    return PrefillCase(shape, 1024, T, qkv.to(dtype), qn.to(dtype), kn.to(dtype))


def planted_logits(g: torch.Generator, rows: int, vocab: int, ties: int = 10) -> torch.Tensor:
    """bf16 logits ~ N(0, 3) with `ties` exact copies of bf16(rowmax + 1) per row.

    One planted index lies in the first 1024 and one in the last 1024, so the
    answer (the smallest planted index) exercises both ends of the row.
    """
    x = (3.0 * torch.randn(rows, vocab, generator=g)).to(torch.bfloat16)
    for r in range(rows):
        top = (x[r].float().max() + 1.0).to(torch.bfloat16)
        first = torch.randint(0, 1024, (1,), generator=g)
        last = torch.randint(vocab - 1024, vocab, (1,), generator=g)
        mid = torch.randint(1024, vocab - 1024, (ties - 2,), generator=g)
        x[r, torch.cat([first, last, mid])] = top
    return x
