"""numpy restatements that pin the torch oracle and the kernels.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

- bf16 helpers: round-to-nearest-even with NaN -> 0x7FC0, the rule torch's
  c10::BFloat16 conversion uses.
- prologue_fixed_order: the reference's QK-RMSNorm + RoPE
  (cuda_graph_executor.py:25-28, :100-102) with the one unspecified step, the
  order of the fp32 sum of squares, fixed to the order the gfx950 kernel uses
  (per 8-element lane chunk left to right, then an xor butterfly over the 16
  chunks at distances 1, 2, 4, 8).  Everything else is IEEE fp32 with a bf16
  rounding after each op the reference rounds.
- attention in fp64 by brute force, with the decode/verify causal rule of
  cuda_graph_executor.py:168 and :250.
- splitkv_combine: the split-KV partial + log-sum-exp merge the decode kernel
  performs, in fp64, to show that splitting does not change the result.
- prefill_blockwise: the prefill kernel's own arithmetic (online softmax over
  64-key blocks with the probabilities rounded to bf16 before the second
  matrix product) in fp64, to pin the kernel's fp32 output tightly.
- argmax_first: first index of the maximum, NaN counted as maximum
  (torch.argmax / numpy.argmax rule).
"""
from __future__ import annotations

import numpy as np

HD = 128


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round to nearest even, NaN -> 0x7FC0."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r[nan] = 0x7FC0
    return r


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 value of the bf16 nearest to x."""
    return bf16_to_f32(bf16_bits(x))


def sum_squares_fixed_order(x: np.ndarray) -> np.ndarray:
    """fp32 sum of squares over the last axis (128) in the kernel's order."""
    x = np.asarray(x, dtype=np.float32)
    sq = (x * x).reshape(*x.shape[:-1], 16, 8)  # bf16 squares are exact in fp32
    s = sq[..., 0].copy()
    for i in range(1, 8):
        s = s + sq[..., i]
    lanes = np.arange(16)
    for off in (1, 2, 4, 8):
        s = s + s[..., lanes ^ off]
    return s[..., 0]


def rmsnorm_fixed_order(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """cuda_graph_executor.py:25-28 over the last axis with the fixed sum order; returns bf16 values (fp32)."""
    x = np.asarray(x, dtype=np.float32)
    mean = sum_squares_fixed_order(x) * np.float32(1.0 / 128.0)
    r = np.float32(1.0) / np.sqrt(mean + np.float32(eps))
    return bf16_round((x * r[..., None]) * np.asarray(w, dtype=np.float32))


def rope_bf16(y: np.ndarray, cos_half: np.ndarray, sin_half: np.ndarray) -> np.ndarray:
    """cuda_graph_executor.py:100-102 on bf16 values: bf16(bf16(y*cos) + bf16(rot(y)*sin)).

    y [..., T, 128]; cos_half/sin_half [T, 64] (the duplicated half of the reference's row).
    """
    c = np.concatenate([cos_half, cos_half], axis=-1).astype(np.float32)
    s = np.concatenate([sin_half, sin_half], axis=-1).astype(np.float32)
    rot = np.concatenate([-y[..., 64:], y[..., :64]], axis=-1)
    return bf16_round(bf16_round(y * c) + bf16_round(rot * s))


def prologue_fixed_order(qkv: np.ndarray, qn_w: np.ndarray, kn_w: np.ndarray, eps: float,
                         cos_half: np.ndarray, sin_half: np.ndarray, nh: int, nkv: int):
    """qkv [T, (nh+2nkv)*128] bf16 values (fp32) -> q [T,nh,128], k [T,nkv,128], v [T,nkv,128].

    cos_half/sin_half: [T, 64] bf16 values for the T positions.
    """
    T = qkv.shape[0]
    x = np.asarray(qkv, dtype=np.float32).reshape(T, nh + 2 * nkv, HD)
    q = rmsnorm_fixed_order(x[:, :nh], qn_w, eps)
    k = rmsnorm_fixed_order(x[:, nh:nh + nkv], kn_w, eps)
    v = x[:, nh + nkv:].copy()
    cs, sn = cos_half[:, None, :], sin_half[:, None, :]
    return rope_bf16(q, cs, sn), rope_bf16(k, cs, sn), v


def attn_fp64(q: np.ndarray, keys: np.ndarray, vals: np.ndarray, scale: float) -> np.ndarray:
    """softmax(q K^T * scale) V in fp64; q [R,hd], keys/vals [L,hd]."""
    s = (np.asarray(q, np.float64) @ np.asarray(keys, np.float64).T) * scale
    s -= s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return p @ np.asarray(vals, np.float64)


def causal_attn_fp64(q: np.ndarray, keys: np.ndarray, vals: np.ndarray, scale: float) -> np.ndarray:
    """Top-left causal attention in fp64, one head: row t of q [T,hd] attends keys/vals 0..t
    (cuda_graph_executor.py:124-130, SDPA is_causal=True over positions 0..T-1).  Returns [T,hd]."""
    q = np.asarray(q, np.float64)
    T = q.shape[0]
    s = (q @ np.asarray(keys, np.float64)[:T].T) * scale
    s[np.triu_indices(T, 1)] = -np.inf
    s -= s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return p @ np.asarray(vals, np.float64)[:T]


def causal_decode_fp64(q: np.ndarray, kc_l: np.ndarray, vc_l: np.ndarray, pos0: int, scale: float) -> np.ndarray:
    """Query t (q [nq,nh,hd]) at position pos0+t attends cache rows 0..pos0+t of its KV head h // g.

    cuda_graph_executor.py:168 (decode, nq = 1) and :250 (verify).  Returns [nq, nh, hd] fp64.
    """
    nq, nh, hd = q.shape
    nkv = kc_l.shape[1]
    g = nh // nkv
    out = np.empty((nq, nh, hd), np.float64)
    for t in range(nq):
        n = pos0 + t + 1
        for h in range(nh):
            out[t, h] = attn_fp64(q[t, h][None], kc_l[:n, h // g], vc_l[:n, h // g], scale)[0]
    return out


def splitkv_combine(q: np.ndarray, keys: np.ndarray, vals: np.ndarray, scale: float, n_split: int) -> np.ndarray:
    """The decode kernel's split-KV scheme in fp64: per split (max, sum, unnormalised output) in
    log2 units, merged by exp2(m_s - M) weights.  q [R,hd]; returns [R,hd]."""
    q = np.asarray(q, np.float64)
    L = keys.shape[0]
    chunk = -(-L // n_split)
    chunk = -(-chunk // 16) * 16
    parts = []
    for s0 in range(0, n_split * chunk, chunk):
        k = keys[s0:min(s0 + chunk, L)]
        if k.shape[0] == 0:
            parts.append((np.full(q.shape[0], -np.inf), np.zeros(q.shape[0]), np.zeros_like(q)))
            continue
        z = (q @ np.asarray(k, np.float64).T) * scale * np.log2(np.e)
        m = z.max(axis=-1)
        p = np.exp2(z - m[:, None])
        parts.append((m, p.sum(axis=-1), p @ np.asarray(vals[s0:s0 + k.shape[0]], np.float64)))
    M = np.max([p[0] for p in parts], axis=0)
    w = [np.where(np.isneginf(p[0]), 0.0, np.exp2(p[0] - M)) for p in parts]
    Lsum = sum(wi * p[1] for wi, p in zip(w, parts))
    O = sum(wi[:, None] * p[2] for wi, p in zip(w, parts))
    return O / Lsum[:, None]


def prefill_blockwise(q: np.ndarray, keys: np.ndarray, vals: np.ndarray, scale: float, block: int = 64,
                      splits: int = 2, lazy: float = 8.0) -> np.ndarray:
    """Causal attention of q [T,hd] (row t at position t) over keys/vals [T,hd] as the prefill kernel
    evaluates it.  The 64-key blocks are dealt round-robin to `splits` independent passes (block b to
    pass b % splits).  Each pass keeps, per row, a reference max M (log2 units) that moves to the
    block's max only when that exceeds M by more than `lazy` (the first visible block always sets
    it); per block p = bf16(2^(s - M)), l = l * 2^(M_old - M) + sum(p_bf16),
    o = o * 2^(M_old - M) + p_bf16 @ V.  The passes are merged by log-sum-exp.  fp64 except the bf16
    rounding of p."""
    q = np.asarray(q, np.float64)
    T = q.shape[0]
    z = (q @ np.asarray(keys, np.float64).T) * scale * np.log2(np.e)
    z[np.triu_indices(T, 1)] = -np.inf
    vals = np.asarray(vals, np.float64)
    parts = []
    for sp in range(splits):
        m = np.full(T, -np.inf)
        l = np.zeros(T)
        o = np.zeros_like(q)
        for k0 in range(sp * block, T, splits * block):
            zb = z[:, k0:k0 + block]
            mx = zb.max(axis=1)
            with np.errstate(invalid="ignore"):  # -inf - -inf in rows with no visible key yet
                bump = mx > m + lazy
                mn = np.where(bump, mx, m)
                live = np.isfinite(mn)
                alpha = np.where(bump & np.isfinite(m), np.exp2(np.where(bump & np.isfinite(m), m - mn, 0.0)), 1.0)
                p = np.where(live[:, None], np.exp2(zb - np.where(live, mn, 0.0)[:, None]), 0.0)
            pb = np.asarray(bf16_round(p), np.float64)
            l = l * alpha + pb.sum(axis=1)
            o = o * alpha[:, None] + pb @ vals[k0:k0 + block]
            m = mn
        parts.append((m, l, o))
    mt = np.max(np.stack([m for m, _, _ in parts]), axis=0)  # finite: pass 0 holds key 0
    with np.errstate(invalid="ignore"):
        w = [np.where(np.isfinite(m), np.exp2(np.where(np.isfinite(m), m - mt, 0.0)), 0.0) for m, _, _ in parts]
    l = sum(wi * lp for wi, (_, lp, _) in zip(w, parts))
    o = sum(wi[:, None] * op for wi, (_, _, op) in zip(w, parts))
    return o / l[:, None]


def argmax_first(x: np.ndarray) -> np.ndarray:
    """Row-wise index of the first maximum, NaN ranked highest (numpy/torch rule)."""
    return np.argmax(np.asarray(x, dtype=np.float32), axis=-1).astype(np.int64)
