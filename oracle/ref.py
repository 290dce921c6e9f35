"""Torch-on-CPU restatement of the reference runner's attention math.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Each function follows
src/solort/model/cuda_graph_executor.py at the cited lines, op for op and in
the same dtype, so that bf16 inputs give the reference's bf16 rounding of
scores, probabilities and outputs.  Inputs are plain torch CPU tensors.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """cuda_graph_executor.py:25-28: fp32 upcast, x * rsqrt(mean(x^2) + eps), times w in fp32, cast back."""
    xf = x.to(torch.float32)
    inv_rms = torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps)
    return ((xf * inv_rms) * w.to(torch.float32)).to(x.dtype)


def inv_freq(hd: int, theta: float) -> torch.Tensor:
    """cuda_graph_executor.py:64-66: 1 / theta^(2i/hd) in fp32."""
    exps = torch.arange(0, hd, 2).to(torch.float32) / hd
    return 1.0 / (float(theta) ** exps)


def cos_sin(positions: torch.Tensor, inv_f: torch.Tensor, dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """cuda_graph_executor.py:95-98: angles pos * inv_freq in fp32, duplicated halves, cast to dtype."""
    ang = positions.reshape(-1, 1).to(torch.float32) * inv_f.reshape(1, -1)
    full = torch.cat((ang, ang), dim=-1)
    return full.cos().to(dtype), full.sin().to(dtype)


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """cuda_graph_executor.py:100-102: x*cos + rotate_half(x)*sin, each op in x's dtype."""
    half = x.shape[-1] // 2
    rotated = torch.cat((x[..., half:].neg(), x[..., :half]), dim=-1)
    return x * cos + rotated * sin


def prologue(qkv: torch.Tensor, qn_w: torch.Tensor, kn_w: torch.Tensor, eps: float,
             cos: torch.Tensor, sin: torch.Tensor, nh: int, nkv: int, hd: int = 128):
    """cuda_graph_executor.py:116-121 (and :172-177, :253-258).

    qkv [T, (nh+2nkv)*hd] -> q [nh,T,hd], k [nkv,T,hd] (normed + roped), v [nkv,T,hd] (raw).
    cos/sin are [T, hd] rows for the T positions.
    """
    T = qkv.shape[0]
    q, k, v = torch.split(qkv, [nh * hd, nkv * hd, nkv * hd], dim=-1)
    q = q.reshape(T, nh, hd).transpose(0, 1)
    k = k.reshape(T, nkv, hd).transpose(0, 1)
    v = v.reshape(T, nkv, hd).transpose(0, 1)
    q = rope(rmsnorm(q, qn_w, eps), cos, sin)
    k = rope(rmsnorm(k, kn_w, eps), cos, sin)
    return q, k, v


def write_kv(kc_l: torch.Tensor, vc_l: torch.Tensor, k: torch.Tensor, v: torch.Tensor, pos0: int) -> None:
    """cuda_graph_executor.py:122-123, :178-179, :259-260: rows pos0..pos0+T-1 of one layer's cache."""
    T = k.shape[1]
    idx = torch.arange(pos0, pos0 + T)
    kc_l.index_copy_(0, idx, k.transpose(0, 1))
    vc_l.index_copy_(0, idx, v.transpose(0, 1))


def decode_attn(q: torch.Tensor, kc_l: torch.Tensor, vc_l: torch.Tensor, pos: int, bound: int,
                scale: float) -> torch.Tensor:
    """cuda_graph_executor.py:168, :180-184: grouped single-token attention over the bucket.

    q [nh,1,hd]; kc_l/vc_l [max_len,nkv,hd]; keys with index > pos are masked.
    Returns ctx [1, nh*hd] in q's dtype.
    """
    nh, hd = q.shape[0], q.shape[-1]
    nkv = kc_l.shape[1]
    qg = q.reshape(nkv, nh // nkv, hd)
    keys_t = kc_l[:bound].permute(1, 2, 0)
    vals = vc_l[:bound].permute(1, 0, 2)
    ignore = (torch.arange(bound) > pos).view(1, 1, bound)
    scores = (torch.matmul(qg, keys_t) * scale).masked_fill(ignore, float("-inf"))
    probs = torch.softmax(scores, dim=-1).to(q.dtype)
    return torch.matmul(probs, vals).reshape(1, nh * hd)


def prefill_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    """cuda_graph_executor.py:124-130: causal SDPA with K/V repeated over the query group.

    q [nh,T,hd], k/v [nkv,T,hd] -> ctx [T, nh*hd].
    """
    nh, T, hd = q.shape
    g = nh // k.shape[0]
    kk = k.repeat_interleave(g, dim=0)
    vv = v.repeat_interleave(g, dim=0)
    out = F.scaled_dot_product_attention(q, kk, vv, is_causal=True, scale=scale)
    return out.transpose(0, 1).reshape(T, nh * hd)


def verify_attn(q: torch.Tensor, kc_l: torch.Tensor, vc_l: torch.Tensor, pos0: int,
                scale: float) -> torch.Tensor:
    """cuda_graph_executor.py:247-250, :261-263: K+1 queries over all max_len keys, key <= pos kept.

    q [nh,K1,hd] -> ctx [K1, nh*hd].
    """
    nh, k1, hd = q.shape
    max_len, nkv = kc_l.shape[0], kc_l.shape[1]
    g = nh // nkv
    pos = pos0 + torch.arange(k1)
    keep = (torch.arange(max_len).view(1, -1) <= pos.view(-1, 1)).view(1, k1, max_len)
    kk = kc_l.permute(1, 0, 2).repeat_interleave(g, dim=0)
    vv = vc_l.permute(1, 0, 2).repeat_interleave(g, dim=0)
    ctx = F.scaled_dot_product_attention(q, kk, vv, attn_mask=keep, scale=scale)
    return ctx.transpose(0, 1).reshape(k1, nh * hd)


def linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """x @ w.T in x's dtype with fp32 accumulation (the bf16 GEMMs of :171, :185, :187, :188, :190),
    evaluated on the CPU in fp32 and rounded once."""
    return (x.float() @ w.float().T).to(x.dtype)


def decode_mlp_block(x: torch.Tensor, ctx: torch.Tensor, wo: torch.Tensor, post_ln: torch.Tensor, wgu: torch.Tensor,
                     wd: torch.Tensor, eps: float) -> torch.Tensor:
    """The non-attention tail of one decode layer, cuda_graph_executor.py:185-188, bf16:
    x = x + ctx @ wo.T; h2 = rmsnorm(x); gate, up = split(h2 @ wgu.T); x = x + (silu(gate) * up) @ wd.T."""
    x = x + linear(ctx, wo)
    h2 = rmsnorm(x, post_ln, eps)
    gate, up = linear(h2, wgu).split(wgu.shape[0] // 2, dim=-1)
    return x + linear(F.silu(gate) * up, wd)


def accept_prefix(tg: torch.Tensor, draft: torch.Tensor) -> tuple[int, int]:
    """cuda_graph_executor.py:476: a = (tg[:k] == draft).cumprod(0).sum(); with the token the round
    appends after the accepted drafts, tg[a] (:478, :481).  tg [k+1], draft [k] int64."""
    k = draft.numel()
    a = int((tg[:k] == draft).cumprod(0).sum().item())
    return a, int(tg[a].item())


def argmax(logits: torch.Tensor) -> torch.Tensor:
    """cuda_graph_executor.py:190, :206 (and :234, :475): argmax(-1) of fp32 logits."""
    return logits.to(torch.float32).argmax(dim=-1)


def decode_layers(qkv: torch.Tensor, qn_w: torch.Tensor, kn_w: torch.Tensor, eps: float,
                  cos: torch.Tensor, sin: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor,
                  pos: int, bound: int, nh: int, nkv: int, scale: float) -> torch.Tensor:
    """The attention part of _decode_forward (cuda_graph_executor.py:164, :169-184) over all layers.

    qkv [L, 1, (nh+2nkv)*hd] per-layer projections; qn_w/kn_w [L, hd]; kc/vc [L, max_len, nkv, hd]
    (written in place); cos/sin [1, hd].  Returns ctx [L, nh*hd].
    """
    out = []
    for li in range(qkv.shape[0]):
        q, k, v = prologue(qkv[li], qn_w[li], kn_w[li], eps, cos, sin, nh, nkv)
        write_kv(kc[li], vc[li], k, v, pos)
        out.append(decode_attn(q, kc[li], vc[li], pos, bound, scale))
    return torch.cat(out, dim=0)


def decode_model_step(w: dict, tok: int, pos: int, kc: torch.Tensor, vc: torch.Tensor, bound: int, nh: int,
                      nkv: int, eps: float = 1e-6, theta: float = 1e6) -> torch.Tensor:
    """One greedy decode step of a whole model, cuda_graph_executor.py:163-190, on the CPU:
    embedding row, per layer input norm + fused QKV, q/k norm + RoPE + KV write + grouped attention,
    o_proj + residual, post norm + fused gate/up + silu(gate) * up + down + residual; final norm and
    lm_head.  w holds CPU tensors (embed, in_ln, post_ln, qn, kn, wqkv, wo, wgu, wd, final_norm,
    lm_head; per-layer entries indexable by layer).  kc/vc [L, max_len, nkv, hd] are written in
    place.  Every intermediate is rounded to the weights' dtype: bf16 as the reference runs, or fp32
    weights and caches for an unrounded yardstick of the same model.  Returns the logits [V]."""
    hd = kc.shape[-1]
    cos, sin = cos_sin(torch.tensor([pos]), inv_freq(hd, theta), w["embed"].dtype)
    x = w["embed"][tok].view(1, -1)
    for li in range(kc.shape[0]):
        h = rmsnorm(x, w["in_ln"][li], eps)
        qkv = linear(h, w["wqkv"][li])
        q, k, v = prologue(qkv, w["qn"][li], w["kn"][li], eps, cos, sin, nh, nkv, hd)
        write_kv(kc[li], vc[li], k, v, pos)
        ctx = decode_attn(q, kc[li], vc[li], pos, bound, hd ** -0.5)
        x = decode_mlp_block(x, ctx.view(1, -1), w["wo"][li], w["post_ln"][li], w["wgu"][li], w["wd"][li], eps)
    return linear(rmsnorm(x, w["final_norm"], eps), w["lm_head"]).view(-1)



def prefill_model(w: dict, ids: list[int], kc: torch.Tensor, vc: torch.Tensor, nh: int, nkv: int, eps: float = 1e-6,
                  theta: float = 1e6) -> torch.Tensor:
    """The prompt forward of a whole model, cuda_graph_executor.py:104-135, on the CPU in the weights'
    dtype: embedding rows, per layer input norm + fused QKV, q/k norm + RoPE + KV write of rows
    0..T-1 + causal grouped attention, o_proj + residual, post norm + gate/up + silu * up + down +
    residual.  kc/vc [L, max_len, nkv, hd] are written in place.  Returns the logits [V] of the
    last row (final norm and lm_head, :135 and :161)."""
    hd = kc.shape[-1]
    T = len(ids)
    cos, sin = cos_sin(torch.arange(T), inv_freq(hd, theta), w["embed"].dtype)
    x = w["embed"][torch.as_tensor(ids, dtype=torch.long)]
    for li in range(kc.shape[0]):
        qkv = linear(rmsnorm(x, w["in_ln"][li], eps), w["wqkv"][li])
        q, k, v = prologue(qkv, w["qn"][li], w["kn"][li], eps, cos, sin, nh, nkv, hd)
        write_kv(kc[li], vc[li], k, v, 0)
        ctx = prefill_attn(q, k, v, hd ** -0.5)
        x = decode_mlp_block(x, ctx, w["wo"][li], w["post_ln"][li], w["wgu"][li], w["wd"][li], eps)
    return linear(rmsnorm(x[T - 1:], w["final_norm"], eps), w["lm_head"]).view(-1)


def verify_model(w: dict, toks: list[int], pos0: int, kc: torch.Tensor, vc: torch.Tensor, nh: int, nkv: int,
                 eps: float = 1e-6, theta: float = 1e6) -> torch.Tensor:
    """The speculative-verify forward of a whole model, cuda_graph_executor.py:245-268, on the CPU in
    the weights' dtype: K+1 tokens at positions pos0..pos0+K, each layer writing their K/V rows and
    attending every cache key <= its position (all max_len keys under the mask).  Returns the
    logits [K+1, V]."""
    hd = kc.shape[-1]
    k1 = len(toks)
    cos, sin = cos_sin(pos0 + torch.arange(k1), inv_freq(hd, theta), w["embed"].dtype)
    x = w["embed"][torch.as_tensor(toks, dtype=torch.long)]
    for li in range(kc.shape[0]):
        qkv = linear(rmsnorm(x, w["in_ln"][li], eps), w["wqkv"][li])
        q, k, v = prologue(qkv, w["qn"][li], w["kn"][li], eps, cos, sin, nh, nkv, hd)
        write_kv(kc[li], vc[li], k, v, pos0)
        ctx = verify_attn(q, kc[li], vc[li], pos0, hd ** -0.5)
        x = decode_mlp_block(x, ctx, w["wo"][li], w["post_ln"][li], w["wgu"][li], w["wd"][li], eps)
    return linear(rmsnorm(x, w["final_norm"], eps), w["lm_head"])

# ---------------------------------------------------------------- paged KV cache (src/solort/cache/kv_cache.py)


def pages_required(token_count: int, page_size: int) -> int:
    """kv_cache.py:100-103."""
    return 0 if token_count <= 0 else (token_count + page_size - 1) // page_size


def last_page_len(token_count: int, page_size: int) -> int:
    """kv_cache.py:147-151."""
    if token_count <= 0:
        return 0
    rem = token_count % page_size
    return rem if rem else page_size


def slot_mapping(block_table: list[int], positions: list[int], page_size: int) -> list[int]:
    """kv_cache.py:131-145: logical position -> physical slot page * page_size + offset; a position
    whose logical page is past the block table raises IndexError."""
    slots = []
    for p in positions:
        lp = p // page_size
        if lp >= len(block_table):
            raise IndexError(f"position {p} needs logical page {lp}, but block table has {len(block_table)} pages")
        slots.append(block_table[lp] * page_size + p % page_size)
    return slots


def metadata_for(block_table: list[int], token_count: int, positions: list[int], page_size: int) -> dict:
    """kv_cache.py:113-129: the page-table view of one sequence."""
    n = pages_required(token_count, page_size)
    return {"page_indptr": [0, len(block_table[:n])], "page_indices": list(block_table[:n]),
            "last_page_len": [last_page_len(token_count, page_size)],
            "slot_mapping": slot_mapping(block_table, positions, page_size)}


def paged_store(kv_layer: torch.Tensor, slots: list[int], k: torch.Tensor, v: torch.Tensor) -> None:
    """store_layer_tokens, kv_cache.py:191-230, for one layer's arena kv_layer [pages, 2, page, nkv, hd]
    and rows k, v [tokens, nkv, hd] (the reference takes HF [1, nkv, tokens, hd] and transposes)."""
    ps = kv_layer.shape[2]
    for i, slot in enumerate(slots):
        kv_layer[slot // ps, 0, slot % ps].copy_(k[i])
        kv_layer[slot // ps, 1, slot % ps].copy_(v[i])


def paged_gather(kv_layer: torch.Tensor, slots: list[int]) -> tuple[torch.Tensor, torch.Tensor]:
    """gather_layer_tokens, kv_cache.py:232-256: rows [tokens, nkv, hd] of the given physical slots
    (slot = page * page_size + offset indexes the flattened [pages, page] grid)."""
    pages, _, ps, nkv, hd = kv_layer.shape
    idx = torch.as_tensor(slots, dtype=torch.long)
    flat_k = kv_layer[:, 0].reshape(pages * ps, nkv, hd)
    flat_v = kv_layer[:, 1].reshape(pages * ps, nkv, hd)
    return flat_k.index_select(0, idx).clone(), flat_v.index_select(0, idx).clone()
