"""torch-tensor front end of the HIP kernels (one function per C-ABI entry point).

Each function validates shapes, dtypes and devices on the host, then launches
on the current torch stream with no host synchronisation, so it can be
recorded inside ``torch.cuda.graph``.  Tensors must live on a ROCm device;
there is no CPU or torch fallback.

Layouts follow the reference runner (src/solort/model/cuda_graph_executor.py):
  qkv      [T, (nh + 2*nkv) * 128] bf16   fused QKV projection output (:115, :171, :253)
  cache    [max_len, nkv, 128] bf16       one layer of kc / vc (:67-69); any
                                           token/head strides with unit dim stride
  q        [T, nh, 128] bf16              prologue output
  ctx      [T, nh * 128]                  attention output, head-major (:129, :184, :264)
"""
from __future__ import annotations

import torch

from . import _lib

HD = 128
DTYPE_BF16 = 0
DTYPE_F32 = 1


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _on_gpu(name: str, t: torch.Tensor, dtype: torch.dtype) -> None:
    _need(t.is_cuda, f"{name} must be a ROCm device tensor (got {t.device})")
    _need(t.dtype == dtype, f"{name} must be {dtype} (got {t.dtype})")
    _need(t.data_ptr() % 16 == 0, f"{name} must be 16-byte aligned")


def _cache_strides(name: str, c: torch.Tensor, nkv: int) -> tuple[int, int, int]:
    _on_gpu(name, c, torch.bfloat16)
    _need(c.dim() == 3 and c.shape[1] == nkv and c.shape[2] == HD,
          f"{name} must be [max_len, {nkv}, {HD}] (got {tuple(c.shape)})")
    _need(c.stride(2) == 1, f"{name} needs unit stride along head_dim")
    return c.stride(0), c.stride(1), c.shape[0]


def inv_freq(hd: int, theta: float, device: torch.device | str) -> torch.Tensor:
    """RoPE frequencies 1 / theta^(2i/hd), fp32 [hd/2] on `device`: the reference's expression
    (cuda_graph_executor.py:64-66) evaluated by torch on the same device."""
    return (1.0 / (float(theta) ** (torch.arange(0, hd, 2, device=device).float() / hd))).contiguous()


def rope_tables(max_pos: int, hd: int, theta: float, device: torch.device | str,
                dtype: torch.dtype = torch.bfloat16) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin tables [max_pos, hd/2] for positions 0..max_pos-1, computed by torch.

    Row p equals the first half of the reference's ``_cos_sin(p)`` row
    (cuda_graph_executor.py:64-66, :95-98), built with the same torch
    expression on the same device; the second half of that row repeats the
    first because ``emb = cat(freqs, freqs)``.  The kernels evaluate these
    values themselves (solort_rope_table shows them); this torch version is
    what they are checked against.
    """
    freqs = torch.arange(max_pos, device=device)[:, None].float() * inv_freq(hd, theta, device)[None, :]
    return freqs.cos().to(dtype).contiguous(), freqs.sin().to(dtype).contiguous()


def rope_tables_device(inv_freq: torch.Tensor, rows: int) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin tables [rows, len(inv_freq)] computed by the library's kernel (solort_rope_table)."""
    _on_gpu("inv_freq", inv_freq, torch.float32)
    _need(inv_freq.dim() == 1 and inv_freq.is_contiguous(), "inv_freq must be 1-D contiguous")
    cos = torch.empty(rows, inv_freq.numel(), dtype=torch.bfloat16, device=inv_freq.device)
    sin = torch.empty_like(cos)
    rc = _lib.load().solort_rope_table(inv_freq.data_ptr(), inv_freq.numel(), rows, cos.data_ptr(),
                                       sin.data_ptr(), _stream(inv_freq))
    _lib.check(rc, "rope_table")
    return cos, sin


def rope_rows(inv_f: torch.Tensor, pos0: torch.Tensor, n: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """cos/sin rows [2, n, 64] bf16 of positions pos0..pos0+n-1 (pos0 int64 on the device), computed once
    per decode/verify step for every layer's decode_layer; see solort_rope_rows."""
    _inv_freq_ok(inv_f)
    _need(pos0.is_cuda and pos0.dtype == torch.int64 and pos0.numel() >= 1, "pos0 must be int64 on the device")
    if out is None:
        out = torch.empty(2, n, HD // 2, dtype=torch.bfloat16, device=inv_f.device)
    _rope_rows_ok(out, n)
    rc = _lib.load().solort_rope_rows(inv_f.data_ptr(), HD // 2, pos0.data_ptr(), int(n), out.data_ptr(),
                                      _stream(inv_f))
    _lib.check(rc, "rope_rows")
    return out


def _rope_rows_ok(cs: torch.Tensor, n: int) -> None:
    _on_gpu("rope_cs", cs, torch.bfloat16)
    _need(cs.shape == (2, n, HD // 2) and cs.is_contiguous() and cs.data_ptr() % 16 == 0,
          f"rope_cs must be [2, {n}, {HD // 2}] contiguous and 16-byte aligned")


def _inv_freq_ok(f: torch.Tensor) -> None:
    _on_gpu("inv_freq", f, torch.float32)
    _need(f.shape == (HD // 2,) and f.is_contiguous(), f"inv_freq must be [{HD // 2}] contiguous fp32")


def qknorm_rope_kvwrite(qkv: torch.Tensor, qn_w: torch.Tensor, kn_w: torch.Tensor, eps: float,
                        inv_f: torch.Tensor, pos0: torch.Tensor | None, q_out: torch.Tensor,
                        k_cache: torch.Tensor, v_cache: torch.Tensor, nh: int, nkv: int) -> None:
    """QK-RMSNorm + RoPE of T tokens at positions pos0..pos0+T-1, writing q_out and the caches.

    inv_f: fp32 [64] RoPE frequencies (inv_freq()); pos0: int64 [1] on the device (None = position 0).
    See solort_qknorm_rope_kvwrite.
    """
    _on_gpu("qkv", qkv, torch.bfloat16)
    _need(qkv.dim() == 2 and qkv.shape[1] == (nh + 2 * nkv) * HD and qkv.stride(1) == 1,
          f"qkv must be [T, {(nh + 2 * nkv) * HD}] with unit column stride")
    T = qkv.shape[0]
    for name, w in (("qn_w", qn_w), ("kn_w", kn_w)):
        _on_gpu(name, w, torch.bfloat16)
        _need(w.shape == (HD,) and w.is_contiguous(), f"{name} must be [{HD}] contiguous")
    _inv_freq_ok(inv_f)
    _on_gpu("q_out", q_out, torch.bfloat16)
    _need(q_out.shape == (T, nh, HD) and q_out.is_contiguous(), f"q_out must be [{T}, {nh}, {HD}]")
    ts, hs, max_len = _cache_strides("k_cache", k_cache, nkv)
    _need(v_cache.shape == k_cache.shape and v_cache.stride() == k_cache.stride(),
          "v_cache must match k_cache in shape and strides")
    _on_gpu("v_cache", v_cache, torch.bfloat16)
    pos_ptr = None
    if pos0 is not None:
        _need(pos0.is_cuda and pos0.dtype == torch.int64 and pos0.numel() >= 1, "pos0 must be int64 on the device")
        pos_ptr = pos0.data_ptr()
    lib = _lib.load()
    rc = lib.solort_qknorm_rope_kvwrite(
        qkv.data_ptr(), qkv.stride(0), T, nh, nkv, HD, qn_w.data_ptr(), kn_w.data_ptr(), float(eps),
        inv_f.data_ptr(), pos_ptr, q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), ts, hs, max_len,
        _stream(qkv))
    _lib.check(rc, "qknorm_rope_kvwrite")


def qknorm_rope_kvwrite_cs(qkv: torch.Tensor, qn_w: torch.Tensor, kn_w: torch.Tensor, eps: float,
                           rope_cs: torch.Tensor, pos0: torch.Tensor | None, q_out: torch.Tensor,
                           k_cache: torch.Tensor, v_cache: torch.Tensor, nh: int, nkv: int) -> None:
    """qknorm_rope_kvwrite with this step's cos/sin rows given: rope_cs = rope_rows(inv_f, pos0, T).
    Bit-identical results; see solort_qknorm_rope_kvwrite_cs."""
    _on_gpu("qkv", qkv, torch.bfloat16)
    _need(qkv.dim() == 2 and qkv.shape[1] == (nh + 2 * nkv) * HD and qkv.stride(1) == 1,
          f"qkv must be [T, {(nh + 2 * nkv) * HD}] with unit column stride")
    T = qkv.shape[0]
    for name, w in (("qn_w", qn_w), ("kn_w", kn_w)):
        _on_gpu(name, w, torch.bfloat16)
        _need(w.shape == (HD,) and w.is_contiguous(), f"{name} must be [{HD}] contiguous")
    _rope_rows_ok(rope_cs, T)
    _on_gpu("q_out", q_out, torch.bfloat16)
    _need(q_out.shape == (T, nh, HD) and q_out.is_contiguous(), f"q_out must be [{T}, {nh}, {HD}]")
    ts, hs, max_len = _cache_strides("k_cache", k_cache, nkv)
    _need(v_cache.shape == k_cache.shape and v_cache.stride() == k_cache.stride(),
          "v_cache must match k_cache in shape and strides")
    _on_gpu("v_cache", v_cache, torch.bfloat16)
    pos_ptr = None
    if pos0 is not None:
        _need(pos0.is_cuda and pos0.dtype == torch.int64 and pos0.numel() >= 1, "pos0 must be int64 on the device")
        pos_ptr = pos0.data_ptr()
    rc = _lib.load().solort_qknorm_rope_kvwrite_cs(
        qkv.data_ptr(), qkv.stride(0), T, nh, nkv, HD, qn_w.data_ptr(), kn_w.data_ptr(), float(eps),
        rope_cs.data_ptr(), pos_ptr, q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), ts, hs, max_len,
        _stream(qkv))
    _lib.check(rc, "qknorm_rope_kvwrite_cs")


def attn_workspace(nq: int, nh: int, nkv: int, n_split: int, device: torch.device | str) -> torch.Tensor:
    """Workspace for decode_attn / verify_attn / decode_layer (the splits' partials; allocate once,
    reuse for any call with no larger nq or n_split)."""
    nbytes = _lib.load().solort_attn_workspace_bytes(nq, nh, nkv, HD, n_split)
    _need(nbytes > 0, f"bad workspace request nq={nq} nh={nh} nkv={nkv} n_split={n_split}")
    return torch.zeros(nbytes, dtype=torch.uint8, device=device)


def _attn(fn_name: str, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
          pos0: torch.Tensor, bound: int, scale: float, ws: torch.Tensor, n_split: int,
          out: torch.Tensor) -> None:
    _on_gpu("q", q, torch.bfloat16)
    _need(q.dim() == 3 and q.shape[2] == HD and q.is_contiguous(), "q must be [nq, nh, 128] contiguous")
    nq, nh = q.shape[0], q.shape[1]
    nkv = k_cache.shape[1] if k_cache.dim() == 3 else -1
    ts, hs, max_len = _cache_strides("k_cache", k_cache, nkv)
    _on_gpu("v_cache", v_cache, torch.bfloat16)
    _need(v_cache.shape == k_cache.shape and v_cache.stride() == k_cache.stride(),
          "v_cache must match k_cache in shape and strides")
    _need(pos0.is_cuda and pos0.dtype == torch.int64 and pos0.numel() >= 1, "pos0 must be int64 on the device")
    _need(out.is_cuda and out.dtype in (torch.bfloat16, torch.float32), "out must be bf16 or fp32 on the device")
    _need(out.shape == (nq, nh * HD) and out.is_contiguous(), f"out must be [{nq}, {nh * HD}] contiguous")
    _need(out.data_ptr() % 16 == 0, "out must be 16-byte aligned")
    lib = _lib.load()
    need = lib.solort_attn_workspace_bytes(nq, nh, nkv, HD, n_split)
    _need(ws.is_cuda and ws.numel() * ws.element_size() >= need and ws.data_ptr() % 16 == 0,
          f"workspace too small: need {need} bytes")
    dt = DTYPE_F32 if out.dtype == torch.float32 else DTYPE_BF16
    rc = getattr(lib, fn_name)(
        q.data_ptr(), nq, nh, nkv, HD, k_cache.data_ptr(), v_cache.data_ptr(), ts, hs, max_len,
        pos0.data_ptr(), int(bound), float(scale), ws.data_ptr(), int(n_split), out.data_ptr(), dt,
        _stream(q))
    _lib.check(rc, fn_name)


def decode_attn(q, k_cache, v_cache, pos0, bound, scale, ws, n_split, out) -> None:
    """Single-token (or few-token) GQA attention over cache rows 0..pos0+nq-1; see solort_decode_attn."""
    _attn("solort_decode_attn", q, k_cache, v_cache, pos0, bound, scale, ws, n_split, out)


def verify_attn(q, k_cache, v_cache, pos0, bound, scale, ws, n_split, out) -> None:
    """K+1 query tokens at pos0..pos0+K, each causal over the cache; see solort_verify_attn."""
    _attn("solort_verify_attn", q, k_cache, v_cache, pos0, bound, scale, ws, n_split, out)


def decode_layer(qkv: torch.Tensor, qn_w: torch.Tensor, kn_w: torch.Tensor, eps: float, rope_cs: torch.Tensor,
                 pos0: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, bound: int, scale: float,
                 ws: torch.Tensor, n_split: int, out: torch.Tensor, nh: int, nkv: int) -> None:
    """One layer's attention block: prologue + KV write of the nq new tokens (qkv [nq, (nh+2nkv)*128])
    at pos0.. and split-KV attention into out [nq, nh*128].

    rope_cs: this step's rope_rows(inv_f, pos0, nq).  Equal to qknorm_rope_kvwrite followed by
    decode_attn; see solort_decode_layer.
    """
    _on_gpu("qkv", qkv, torch.bfloat16)
    _need(qkv.dim() == 2 and qkv.shape[1] == (nh + 2 * nkv) * HD and qkv.stride(1) == 1,
          f"qkv must be [nq, {(nh + 2 * nkv) * HD}] with unit column stride")
    nq = qkv.shape[0]
    for name, w in (("qn_w", qn_w), ("kn_w", kn_w)):
        _on_gpu(name, w, torch.bfloat16)
        _need(w.shape == (HD,) and w.is_contiguous(), f"{name} must be [{HD}] contiguous")
    _rope_rows_ok(rope_cs, nq)
    ts, hs, max_len = _cache_strides("k_cache", k_cache, nkv)
    _on_gpu("v_cache", v_cache, torch.bfloat16)
    _need(v_cache.shape == k_cache.shape and v_cache.stride() == k_cache.stride(),
          "v_cache must match k_cache in shape and strides")
    _need(pos0.is_cuda and pos0.dtype == torch.int64 and pos0.numel() >= 1, "pos0 must be int64 on the device")
    _need(out.is_cuda and out.dtype in (torch.bfloat16, torch.float32), "out must be bf16 or fp32 on the device")
    _need(out.shape == (nq, nh * HD) and out.is_contiguous() and out.data_ptr() % 16 == 0,
          f"out must be [{nq}, {nh * HD}] contiguous and 16-byte aligned")
    lib = _lib.load()
    need = lib.solort_attn_workspace_bytes(nq, nh, nkv, HD, n_split)
    _need(ws.is_cuda and ws.numel() * ws.element_size() >= need and ws.data_ptr() % 16 == 0,
          f"workspace too small: need {need} bytes")
    dt = DTYPE_F32 if out.dtype == torch.float32 else DTYPE_BF16
    rc = lib.solort_decode_layer(
        qkv.data_ptr(), qkv.stride(0), nq, nh, nkv, HD, qn_w.data_ptr(), kn_w.data_ptr(), float(eps),
        rope_cs.data_ptr(), pos0.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), ts, hs, max_len, int(bound),
        float(scale), ws.data_ptr(), int(n_split), out.data_ptr(), dt, _stream(qkv))
    _lib.check(rc, "decode_layer")


def decode_qkv_workspace(nh: int, nkv: int, n_split: int, device: torch.device | str) -> torch.Tensor:
    """Workspace for decode_qkv_layer (the splits' partials and the handed-over qkv rows)."""
    nbytes = _lib.load().solort_decode_qkv_workspace_bytes(nh, nkv, n_split)
    _need(nbytes > 0, f"bad workspace request nh={nh} nkv={nkv} n_split={n_split}")
    return torch.zeros(nbytes, dtype=torch.uint8, device=device)


def decode_qkv_layer(x: torch.Tensor, in_w: torch.Tensor, in_eps: float, wqkv: torch.Tensor, qn_w: torch.Tensor,
                     kn_w: torch.Tensor, eps: float, rope_cs: torch.Tensor, pos0: torch.Tensor, k_cache: torch.Tensor,
                     v_cache: torch.Tensor, bound: int, scale: float, ws: torch.Tensor, n_split: int,
                     qkv_out: torch.Tensor, out: torch.Tensor, nh: int, nkv: int) -> None:
    """One token's qkv product and attention block: qkv = rmsnorm(x, in_w) @ wqkv^T, then decode_layer
    on it into out [1, nh*128]; see solort_decode_qkv_layer (one launch where the shapes allow,
    else the product into qkv_out [(nh+2nkv)*128] and then decode_layer)."""
    width = (nh + 2 * nkv) * HD
    _on_gpu("x", x, torch.bfloat16)
    hidden = x.numel()
    _need(x.is_contiguous() and x.data_ptr() % 16 == 0, "x must be contiguous and 16-byte aligned")
    _on_gpu("in_w", in_w, torch.bfloat16)
    _need(in_w.shape == (hidden,) and in_w.is_contiguous(), f"in_w must be [{hidden}] contiguous")
    _on_gpu("wqkv", wqkv, torch.bfloat16)
    _need(wqkv.dim() == 2 and wqkv.shape == (width, hidden) and wqkv.stride(1) == 1,
          f"wqkv must be [{width}, {hidden}] with unit column stride")
    for name, w in (("qn_w", qn_w), ("kn_w", kn_w)):
        _on_gpu(name, w, torch.bfloat16)
        _need(w.shape == (HD,) and w.is_contiguous(), f"{name} must be [{HD}] contiguous")
    _rope_rows_ok(rope_cs, 1)
    ts, hs, max_len = _cache_strides("k_cache", k_cache, nkv)
    _on_gpu("v_cache", v_cache, torch.bfloat16)
    _need(v_cache.shape == k_cache.shape and v_cache.stride() == k_cache.stride(),
          "v_cache must match k_cache in shape and strides")
    _need(pos0.is_cuda and pos0.dtype == torch.int64 and pos0.numel() >= 1, "pos0 must be int64 on the device")
    _on_gpu("qkv_out", qkv_out, torch.bfloat16)
    _need(qkv_out.numel() >= width and qkv_out.is_contiguous(), f"qkv_out must hold {width} contiguous elements")
    _need(out.is_cuda and out.dtype in (torch.bfloat16, torch.float32), "out must be bf16 or fp32 on the device")
    _need(out.shape == (1, nh * HD) and out.is_contiguous() and out.data_ptr() % 16 == 0,
          f"out must be [1, {nh * HD}] contiguous and 16-byte aligned")
    lib = _lib.load()
    need = lib.solort_decode_qkv_workspace_bytes(nh, nkv, n_split)
    _need(ws.is_cuda and ws.numel() * ws.element_size() >= need and ws.data_ptr() % 16 == 0,
          f"workspace too small: need {need} bytes")
    dt = DTYPE_F32 if out.dtype == torch.float32 else DTYPE_BF16
    rc = lib.solort_decode_qkv_layer(
        x.data_ptr(), hidden, in_w.data_ptr(), float(in_eps), wqkv.data_ptr(), wqkv.stride(0), nh, nkv, HD,
        qn_w.data_ptr(), kn_w.data_ptr(), float(eps), rope_cs.data_ptr(), pos0.data_ptr(), k_cache.data_ptr(),
        v_cache.data_ptr(), ts, hs, max_len, int(bound), float(scale), ws.data_ptr(), int(n_split),
        qkv_out.data_ptr(), out.data_ptr(), dt, _stream(x))
    _lib.check(rc, "decode_qkv_layer")


def decode_layer_noalloc(qkv: torch.Tensor, qn_w: torch.Tensor, kn_w: torch.Tensor, eps: float,
                         rope_cs: torch.Tensor, pos0: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                         bound: int, scale: float, n_split: int, out: torch.Tensor, nh: int, nkv: int) -> None:
    """decode_layer with the partials in the library's fixed per-GPU scratch array instead of a
    workspace (no allocation anywhere; calls that overlap on one GPU race); see
    solort_decode_layer_noalloc."""
    _on_gpu("qkv", qkv, torch.bfloat16)
    _need(qkv.dim() == 2 and qkv.shape[1] == (nh + 2 * nkv) * HD and qkv.stride(1) == 1,
          f"qkv must be [nq, {(nh + 2 * nkv) * HD}] with unit column stride")
    nq = qkv.shape[0]
    for name, w in (("qn_w", qn_w), ("kn_w", kn_w)):
        _on_gpu(name, w, torch.bfloat16)
        _need(w.shape == (HD,) and w.is_contiguous(), f"{name} must be [{HD}] contiguous")
    _rope_rows_ok(rope_cs, nq)
    ts, hs, max_len = _cache_strides("k_cache", k_cache, nkv)
    _on_gpu("v_cache", v_cache, torch.bfloat16)
    _need(v_cache.shape == k_cache.shape and v_cache.stride() == k_cache.stride(),
          "v_cache must match k_cache in shape and strides")
    _need(pos0.is_cuda and pos0.dtype == torch.int64 and pos0.numel() >= 1, "pos0 must be int64 on the device")
    _need(out.is_cuda and out.dtype in (torch.bfloat16, torch.float32), "out must be bf16 or fp32 on the device")
    _need(out.shape == (nq, nh * HD) and out.is_contiguous() and out.data_ptr() % 16 == 0,
          f"out must be [{nq}, {nh * HD}] contiguous and 16-byte aligned")
    dt = DTYPE_F32 if out.dtype == torch.float32 else DTYPE_BF16
    rc = _lib.load().solort_decode_layer_noalloc(
        qkv.data_ptr(), qkv.stride(0), nq, nh, nkv, HD, qn_w.data_ptr(), kn_w.data_ptr(), float(eps),
        rope_cs.data_ptr(), pos0.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), ts, hs, max_len, int(bound),
        float(scale), int(n_split), out.data_ptr(), dt, _stream(qkv))
    _lib.check(rc, "decode_layer_noalloc")


def paged_decode_layer(qkv: torch.Tensor, qn_w: torch.Tensor, kn_w: torch.Tensor, eps: float, rope_cs: torch.Tensor,
                       pos0: torch.Tensor, kv_pages: torch.Tensor, page_table: torch.Tensor, bound: int,
                       scale: float, ws: torch.Tensor, n_split: int, out: torch.Tensor, nh: int, nkv: int) -> None:
    """decode_layer over one layer of a paged KV cache kv_pages [num_pages, 2, page_size, nkv, 128] bf16
    (the reference PagedKVCache's per-layer arena, kv_cache.py:71-100), through page_table int32
    [>= ceil(bound / page_size)] (logical page -> physical page); see solort_paged_decode_layer."""
    _on_gpu("qkv", qkv, torch.bfloat16)
    _need(qkv.dim() == 2 and qkv.shape[1] == (nh + 2 * nkv) * HD and qkv.stride(1) == 1,
          f"qkv must be [nq, {(nh + 2 * nkv) * HD}] with unit column stride")
    nq = qkv.shape[0]
    for name, w in (("qn_w", qn_w), ("kn_w", kn_w)):
        _on_gpu(name, w, torch.bfloat16)
        _need(w.shape == (HD,) and w.is_contiguous(), f"{name} must be [{HD}] contiguous")
    _rope_rows_ok(rope_cs, nq)
    _on_gpu("kv_pages", kv_pages, torch.bfloat16)
    _need(kv_pages.dim() == 5 and kv_pages.shape[1] == 2 and kv_pages.shape[3] == nkv and kv_pages.shape[4] == HD
          and kv_pages.stride(4) == 1, f"kv_pages must be [num_pages, 2, page_size, {nkv}, {HD}]")
    num_pages, _, page_size = kv_pages.shape[:3]
    _need(page_table.is_cuda and page_table.dtype == torch.int32 and page_table.dim() == 1
          and page_table.is_contiguous(), "page_table must be a contiguous int32 vector on the device")
    _need(page_table.numel() * page_size >= bound, f"page_table covers {page_table.numel() * page_size} < bound {bound}")
    _need(pos0.is_cuda and pos0.dtype == torch.int64 and pos0.numel() >= 1, "pos0 must be int64 on the device")
    _need(out.is_cuda and out.dtype in (torch.bfloat16, torch.float32), "out must be bf16 or fp32 on the device")
    _need(out.shape == (nq, nh * HD) and out.is_contiguous() and out.data_ptr() % 16 == 0,
          f"out must be [{nq}, {nh * HD}] contiguous and 16-byte aligned")
    lib = _lib.load()
    need = lib.solort_attn_workspace_bytes(nq, nh, nkv, HD, n_split)
    _need(ws.is_cuda and ws.numel() * ws.element_size() >= need and ws.data_ptr() % 16 == 0,
          f"workspace too small: need {need} bytes")
    dt = DTYPE_F32 if out.dtype == torch.float32 else DTYPE_BF16
    k_pages, v_pages = kv_pages[:, 0], kv_pages[:, 1]
    rc = lib.solort_paged_decode_layer(
        qkv.data_ptr(), qkv.stride(0), nq, nh, nkv, HD, qn_w.data_ptr(), kn_w.data_ptr(), float(eps),
        rope_cs.data_ptr(), pos0.data_ptr(), k_pages.data_ptr(), v_pages.data_ptr(), kv_pages.stride(0),
        kv_pages.stride(2), kv_pages.stride(3), int(page_size), int(num_pages), page_table.data_ptr(),
        page_table.numel(), int(bound), float(scale), ws.data_ptr(), int(n_split), out.data_ptr(), dt, _stream(qkv))
    _lib.check(rc, "paged_decode_layer")


def _paged_arena(kv_pages: torch.Tensor) -> tuple[int, int, int]:
    _on_gpu("kv_pages", kv_pages, torch.bfloat16)
    _need(kv_pages.dim() == 5 and kv_pages.shape[1] == 2 and kv_pages.shape[4] == HD and kv_pages.stride(4) == 1,
          f"kv_pages must be [num_pages, 2, page_size, nkv, {HD}]")
    return kv_pages.shape[0], kv_pages.shape[2], kv_pages.shape[3]


def _slot_rows(k_rows: torch.Tensor, v_rows: torch.Tensor, slot_mapping: torch.Tensor, nkv: int) -> int:
    for name, t in (("k_rows", k_rows), ("v_rows", v_rows)):
        _on_gpu(name, t, torch.bfloat16)
        _need(t.dim() == 3 and t.shape[1] == nkv and t.shape[2] == HD and t.stride(2) == 1,
              f"{name} must be [T, {nkv}, {HD}] with unit dim stride")
    _need(v_rows.shape == k_rows.shape and v_rows.stride() == k_rows.stride(), "k_rows and v_rows must match")
    T = k_rows.shape[0]
    _need(slot_mapping.is_cuda and slot_mapping.dtype == torch.int64 and slot_mapping.is_contiguous()
          and slot_mapping.numel() == T, f"slot_mapping must be int64 [{T}] on the device")
    return T


def paged_kv_store(k_rows: torch.Tensor, v_rows: torch.Tensor, slot_mapping: torch.Tensor,
                   kv_pages: torch.Tensor) -> None:
    """Rows k_rows/v_rows [T, nkv, 128] -> physical slots slot_mapping [T] of the paged arena kv_pages
    [num_pages, 2, page_size, nkv, 128] (store_layer_tokens, kv_cache.py:191-230); see
    solort_paged_kv_store."""
    num_pages, page_size, nkv = _paged_arena(kv_pages)
    T = _slot_rows(k_rows, v_rows, slot_mapping, nkv)
    rc = _lib.load().solort_paged_kv_store(
        k_rows.data_ptr(), v_rows.data_ptr(), k_rows.stride(0), k_rows.stride(1), T, nkv, HD, slot_mapping.data_ptr(),
        kv_pages[:, 0].data_ptr(), kv_pages[:, 1].data_ptr(), kv_pages.stride(0), kv_pages.stride(2),
        kv_pages.stride(3), page_size, num_pages, _stream(kv_pages))
    _lib.check(rc, "paged_kv_store")


def paged_kv_gather(kv_pages: torch.Tensor, slot_mapping: torch.Tensor, k_rows: torch.Tensor,
                    v_rows: torch.Tensor) -> None:
    """Physical slots slot_mapping [T] of kv_pages -> rows k_rows/v_rows [T, nkv, 128]
    (gather_layer_tokens, kv_cache.py:232-256); see solort_paged_kv_gather."""
    num_pages, page_size, nkv = _paged_arena(kv_pages)
    T = _slot_rows(k_rows, v_rows, slot_mapping, nkv)
    rc = _lib.load().solort_paged_kv_gather(
        kv_pages[:, 0].data_ptr(), kv_pages[:, 1].data_ptr(), kv_pages.stride(0), kv_pages.stride(2),
        kv_pages.stride(3), page_size, num_pages, slot_mapping.data_ptr(), T, nkv, HD, k_rows.data_ptr(),
        v_rows.data_ptr(), k_rows.stride(0), k_rows.stride(1), _stream(kv_pages))
    _lib.check(rc, "paged_kv_gather")


def prefill_attn(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, scale: float,
                 out: torch.Tensor) -> None:
    """Causal GQA attention of T prompt rows (q [T, nh, 128]) over cache rows 0..T-1 into
    out [T, nh*128]; see solort_prefill_attn."""
    _on_gpu("q", q, torch.bfloat16)
    _need(q.dim() == 3 and q.shape[2] == HD and q.is_contiguous(), "q must be [T, nh, 128] contiguous")
    T, nh = q.shape[0], q.shape[1]
    nkv = k_cache.shape[1] if k_cache.dim() == 3 else -1
    ts, hs, max_len = _cache_strides("k_cache", k_cache, nkv)
    _on_gpu("v_cache", v_cache, torch.bfloat16)
    _need(v_cache.shape == k_cache.shape and v_cache.stride() == k_cache.stride(),
          "v_cache must match k_cache in shape and strides")
    _need(out.is_cuda and out.dtype in (torch.bfloat16, torch.float32), "out must be bf16 or fp32 on the device")
    _need(out.shape == (T, nh * HD) and out.is_contiguous() and out.data_ptr() % 16 == 0,
          f"out must be [{T}, {nh * HD}] contiguous and 16-byte aligned")
    dt = DTYPE_F32 if out.dtype == torch.float32 else DTYPE_BF16
    rc = _lib.load().solort_prefill_attn(q.data_ptr(), T, nh, nkv, HD, k_cache.data_ptr(), v_cache.data_ptr(), ts,
                                         hs, max_len, float(scale), out.data_ptr(), dt, _stream(q))
    _lib.check(rc, "prefill_attn")


def prefill_layer(qkv: torch.Tensor, qn_w: torch.Tensor, kn_w: torch.Tensor, eps: float, rope_cs: torch.Tensor,
                  k_cache: torch.Tensor, v_cache: torch.Tensor, scale: float, out: torch.Tensor, nh: int,
                  nkv: int) -> None:
    """One layer's prefill attention block for T prompt rows at positions 0..T-1: qkv
    [T, (nh+2nkv)*128] -> K/V cache rows 0..T-1 and out [T, nh*128]; rope_cs = rope_rows(inv_f,
    0, T).  Equal, bit for bit, to qknorm_rope_kvwrite_cs + prefill_attn; see solort_prefill_layer."""
    _on_gpu("qkv", qkv, torch.bfloat16)
    _need(qkv.dim() == 2 and qkv.shape[1] == (nh + 2 * nkv) * HD and qkv.stride(1) == 1,
          f"qkv must be [T, {(nh + 2 * nkv) * HD}] with unit column stride")
    T = qkv.shape[0]
    for name, w in (("qn_w", qn_w), ("kn_w", kn_w)):
        _on_gpu(name, w, torch.bfloat16)
        _need(w.shape == (HD,) and w.is_contiguous(), f"{name} must be [{HD}] contiguous")
    _rope_rows_ok(rope_cs, T)
    ts, hs, max_len = _cache_strides("k_cache", k_cache, nkv)
    _on_gpu("v_cache", v_cache, torch.bfloat16)
    _need(v_cache.shape == k_cache.shape and v_cache.stride() == k_cache.stride(),
          "v_cache must match k_cache in shape and strides")
    _need(out.is_cuda and out.dtype in (torch.bfloat16, torch.float32), "out must be bf16 or fp32 on the device")
    _need(out.shape == (T, nh * HD) and out.is_contiguous() and out.data_ptr() % 16 == 0,
          f"out must be [{T}, {nh * HD}] contiguous and 16-byte aligned")
    dt = DTYPE_F32 if out.dtype == torch.float32 else DTYPE_BF16
    rc = _lib.load().solort_prefill_layer(
        qkv.data_ptr(), qkv.stride(0), T, nh, nkv, HD, qn_w.data_ptr(), kn_w.data_ptr(), float(eps),
        rope_cs.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), ts, hs, max_len, float(scale), out.data_ptr(), dt,
        _stream(qkv))
    _lib.check(rc, "prefill_layer")


def argmax_workspace(rows: int, device: torch.device | str) -> torch.Tensor:
    """Zero-filled workspace for argmax_rows (allocate once, reuse)."""
    nbytes = _lib.load().solort_argmax_workspace_bytes(rows)
    _need(nbytes > 0, f"bad argmax workspace request rows={rows}")
    return torch.zeros(nbytes, dtype=torch.uint8, device=device)


def argmax_rows(logits: torch.Tensor, out: torch.Tensor, ws: torch.Tensor) -> None:
    """out[r] = index of the max of logits[r] (lowest index on ties, NaN is max)."""
    _need(logits.is_cuda, f"logits must be a ROCm device tensor (got {logits.device})")
    _need(logits.dtype in (torch.bfloat16, torch.float32), f"logits must be bf16 or fp32 (got {logits.dtype})")
    _need(logits.dim() == 2 and logits.stride(1) == 1, "logits must be [rows, vocab] with unit column stride")
    rows, vocab = logits.shape
    _need(out.is_cuda and out.dtype == torch.int64 and out.shape == (rows,) and out.is_contiguous(),
          f"out must be int64 [{rows}] on the device")
    lib = _lib.load()
    need = lib.solort_argmax_workspace_bytes(rows)
    _need(ws.is_cuda and ws.numel() * ws.element_size() >= need and ws.data_ptr() % 16 == 0,
          f"argmax workspace too small: need {need} bytes")
    dt = DTYPE_F32 if logits.dtype == torch.float32 else DTYPE_BF16
    rc = lib.solort_argmax_rows(logits.data_ptr(), dt, rows, vocab, logits.stride(0), out.data_ptr(),
                                ws.data_ptr(), _stream(logits))
    _lib.check(rc, "argmax_rows")


def argmax_mode(mode: int = -1) -> int:
    """Reduction mode of argmax_rows on the current device: 1 = one launch (where the placement
    check passed), 0 = always a second launch, 2 = one launch whose reducing block gives up at once
    (test mode of the failure path), -1 = query; returns the mode in effect."""
    rc = _lib.load().solort_argmax_mode(int(mode))
    if rc < 0:
        _lib.check(rc, f"argmax_mode({mode})")
    return rc


# 16-byte items per argmax row: 64 chunk slots, then (epoch, failure count, -, -).
_ARGMAX_ROW_ITEMS = 65


def argmax_failures(ws: torch.Tensor, rows: int) -> int:
    """Total failure count of the first `rows` rows of an argmax_rows workspace: calls whose
    reduction did not see every block's key (their index is the best key found).  Reads the
    device (one synchronisation)."""
    w = ws[: rows * _ARGMAX_ROW_ITEMS * 16].view(torch.int32).view(rows, _ARGMAX_ROW_ITEMS * 4)
    return int(w[:, 64 * 4 + 1].sum().item())


def check_tokens(tokens: list[int], vocab: int, what: str) -> list[int]:
    """Raises RuntimeError unless every token lies in [0, vocab)."""
    bad = [t for t in tokens if not 0 <= t < vocab]
    if bad:
        raise RuntimeError(f"{what}: token(s) {bad[:4]} outside the vocabulary [0, {vocab})")
    return tokens


def accept_prefix(target: torch.Tensor, draft: torch.Tensor, out: torch.Tensor) -> None:
    """out[0] = length of the prefix of draft [k] that target [k+1] agrees with, out[1] = target[out[0]]
    (int64, on the device); see solort_accept_prefix."""
    _need(target.is_cuda and draft.is_cuda and out.is_cuda, "target, draft and out must be on the ROCm device")
    _need(target.dtype == torch.int64 and draft.dtype == torch.int64 and out.dtype == torch.int64,
          "target, draft and out must be int64")
    k = draft.numel()
    _need(draft.is_contiguous() and target.is_contiguous() and target.numel() == k + 1,
          f"target must hold k+1 = {k + 1} tokens")
    _need(out.is_contiguous() and out.numel() >= 2, "out must hold 2 int64")
    rc = _lib.load().solort_accept_prefix(target.data_ptr(), draft.data_ptr(), k, out.data_ptr(), _stream(target))
    _lib.check(rc, "accept_prefix")


GEMV_PLAIN, GEMV_RESID, GEMV_SWIGLU = 0, 1, 2


def gemv(w: torch.Tensor, x: torch.Tensor, out: torch.Tensor, norm_w: torch.Tensor | None = None,
         eps: float = 1e-6, res: torch.Tensor | None = None, mode: int = GEMV_PLAIN, inter: int = 0) -> None:
    """One-token matrix-vector product out = W x with the decode step's fused neighbours (see
    solort_gemv): optional RMSNorm of x (norm_w), residual add (mode GEMV_RESID, res, may be out), or
    SwiGLU over gate rows 0..n-1 and up rows inter..inter+n-1 (GEMV_SWIGLU).  w [rows, k] bf16, x [k]
    bf16, out [n] bf16."""
    for name, t in (("w", w), ("x", x), ("out", out)):
        _on_gpu(name, t, torch.bfloat16)
    _need(w.dim() == 2 and w.stride(1) == 1, "w must be [rows, k] with unit column stride")
    k = w.shape[1]
    _need(x.numel() == k and x.is_contiguous(), f"x must hold k = {k} contiguous values")
    n = out.numel()
    _need(out.is_contiguous(), "out must be contiguous")
    if mode == GEMV_SWIGLU:
        _need(inter >= n and w.shape[0] >= inter + n, f"w must hold gate and up rows (inter {inter}, n {n})")
    else:
        _need(w.shape[0] >= n, f"w has {w.shape[0]} rows, fewer than n = {n}")
    if norm_w is not None:
        _on_gpu("norm_w", norm_w, torch.bfloat16)
        _need(norm_w.numel() == k and norm_w.is_contiguous(), f"norm_w must hold k = {k} values")
    if mode == GEMV_RESID:
        _need(res is not None, "GEMV_RESID needs res")
        _on_gpu("res", res, torch.bfloat16)
        _need(res.numel() == n and res.is_contiguous(), f"res must hold n = {n} values")
    rc = _lib.load().solort_gemv(w.data_ptr(), w.stride(0), n, k, x.data_ptr(),
                                 None if norm_w is None else norm_w.data_ptr(), float(eps),
                                 None if res is None else res.data_ptr(), int(mode), int(inter), out.data_ptr(),
                                 _stream(w))
    _lib.check(rc, "gemv")


def gemv_argmax_workspace(n_out: int, device: torch.device | str) -> torch.Tensor:
    """Workspace for gemv_argmax over n_out outputs (allocate once, reuse)."""
    nbytes = _lib.load().solort_gemv_argmax_workspace_bytes(int(n_out))
    _need(nbytes > 0, f"bad gemv_argmax workspace request n_out={n_out}")
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def gemv_argmax(w: torch.Tensor, x: torch.Tensor, out_idx: torch.Tensor | None, ws: torch.Tensor,
                norm_w: torch.Tensor | None = None, eps: float = 1e-6, logits: torch.Tensor | None = None) -> None:
    """out_idx[0] = argmax(rmsnorm(x, norm_w) @ w.T) (lowest index on ties, NaN is max), the argmax
    folded into the product's workgroups, optionally writing the bf16 logits; see solort_gemv_argmax.
    w [V, k] bf16, x [k] bf16, out_idx int64 [1] (None: leave the keys in ws for greedy_advance), ws from
    gemv_argmax_workspace(V)."""
    for name, t in (("w", w), ("x", x)):
        _on_gpu(name, t, torch.bfloat16)
    _need(w.dim() == 2 and w.stride(1) == 1, "w must be [rows, k] with unit column stride")
    n, k = w.shape
    _need(x.numel() == k and x.is_contiguous(), f"x must hold k = {k} contiguous values")
    if out_idx is not None:
        _need(out_idx.is_cuda and out_idx.dtype == torch.int64 and out_idx.numel() >= 1 and out_idx.is_contiguous(),
              "out_idx must be int64 on the device")
    lib = _lib.load()
    need = lib.solort_gemv_argmax_workspace_bytes(n)
    _need(need > 0 and ws.is_cuda and ws.numel() * ws.element_size() >= need and ws.data_ptr() % 8 == 0,
          f"gemv_argmax workspace too small or misaligned: need {need} bytes, 8-byte aligned")
    if norm_w is not None:
        _on_gpu("norm_w", norm_w, torch.bfloat16)
        _need(norm_w.numel() == k and norm_w.is_contiguous(), f"norm_w must hold k = {k} values")
    if logits is not None:
        _on_gpu("logits", logits, torch.bfloat16)
        _need(logits.numel() == n and logits.is_contiguous(), f"logits must hold {n} values")
    rc = lib.solort_gemv_argmax(w.data_ptr(), w.stride(0), n, k, x.data_ptr(),
                                None if norm_w is None else norm_w.data_ptr(), float(eps),
                                None if logits is None else logits.data_ptr(),
                                None if out_idx is None else out_idx.data_ptr(), ws.data_ptr(), _stream(w))
    _lib.check(rc, "gemv_argmax")


def greedy_advance(ws: torch.Tensor, vocab: int, embed: torch.Tensor, x: torch.Tensor, tok: torch.Tensor,
                   tokens: torch.Tensor | None, step: torch.Tensor, pos: torch.Tensor) -> None:
    """After gemv_argmax(..., out_idx=None, ws): tok = the argmax token, tokens[step] = tok (if step <
    tokens.numel()), step += 1, pos += 1, x = embed[tok]; see solort_greedy_advance.  embed [vocab,
    hidden] bf16, x [hidden] bf16, tok/step/pos int64 [1], tokens int64 [max_tokens]."""
    _on_gpu("embed", embed, torch.bfloat16)
    _on_gpu("x", x, torch.bfloat16)
    _need(embed.dim() == 2 and embed.stride(1) == 1 and embed.shape[0] >= vocab, "embed must be [>= vocab, hidden]")
    hidden = embed.shape[1]
    _need(x.numel() == hidden and x.is_contiguous(), f"x must hold hidden = {hidden} values")
    for name, t in (("tok", tok), ("step", step), ("pos", pos)) + ((("tokens", tokens),) if tokens is not None else ()):
        _need(t.is_cuda and t.dtype == torch.int64 and t.is_contiguous() and t.numel() >= 1,
              f"{name} must be int64 on the device")
    lib = _lib.load()
    _need(ws.is_cuda and ws.numel() * ws.element_size() >= lib.solort_gemv_argmax_workspace_bytes(int(vocab)),
          "ws must be the gemv_argmax workspace of this vocabulary")
    rc = lib.solort_greedy_advance(ws.data_ptr(), int(vocab), embed.data_ptr(), embed.stride(0), hidden, x.data_ptr(),
                                   tok.data_ptr(), None if tokens is None else tokens.data_ptr(),
                                   0 if tokens is None else tokens.numel(), step.data_ptr(), pos.data_ptr(),
                                   _stream(x))
    _lib.check(rc, "greedy_advance")
