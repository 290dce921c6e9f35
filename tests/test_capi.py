"""C-ABI checks that need no GPU: the library loads, exports every function the
header declares with the bound signature, and rejects bad arguments before any
launch.  The torch front end refuses CPU tensors (no CPU fallback)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from solort_amd import _lib, ops

HEADER = Path(__file__).resolve().parents[1] / "include" / "solort_hip.h"
EINVAL = -22


def _declared() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(solort_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_header_and_binding_agree():
    assert _declared() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.solort_abi_version() == _lib.ABI_VERSION


def test_workspace_sizes(lib):
    n = lib.solort_attn_workspace_bytes(1, 32, 8, 128, 32)
    # partial outputs [8][32][4][128] fp32 + (max, sum) per partial row
    assert n >= 8 * 32 * 4 * 128 * 4 + 8 * 32 * 4 * 2 * 4
    assert n % 256 == 0
    assert lib.solort_attn_workspace_bytes(1, 32, 8, 64, 32) == 0
    assert lib.solort_attn_workspace_bytes(1, 30, 8, 128, 32) == 0
    assert lib.solort_argmax_workspace_bytes(5) >= 5 * 12
    assert lib.solort_argmax_workspace_bytes(0) == 0


def _err(lib) -> str:
    return lib.solort_last_error().decode()


def test_decode_rejects_bad_arguments_without_launching(lib):
    p = ctypes.c_void_p(16 * 1024)  # never dereferenced: validation fails first
    args = dict(q=p, nq=1, nh=32, nkv=8, hd=128, k=p, v=p, ts=1024, hs=128, max_len=1024, pos=p,
                bound=1024, scale=0.088, ws=p, n_split=32, out=p, dt=0, stream=None)

    def call(**kw):
        a = {**args, **kw}
        return lib.solort_decode_attn(a["q"], a["nq"], a["nh"], a["nkv"], a["hd"], a["k"], a["v"], a["ts"],
                                      a["hs"], a["max_len"], a["pos"], a["bound"], a["scale"], a["ws"],
                                      a["n_split"], a["out"], a["dt"], a["stream"])

    assert call(hd=64) == EINVAL and "head_dim" in _err(lib)
    assert call(nh=30) == EINVAL
    assert call(nh=24, nkv=8) == EINVAL and "group" in _err(lib)
    assert call(nq=9) == EINVAL
    assert call(bound=2048) == EINVAL and "bound" in _err(lib)
    assert call(n_split=0) == EINVAL
    assert call(ts=1004) == EINVAL
    assert call(q=ctypes.c_void_p(16 * 1024 + 2)) == EINVAL and "aligned" in _err(lib)
    assert call(pos=None) == EINVAL
    assert call(dt=7) == EINVAL


def test_decode_qkv_layer_workspace_and_rejections(lib):
    # The attention's partials and counters, then per KV head (G + 2) rows of 128 handed-over
    # outputs as 8-byte (two bf16, tag) items.
    n = lib.solort_decode_qkv_workspace_bytes(32, 8, 32)
    assert n >= lib.solort_attn_workspace_bytes(1, 32, 8, 128, 32) + 8 * 6 * 64 * 8
    assert n % 256 == 0
    assert lib.solort_decode_qkv_workspace_bytes(30, 8, 32) == 0
    assert lib.solort_decode_qkv_workspace_bytes(32, 8, 0) == 0

    p = ctypes.c_void_p(16 * 1024)  # never dereferenced: validation fails first
    args = dict(x=p, hidden=2560, in_w=p, wqkv=p, wstride=2560, nh=32, nkv=8, hd=128, qn=p, kn=p, cs=p, pos=p,
                k=p, v=p, ts=1024, hs=128, max_len=1024, bound=1024, ws=p, n_split=32, qkv_out=p, out=p, dt=0)

    def call(**kw):
        a = {**args, **kw}
        return lib.solort_decode_qkv_layer(a["x"], a["hidden"], a["in_w"], 1e-6, a["wqkv"], a["wstride"], a["nh"],
                                           a["nkv"], a["hd"], a["qn"], a["kn"], 1e-6, a["cs"], a["pos"], a["k"],
                                           a["v"], a["ts"], a["hs"], a["max_len"], a["bound"], 0.088, a["ws"],
                                           a["n_split"], a["qkv_out"], a["out"], a["dt"], None)

    assert call(hd=64) == EINVAL and "head_dim" in _err(lib)
    assert call(bound=2048) == EINVAL and "bound" in _err(lib)
    assert call(pos=None) == EINVAL
    assert call(x=None) == EINVAL and "null" in _err(lib)
    assert call(wqkv=None) == EINVAL and "null" in _err(lib)
    assert call(qkv_out=None) == EINVAL and "null" in _err(lib)
    assert call(x=ctypes.c_void_p(16 * 1024 + 2)) == EINVAL and "aligned" in _err(lib)
    assert call(in_w=ctypes.c_void_p(16 * 1024 + 8)) == EINVAL and "aligned" in _err(lib)
    assert call(hidden=2564) == EINVAL and "hidden" in _err(lib)
    assert call(hidden=0) == EINVAL and "hidden" in _err(lib)
    assert call(wstride=2552) == EINVAL and "wqkv_row_stride" in _err(lib)


def test_prologue_and_argmax_reject_bad_arguments(lib):
    p = ctypes.c_void_p(4096)
    rc = lib.solort_qknorm_rope_kvwrite(p, 6144, 1, 32, 8, 100, p, p, 1e-6, p, None, p, p, p, 1024, 128, 1024,
                                        None)
    assert rc == EINVAL and "head_dim" in _err(lib)
    rc = lib.solort_qknorm_rope_kvwrite(p, 6000, 1, 32, 8, 128, p, p, 1e-6, p, None, p, p, p, 1024, 128, 1024,
                                        None)
    assert rc == EINVAL and "stride" in _err(lib)
    rc = lib.solort_qknorm_rope_kvwrite_cs(p, 6144, 4, 32, 8, 128, p, p, 1e-6, None, None, p, p, p, 1024, 128,
                                           1024, None)
    assert rc == EINVAL and "null" in _err(lib)
    rc = lib.solort_qknorm_rope_kvwrite_cs(p, 6144, 4, 30, 8, 128, p, p, 1e-6, p, None, p, p, p, 1024, 128, 1024,
                                           None)
    assert rc == EINVAL and "shape" in _err(lib)
    rc = lib.solort_decode_layer(p, 6144, 1, 32, 8, 128, p, p, 1e-6, None, p, p, p, 1024, 128, 1024, 1024, 0.088,
                                 p, 32, p, 0, None)
    assert rc == EINVAL and "null" in _err(lib)
    rc = lib.solort_rope_table(p, 60, 10, p, p, None)
    assert rc == EINVAL and "half_dim" in _err(lib)
    rc = lib.solort_rope_rows(p, 64, p, 0, p, None)
    assert rc == EINVAL and "n=0" in _err(lib)
    rc = lib.solort_rope_rows(p, 64, None, 1, p, None)
    assert rc == EINVAL and "null" in _err(lib)
    rc = lib.solort_argmax_rows(p, 3, 1, 10, 10, p, p, None)
    assert rc == EINVAL and "dtype" in _err(lib)
    rc = lib.solort_argmax_rows(p, 0, 1, 10, 5, p, p, None)
    assert rc == EINVAL


def test_prefill_entry_points_reject_bad_arguments(lib):
    p = ctypes.c_void_p(4096)
    rc = lib.solort_prefill_layer(p, 6144, 100, 24, 8, 128, p, p, 1e-6, p, p, p, 1024, 128, 1024, 0.088, p, 0, None)
    assert rc == EINVAL and "group" in _err(lib)
    rc = lib.solort_prefill_layer(p, 6144, 100, 32, 8, 128, p, p, 1e-6, None, p, p, 1024, 128, 1024, 0.088, p, 0,
                                  None)
    assert rc == EINVAL and "null" in _err(lib)
    rc = lib.solort_prefill_layer(p, 6000, 100, 32, 8, 128, p, p, 1e-6, p, p, p, 1024, 128, 1024, 0.088, p, 0, None)
    assert rc == EINVAL and "stride" in _err(lib)
    rc = lib.solort_prefill_layer(p, 6144, 2000, 32, 8, 128, p, p, 1e-6, p, p, p, 1024, 128, 1024, 0.088, p, 0,
                                  None)
    assert rc == EINVAL and "max_len" in _err(lib)
    rc = lib.solort_prefill_attn(p, 100, 32, 8, 128, p, p, 1024, 128, 1024, 0.088, p, 5, None)
    assert rc == EINVAL and "out_dtype" in _err(lib)
    rc = lib.solort_prefill_attn(None, 100, 32, 8, 128, p, p, 1024, 128, 1024, 0.088, p, 0, None)
    assert rc == EINVAL and "null" in _err(lib)


def test_gemv_entry_points_reject_bad_arguments(lib):
    p = ctypes.c_void_p(4096)
    rc = lib.solort_gemv(p, 2560, 100, 2560, p, None, 1e-6, None, 3, 0, p, None)
    assert rc == EINVAL and "mode" in _err(lib)
    rc = lib.solort_gemv(p, 2560, 100, 2564, p, None, 1e-6, None, 0, 0, p, None)
    assert rc == EINVAL and "shape" in _err(lib)
    rc = lib.solort_gemv(p, 2560, 100, 2560, p, None, 1e-6, None, 1, 0, p, None)
    assert rc == EINVAL and "null" in _err(lib)
    rc = lib.solort_gemv(p, 2560, 100, 2560, p, None, 1e-6, None, 2, 50, p, None)
    assert rc == EINVAL and "swiglu" in _err(lib)
    rc = lib.solort_gemv_argmax(p, 2560, 100, 2560, p, None, 1e-6, None, p, None, None)
    assert rc == EINVAL and "null" in _err(lib)
    rc = lib.solort_gemv_argmax(p, 2560, 100, 2560, p, None, 1e-6, None, p, ctypes.c_void_p(4096 + 4), None)
    assert rc == EINVAL and "aligned" in _err(lib)
    assert lib.solort_gemv_argmax_workspace_bytes(0) == 0
    assert lib.solort_gemv_argmax_workspace_bytes(151936) >= 151936 // 4 * 8
    rc = lib.solort_gemv_argmax(p, 2000, 100, 2560, p, None, 1e-6, None, p, p, None)
    assert rc == EINVAL and "stride" in _err(lib)


def test_paged_decode_rejects_bad_arguments(lib):
    p = ctypes.c_void_p(4096)
    args = lambda ps=16, pages=64, table=p, tlen=64, stride=2 * 16 * 1024: (  # noqa: E731
        p, 6144, 1, 32, 8, 128, p, p, 1e-6, p, p, p, p, stride, 1024, 128, ps, pages, table, tlen, 1024, 0.088, p,
        32, p, 0, None)
    assert lib.solort_paged_decode_layer(*args(ps=12)) == EINVAL and "power of two" in _err(lib)
    assert lib.solort_paged_decode_layer(*args(table=None)) == EINVAL and "page_table" in _err(lib)
    assert lib.solort_paged_decode_layer(*args(stride=1000)) == EINVAL and "page_stride" in _err(lib)
    assert lib.solort_paged_decode_layer(*args(tlen=32)) == EINVAL and "bound" in _err(lib)  # 512 rows < 1024
    assert lib.solort_paged_decode_layer(*args(pages=0)) == EINVAL


def test_paged_kv_copies_reject_bad_arguments(lib):
    p = ctypes.c_void_p(4096)
    st = lambda T=4, hd=128, slots=p, ps=16, stride=32768: lib.solort_paged_kv_store(  # noqa: E731
        p, p, 1024, 128, T, 8, hd, slots, p, p, stride, 1024, 128, ps, 8, None)
    assert st(hd=64) == EINVAL and "head_dim" in _err(lib)
    assert st(slots=None) == EINVAL and "null" in _err(lib)
    assert st(stride=1000) == EINVAL and "page" in _err(lib)
    assert st(ps=0) == EINVAL
    assert st(T=0) == 0  # nothing to copy
    rc = lib.solort_paged_kv_gather(p, p, 32768, 1024, 128, 16, 8, ctypes.c_void_p(4100), 4, 8, 128, p, p, 1024, 128,
                                    None)
    assert rc == EINVAL and "aligned" in _err(lib)


def test_read_heads_probe_rejects_bad_arguments(lib):
    p = ctypes.c_void_p(4096)
    rd = lambda k=p, rows=4096, nkv=8, ns=32, d=1: lib.solort_probe_read_heads(k, p, rows, nkv, ns, d, p,  # noqa: E731
                                                                             None)
    assert rd(k=None) == EINVAL and "aligned" in _err(lib)
    assert rd(k=ctypes.c_void_p(4100)) == EINVAL
    assert rd(rows=4000) == EINVAL and "multiple of 128" in _err(lib)
    assert rd(ns=3) == EINVAL
    assert rd(nkv=0) == EINVAL
    assert rd(d=3) == EINVAL and "tiles_in_flight" in _err(lib)


def test_torch_front_end_refuses_cpu_tensors():
    q = torch.zeros(1, 32, 128, dtype=torch.bfloat16)
    kc = torch.zeros(1024, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm device"):
        ops.decode_attn(q, kc, kc, torch.zeros(1, dtype=torch.long), 1024, 0.088,
                        torch.zeros(1 << 20, dtype=torch.uint8), 32, torch.zeros(1, 4096))
    with pytest.raises(RuntimeError, match="ROCm device"):
        ops.argmax_rows(torch.zeros(1, 10), torch.zeros(1, dtype=torch.long), torch.zeros(512, dtype=torch.uint8))


TRACE_HEADER = Path(__file__).resolve().parents[1] / "include" / "solort_trace.h"


def test_trace_header_binding_and_builds_agree(lib):
    """The tracing build's readers: declared in solort_trace.h exactly as bound, absent from the
    normal library (its kernels carry no stamps), present in the tracing build when it is built."""
    text = re.sub(r"/\*.*?\*/", "", TRACE_HEADER.read_text(), flags=re.S)
    declared = sorted(set(re.findall(r"\b(solort_[a-z0-9_]+)\s*\(", text)))
    assert declared == sorted(_lib.TRACE_SIGNATURES)
    assert not set(declared) & set(_lib.SIGNATURES)
    for name in declared:
        assert not hasattr(lib, name), name
    stamps = _lib.LIB_PATH.parent / "libsolort_hip_stamps.so"
    if stamps.exists():  # loaded in a process of its own: it registers the same kernels
        import subprocess
        import sys
        code = (f"import ctypes; l = ctypes.CDLL({str(stamps)!r}); "
                f"print(all(hasattr(l, n) for n in {declared!r}), l.solort_abi_version())")
        out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
        assert out.stdout.split() == ["True", str(_lib.ABI_VERSION)], out.stderr


def test_stamp_summary_on_synthetic_stamps():
    """bench.py's phase summary: microseconds after the first start, stale and missing slots
    (earlier launches, zeros) left out."""
    import numpy as np

    import bench

    t0 = 10_000_000
    st = np.zeros((4, 8), dtype=np.uint64)
    st[:, 0] = [t0, t0 + 10, t0 + 20, t0 + 30]       # starts: 0, 0.1, 0.2, 0.3 us
    st[:, 5] = [t0 + 500, t0 + 600, t0 + 700, 5]       # ends; the last is a stale stamp
    s = bench._stamp_summary(np, st, {0: "start", 5: "end", 6: "never"})
    assert s["start"]["max"] == 0.3 and s["start"]["workgroups"] == 4
    assert s["end"] == {"min": 5.0, "median": 6.0, "p90": 6.8, "max": 7.0, "workgroups": 3}
    assert "never" not in s
