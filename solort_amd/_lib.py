"""ctypes binding of libsolort_hip.so (the C ABI declared in include/solort_hip.h).

The library must already be built (``python -m solort_amd.build``); there is
no fallback: a missing or stale library raises ``RuntimeError``.  torch is
imported first so that the HIP runtime torch ships is the one the library
binds to (both carry the soname libamdhip64.so.7), which makes torch's
stream handles valid arguments.
"""
from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_int64, c_size_t, c_void_p
from pathlib import Path

import torch  # noqa: F401  (loads torch's HIP runtime before ours)

LIB_PATH = Path(__file__).resolve().parent / "libsolort_hip.so"
ABI_VERSION = 10

# name -> (restype, argtypes); mirrors include/solort_hip.h
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "solort_abi_version": (c_int, []),
    "solort_source_id": (ctypes.c_uint64, []),
    "solort_last_error": (ctypes.c_char_p, []),
    "solort_init": (c_int, []),
    "solort_combine_mode": (c_int, [c_int]),
    "solort_argmax_mode": (c_int, [c_int]),
    "solort_probe_placement": (c_int, [c_void_p, c_int, c_void_p]),
    "solort_probe_empty": (c_int, [c_int, c_void_p]),
    "solort_probe_read": (c_int, [c_void_p, c_int64, c_int, c_int, c_void_p, c_void_p]),
    "solort_probe_read_heads": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_void_p, c_void_p]),
    "solort_qknorm_rope_kvwrite": (
        c_int,
        [c_void_p, c_int64, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_float, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p],
    ),
    "solort_qknorm_rope_kvwrite_cs": (
        c_int,
        [c_void_p, c_int64, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_float, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p],
    ),
    "solort_rope_table": (c_int, [c_void_p, c_int, c_int64, c_void_p, c_void_p, c_void_p]),
    "solort_rope_rows": (c_int, [c_void_p, c_int, c_void_p, c_int, c_void_p, c_void_p]),
    "solort_attn_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "solort_decode_attn": (
        c_int,
        [c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_int64, c_int64, c_int64,
         c_void_p, c_int, c_float, c_void_p, c_int, c_void_p, c_int, c_void_p],
    ),
    "solort_verify_attn": (
        c_int,
        [c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_int64, c_int64, c_int64,
         c_void_p, c_int, c_float, c_void_p, c_int, c_void_p, c_int, c_void_p],
    ),
    "solort_decode_layer": (
        c_int,
        [c_void_p, c_int64, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_float, c_void_p, c_void_p,
         c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int, c_float, c_void_p, c_int, c_void_p, c_int,
         c_void_p],
    ),
    "solort_prefill_attn": (
        c_int,
        [c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_float,
         c_void_p, c_int, c_void_p],
    ),
    "solort_decode_qkv_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "solort_decode_qkv_layer": (
        c_int,
        [c_void_p, c_int, c_void_p, c_float, c_void_p, c_int64, c_int, c_int, c_int, c_void_p, c_void_p, c_float,
         c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int, c_float, c_void_p, c_int, c_void_p,
         c_void_p, c_int, c_void_p],
    ),
    "solort_decode_layer_noalloc": (
        c_int,
        [c_void_p, c_int64, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_float, c_void_p, c_void_p,
         c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int, c_float, c_int, c_void_p, c_int, c_void_p],
    ),
    "solort_paged_decode_layer": (
        c_int,
        [c_void_p, c_int64, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_float, c_void_p, c_void_p, c_void_p,
         c_void_p, c_int64, c_int64, c_int64, c_int, c_int, c_void_p, c_int, c_int, c_float, c_void_p, c_int,
         c_void_p, c_int, c_void_p],
    ),
    "solort_paged_kv_store": (
        c_int,
        [c_void_p, c_void_p, c_int64, c_int64, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_int64, c_int64,
         c_int64, c_int, c_int, c_void_p],
    ),
    "solort_paged_kv_gather": (
        c_int,
        [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int, c_int, c_void_p, c_int, c_int, c_int, c_void_p,
         c_void_p, c_int64, c_int64, c_void_p],
    ),
    "solort_prefill_layer": (
        c_int,
        [c_void_p, c_int64, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_float, c_void_p, c_void_p, c_void_p,
         c_int64, c_int64, c_int64, c_float, c_void_p, c_int, c_void_p],
    ),
    "solort_accept_prefix": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p]),
    "solort_gemv": (
        c_int,
        [c_void_p, c_int64, c_int, c_int, c_void_p, c_void_p, c_float, c_void_p, c_int, c_int64, c_void_p, c_void_p],
    ),
    "solort_gemv_argmax_workspace_bytes": (c_size_t, [c_int]),
    "solort_gemv_argmax": (
        c_int, [c_void_p, c_int64, c_int, c_int, c_void_p, c_void_p, c_float, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "solort_greedy_advance": (
        c_int, [c_void_p, c_int, c_void_p, c_int64, c_int, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p,
                c_void_p],
    ),
    "solort_argmax_workspace_bytes": (c_size_t, [c_int]),
    "solort_argmax_rows": (
        c_int, [c_void_p, c_int, c_int, c_int64, c_int64, c_void_p, c_void_p, c_void_p]
    ),
}

_lib: ctypes.CDLL | None = None
_init_devices: set[int] = set()


def _source_id() -> int | None:
    """The hash the build compiles into the library, over the sources present next to this
    package (None when they are not shipped)."""
    from . import build
    if not build.CSRC.is_dir():
        return None
    return build.source_id()


def _init_device(lib: ctypes.CDLL) -> None:
    """solort_init once per device, outside graph capture (it synchronises): checks the
    workgroup placement the in-launch split merge relies on."""
    if not torch.cuda.is_available():
        return
    dev = torch.cuda.current_device()
    if dev in _init_devices or torch.cuda.is_current_stream_capturing():
        return
    rc = lib.solort_init()
    if rc != 0:
        raise RuntimeError(f"solort_init failed ({rc}): {lib.solort_last_error().decode(errors='replace')}")
    _init_devices.add(dev)


# Phase-stamp readers of the tracing build (include/solort_trace.h).
TRACE_SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "solort_phase_stamps_decode": (c_int, [c_void_p, c_int]),
    "solort_phase_stamps_prefill": (c_int, [c_void_p, c_int]),
}


def use_stamp_build() -> None:
    """Makes load() bind the tracing build (libsolort_hip_stamps.so: the same kernels with phase
    stamps, python -m solort_amd.build --stamps) instead of the normal library.  Call before the
    first load()."""
    global LIB_PATH
    if _lib is not None:
        raise RuntimeError("use_stamp_build() must come before the library is loaded")
    LIB_PATH = Path(__file__).resolve().parent / "libsolort_hip_stamps.so"
    SIGNATURES.update(TRACE_SIGNATURES)


def load() -> ctypes.CDLL:
    """Loads (once) and returns the library, initialised for the current device; raises
    RuntimeError if it is missing, of another ABI, or built from other sources."""
    global _lib
    if _lib is not None:
        if torch.cuda.is_available() and torch.cuda.current_device() not in _init_devices:
            _init_device(_lib)
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python -m solort_amd.build"
            f"{' --stamps' if 'stamps' in LIB_PATH.name else ''}` (hipcc, gfx950)"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    ver = lib.solort_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH} has ABI {ver}, expected {ABI_VERSION}; rebuild it")
    sid = _source_id()
    if sid is not None and lib.solort_source_id() != sid:
        raise RuntimeError(f"{LIB_PATH} was built from other sources than those in {LIB_PATH.parent / 'csrc'}; "
                           "rebuild it (python -m solort_amd.build)")
    _init_device(lib)
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    """Raises RuntimeError with the library's message when rc != 0."""
    if rc != 0:
        msg = load().solort_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")
