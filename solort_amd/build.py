"""Builds libsolort_hip.so (the gfx950 kernels + C ABI) in-tree with hipcc.

Every HIP source under csrc/ is compiled for gfx950 only and linked into one
shared library next to this file.  Usage: ``python -m solort_amd.build
[--reuse] [--stamps]`` (--stamps: the tracing build, libsolort_hip_stamps.so).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB_NAME = "libsolort_hip.so"
LIB_PATH = PKG / LIB_NAME
OBJ_DIR = PKG / "_build"
# The tracing build (phase stamps in the decode and prefill kernels, include/solort_trace.h).
STAMPS_LIB_PATH = PKG / "libsolort_hip_stamps.so"
STAMPS_OBJ_DIR = PKG / "_build_stamps"

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed fp32 instructions are disabled for all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Leading scalar/pointer kernel arguments arrive preloaded in SGPRs, so a
    # kernel's first loads do not wait for the kernel-argument fetch.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def source_id() -> int:
    """64-bit hash of every source the library is built from (csrc/*.hip, csrc/*.h,
    include/*.h): compiled into the library and compared by the loader, which refuses
    a library built from other sources."""
    import hashlib
    h = hashlib.sha256()
    files = sorted([*CSRC.glob("*.hip"), *CSRC.glob("*.h"), *(PKG.parent / "include").glob("*.h")])
    for f in files:
        h.update(f.name.encode())
        h.update(b"\0")
        h.update(f.read_bytes())
        h.update(b"\0")
    return int.from_bytes(h.digest()[:8], "little")


# Per-source extra flags.  prefill.hip: MFMA results stay in architectural
# VGPRs, where the softmax reads and rescales them, instead of AGPRs that
# every VALU access would first have to copy out.
EXTRA_FLAGS = {"prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src: Path, sid: int, reuse: bool = False, stamps: bool = False) -> Path:
    """Compiles one source; with `reuse`, an object whose recorded compile command and
    inputs (the source, every csrc/ and include/ header) are unchanged is kept."""
    import hashlib
    obj = (STAMPS_OBJ_DIR if stamps else OBJ_DIR) / (src.stem + ".o")
    # Only capi.hip reports the source id; other objects do not depend on it.
    sid_flag = [f"-DSOLORT_SOURCE_ID={sid}ULL"] if src.name == "capi.hip" else []
    stamp_flag = ["-DSOLORT_PHASE_STAMPS"] if stamps else []
    cmd = [hipcc(), *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), *sid_flag, *stamp_flag, "-I",
           str(PKG.parent / "include"), "-c", str(src), "-o", str(obj)]
    h = hashlib.sha256("\0".join(cmd).encode())
    for f in [src, *sorted(CSRC.glob("*.h")), *sorted((PKG.parent / "include").glob("*.h"))]:
        h.update(f.read_bytes())
    stamp = obj.with_suffix(".stamp")
    if reuse and obj.exists() and stamp.exists() and stamp.read_text() == h.hexdigest():
        return obj
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    stamp.write_text(h.hexdigest())
    return obj


def build(verbose: bool = False, reuse: bool = False, stamps: bool = False) -> Path:
    """Compiles every csrc/*.hip for gfx950 and links LIB_PATH (with `stamps`, the tracing build
    STAMPS_LIB_PATH); returns its path.  With `reuse`, objects whose inputs and compile command are
    unchanged are not compiled again."""
    lib_path = STAMPS_LIB_PATH if stamps else LIB_PATH
    (STAMPS_OBJ_DIR if stamps else OBJ_DIR).mkdir(exist_ok=True)
    srcs = sources()
    jobs = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    sid = source_id()
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda f: _compile(f, sid, reuse, stamps), srcs))
    tmp = lib_path.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, lib_path)
    if verbose:
        print(f"built {lib_path} from {len(srcs)} sources")
    return lib_path


if __name__ == "__main__":
    build(verbose=True, reuse="--reuse" in sys.argv, stamps="--stamps" in sys.argv)
    sys.exit(0)
