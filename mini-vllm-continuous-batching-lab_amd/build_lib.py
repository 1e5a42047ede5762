"""Builds libmvattn.so (the C-ABI paged-attention library) for gfx950.

Usage: ``python build_lib.py`` (or ``build()`` from Python). The library
lands in ``lib/libmvattn.so`` next to this file, where
``mini_vllm.attention._hip`` loads it.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
LIB_DIR = os.path.join(HERE, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libmvattn.so")

SOURCES = ("mv_error.hip", "kv_cache_write.hip", "paged_decode.hip", "gather_paged_kv.hip",
           "rope_kv_write.hip", "paged_prefill.hip")

# gfx950 only. Packed-fp32 VALU ops are disabled: hipcc must not emit
# v_pk_{add,mul,fma}_f32 (their results are not trusted on this hardware).
HIPCC_FLAGS = (
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
)


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    if os.path.exists(path):
        return path
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def build(verbose: bool = False) -> str:
    """Compile every source into lib/libmvattn.so; returns the library path."""
    os.makedirs(LIB_DIR, exist_ok=True)
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    # Build to a temporary name, then rename: a process that already mapped
    # the old library keeps a consistent file.
    fd, tmp = tempfile.mkstemp(prefix="libmvattn.", suffix=".so.tmp", dir=LIB_DIR)
    os.close(fd)
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", INCLUDE, "-I", CSRC, *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the packed-fp32 feature and says so; that
    # warning is expected and filtered out.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        os.unlink(tmp)
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
