"""Builds libmvattn.so (the C-ABI paged-attention library) for gfx950.

Usage: ``python build_lib.py`` (or ``build()`` from Python). The library
lands in ``lib/libmvattn.so`` next to this file, where
``mini_vllm.attention._hip`` loads it. A measurement variant builds
elsewhere: ``python build_lib.py --define MV_DECODE_QK_VALU --out
/tmp/libmvattn_valu.so``, loaded with ``MVATTN_LIB=/tmp/libmvattn_valu.so``.
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


# Build-time variants (``--define NAME``), each measured against the default:
#   MV_DECODE_QK_VALU  the decode's K Q^T on VALU dot products instead of MFMA
VARIANT_DEFINES = ("MV_DECODE_QK_VALU",)


def build(verbose: bool = False, defines=(), out: str = LIB_PATH) -> str:
    """Compile every source into ``out`` (default lib/libmvattn.so); returns
    its path. ``defines``: names from ``VARIANT_DEFINES``; a variant library
    is loaded through ``MVATTN_LIB``."""
    for d in defines:
        if d not in VARIANT_DEFINES:
            raise ValueError(f"unknown build variant {d!r} (known: {', '.join(VARIANT_DEFINES)})")
    out_dir = os.path.dirname(os.path.abspath(out))
    os.makedirs(out_dir, exist_ok=True)
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    # Build to a temporary name, then rename: a process that already mapped
    # the old library keeps a consistent file.
    fd, tmp = tempfile.mkstemp(prefix="libmvattn.", suffix=".so.tmp", dir=out_dir)
    os.close(fd)
    cmd = [hipcc(), *HIPCC_FLAGS, *(f"-D{d}" for d in defines), "-I", INCLUDE, "-I", CSRC,
           *srcs, "-o", tmp]
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
    os.replace(tmp, out)
    return out


LAUNCHER_SOURCE = os.path.join(CSRC, "py_launch.c")
LAUNCHER_DIR = os.path.join(HERE, "mini_vllm", "attention")


def build_launcher(verbose: bool = False) -> str:
    """Compile the CPython fast-call wrappers (``csrc/py_launch.c``, host C
    only) into ``mini_vllm/attention/_mvlaunch<EXT_SUFFIX>``; returns its
    path. Without it the wrappers call the same entry points through
    ctypes."""
    import sysconfig

    out = os.path.join(LAUNCHER_DIR, "_mvlaunch" + sysconfig.get_config_var("EXT_SUFFIX"))
    cc = shutil.which("gcc") or shutil.which("cc")
    if not cc:
        raise RuntimeError("no C compiler (gcc) for the launcher extension")
    fd, tmp = tempfile.mkstemp(prefix="_mvlaunch.", suffix=".so.tmp", dir=LAUNCHER_DIR)
    os.close(fd)
    cmd = [cc, "-O2", "-shared", "-fPIC", "-Wall", "-Wextra", "-Werror",
           "-I", sysconfig.get_paths()["include"], "-I", INCLUDE, LAUNCHER_SOURCE, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        os.unlink(tmp)
        raise RuntimeError(f"launcher build failed ({proc.returncode}):\n{proc.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    import argparse

    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--define", action="append", default=[], choices=VARIANT_DEFINES,
                    help="build a variant (load it with MVATTN_LIB=<out>)")
    ap.add_argument("--out", default=LIB_PATH)
    args = ap.parse_args()
    if args.define and os.path.abspath(args.out) == LIB_PATH:
        ap.error("a variant needs --out: lib/libmvattn.so is the default build")
    print(build(verbose=True, defines=args.define, out=args.out))
    print(build_launcher(verbose=True))
