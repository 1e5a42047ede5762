"""Every HIP kernel compiles for gfx950 without scratch (register spills to
memory): a spill in the decode or prefill loop costs more than the tile it
serves. Compiles each kernel source with the library's flags and reads the
compiler's resource report; no GPU needed."""

import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mini-vllm-continuous-batching-lab_amd")
sys.path.insert(0, PKG)

import build_lib  # noqa: E402

KERNEL_SOURCES = [s for s in build_lib.SOURCES if s != "mv_error.hip"]


def _hipcc():
    try:
        return build_lib.hipcc()
    except RuntimeError:
        return None


@pytest.mark.skipif(_hipcc() is None, reason="hipcc not installed")
@pytest.mark.parametrize("src", KERNEL_SOURCES)
def test_no_scratch(src, tmp_path):
    flags = [f for f in build_lib.HIPCC_FLAGS if f != "-shared"]
    cmd = [_hipcc(), *flags, "-c", "-I", build_lib.INCLUDE, "-I", build_lib.CSRC,
           os.path.join(build_lib.CSRC, src),
           "-o", str(tmp_path / "k.o"), "-Rpass-analysis=kernel-resource-usage"]
    out = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stderr[-2000:]
    names = re.findall(r"Function Name: (\S+)", out.stderr)
    scratch = [int(x) for x in re.findall(r"ScratchSize \[bytes/lane\]: (\d+)", out.stderr)]
    assert names and len(names) == len(scratch), out.stderr[-2000:]
    spilled = [(n, s) for n, s in zip(names, scratch) if s]
    assert not spilled, spilled
