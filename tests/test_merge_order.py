"""The split-K hand-off in the built code (no GPU needed).

The decode kernel's partition merge and the prefill kernel's key-split
merge hand partial rows from one work group to another within a launch
without a cache writeback: every partial is stored with a device-coherent
(agent-scope, `sc1`) store, each wave waits for its stores' acknowledgement
(`s_waitcnt vmcnt(0)`), the work group meets at a barrier, and only then
does one thread count the group on the unit's counter (`global_atomic_add`,
relaxed, agent scope). The group that completes the count reads the
partials with device-coherent (`sc1`) loads. The source states that order
with relaxed atomics and an explicit wait, which the compiler is free to
move; this test compiles the two kernel sources for gfx950 and checks the
order in their AMD assembly, for every kernel instantiation that has a
merge, so a compiler change that reorders the hand-off fails here instead
of in a rare wrong row.
"""

import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mini-vllm-continuous-batching-lab_amd")
sys.path.insert(0, PKG)

import build_lib  # noqa: E402


def _hipcc():
    try:
        return build_lib.hipcc()
    except RuntimeError:
        return None


def device_asm(src, tmp_path):
    flags = [f for f in build_lib.HIPCC_FLAGS if f not in ("-shared", "-fPIC")]
    out = tmp_path / (src + ".s")
    cmd = [_hipcc(), *flags, "--cuda-device-only", "-S", "-I", build_lib.INCLUDE, "-I",
           build_lib.CSRC, os.path.join(build_lib.CSRC, src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    assert proc.returncode == 0, proc.stderr[-2000:]
    return out.read_text()


def kernels(asm, name_part):
    """{symbol: [instruction lines]} of the kernels whose symbol contains
    ``name_part``."""
    out = {}
    cur = None
    for line in asm.splitlines():
        m = re.match(r"^(_Z\S+):", line)
        if m:
            cur = m.group(1) if name_part in m.group(1) else None
            if cur:
                out[cur] = []
            continue
        if cur is None:
            continue
        if line.startswith("\t.end_amdhsa_kernel") or line.startswith(".Lfunc_end"):
            cur = None
            continue
        ins = line.split(";")[0].strip()
        if ins and not ins.startswith(".") and not ins.endswith(":"):
            out[cur].append(ins)
    return out


def check_handoff(name, ins):
    atomics = [i for i, x in enumerate(ins) if x.startswith("global_atomic_add")]
    assert len(atomics) == 1, (name, [ins[i] for i in atomics])
    a = atomics[0]
    stores = [i for i in range(a) if ins[i].startswith("global_store") and ins[i].endswith(" sc1")]
    assert stores, (name, "no device-coherent partial store before the counter atomic")
    last = stores[-1]
    between = ins[last + 1:a]
    waits = [k for k, x in enumerate(between) if re.match(r"s_waitcnt\b.*\bvmcnt\(0\)", x)]
    assert waits, (name, "no vmcnt(0) between the partial stores and the counter atomic")
    assert any(x == "s_barrier" for x in between[waits[0]:]), (
        name, "no barrier after the stores' acknowledgement, before the counter atomic")
    # nothing the merger reads is a plain (possibly stale) load
    loads = [x for x in ins[a + 1:] if x.startswith("global_load")]
    assert loads, (name, "no merge loads after the counter atomic")
    plain = [x for x in loads if not x.endswith(" sc1")]
    assert not plain, (name, plain[:4])
    # the hand-off needs no cache writeback or invalidate anywhere
    assert not [x for x in ins if x.startswith(("buffer_wbl2", "buffer_inv"))], name


@pytest.mark.skipif(_hipcc() is None, reason="hipcc not installed")
@pytest.mark.parametrize("src,kernel,count", [
    # decode: 3 dtypes x 2 head dims x (plain, fused write, fused RoPE +
    # write), plus the three-stage forms of the 16-bit head_dim-64 kernels
    ("paged_decode.hip", "paged_decode_kernel", 24),
    ("paged_prefill.hip", "paged_prefill_kernel", 12),
])
def test_partials_are_published_before_the_counter(src, kernel, count, tmp_path):
    ks = kernels(device_asm(src, tmp_path), kernel)
    assert len(ks) == count, sorted(ks)
    for name, ins in ks.items():
        check_handoff(name, ins)


def test_checker_rejects_a_missing_wait():
    """The checker itself: an atomic right after the stores, or a plain
    merge load, fails it."""
    good = ["global_store_dword v[4:5], v10, off sc1", "s_waitcnt vmcnt(0)", "s_barrier",
            "global_atomic_add v2, v2, v3, s[20:21] sc0", "global_load_dwordx2 v[6:7], v[4:5], off sc1"]
    check_handoff("good", good)
    with pytest.raises(AssertionError, match="vmcnt"):
        check_handoff("no wait", [good[0], good[2], good[3], good[4]])
    with pytest.raises(AssertionError, match="barrier"):
        check_handoff("no barrier", [good[0], good[1], good[3], good[4]])
    with pytest.raises(AssertionError):
        check_handoff("plain load", good[:4] + ["global_load_dwordx2 v[6:7], v[4:5], off"])
