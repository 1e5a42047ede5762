"""C-ABI library checks that need no GPU.

* libmvattn.so loads and exports every function include/mvattn.h declares,
  and the ctypes table declares the same parameter count;
* host-side argument checks return the documented codes without touching
  the device.
"""

import ctypes
import os
import re

import pytest
import torch

from mini_vllm.attention import _hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mvattn.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(mv_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        params = m.group(2).strip()
        n = 0 if params in ("", "void") else len(params.split(","))
        out[m.group(1)] = n
    return out


@pytest.fixture(scope="module")
def lib():
    import importlib.util

    launcher = importlib.util.find_spec("mini_vllm.attention._mvlaunch")
    if not os.path.exists(_hip.library_path()) or launcher is None:
        spec = importlib.util.spec_from_file_location(
            "build_lib", os.path.join(ROOT, "mini-vllm-continuous-batching-lab_amd", "build_lib.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        if not os.path.exists(_hip.library_path()):
            mod.build()
        if launcher is None:
            mod.build_launcher()
    return _hip.load()


def test_header_declares_the_path():
    decl = _declared_functions()
    for name in ("mv_kv_cache_write", "mv_kv_slots_check", "mv_decode_plan", "mv_paged_decode",
                 "mv_paged_decode_workspace_bytes", "mv_gather_paged_kv", "mv_last_error"):
        assert name in decl


def test_c_host_compiles_and_links_against_the_header(lib, tmp_path):
    """A plain C99 host (gcc, no HIP headers) that takes the address of
    every function mvattn.h declares and calls the ones that need no
    device: the header stands alone and the library resolves it all."""
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not found")
    decl = _declared_functions()
    src = tmp_path / "host.c"
    src.write_text(
        "#include <stdio.h>\n#include \"mvattn.h\"\n"
        "int main(void) {\n"
        "  void* fns[] = {" + ", ".join(f"(void*){n}" for n in sorted(decl)) + "};\n"
        "  for (unsigned i = 0; i < sizeof fns / sizeof fns[0]; ++i) if (!fns[i]) return 2;\n"
        "  if (mv_abi_version() != MVATTN_ABI_VERSION) return 3;\n"
        "  if (mv_decode_chunk_tokens(64, MV_DTYPE_BF16) != 64) return 4;\n"
        "  if (mv_prefill_tokens_per_group(14, 2, 64, MV_DTYPE_BF16) != 16) return 5;\n"
        "  printf(\"ok %u\\n\", (unsigned)(sizeof fns / sizeof fns[0]));\n"
        "  return 0;\n}\n")
    exe = tmp_path / "host"
    libdir = os.path.dirname(_hip.library_path())
    subprocess.run([gcc, "-std=c99", "-Wall", "-Werror", "-I", os.path.dirname(HEADER), str(src),
                    "-L", libdir, "-lmvattn", f"-Wl,-rpath,{libdir}", "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, (out.returncode, out.stderr)
    assert out.stdout.strip() == f"ok {len(decl)}"


def test_every_declared_symbol_is_exported_and_typed(lib):
    decl = _declared_functions()
    for name, nparams in decl.items():
        assert hasattr(lib, name), f"{name} not exported"
        assert name in _hip.SIGNATURES, f"{name} missing from the ctypes table"
        assert len(_hip.SIGNATURES[name][1]) == nparams, name
    assert set(_hip.SIGNATURES) == set(decl)


def test_abi_queries(lib):
    assert lib.mv_abi_version() == _hip.ABI_VERSION == 7
    assert lib.mv_decode_chunk_tokens(64, 2) == 64       # 4 waves x one 16-token tile
    assert lib.mv_decode_chunk_tokens(128, 0) == 64
    assert lib.mv_decode_chunk_tokens(96, 2) == 0
    assert lib.mv_decode_groups_per_cu(64, 2) == 4       # 2 stages x 4 waves x 4 KiB + 2 KiB ids + 2 KiB Q
    assert lib.mv_decode_groups_per_cu(128, 2) == 2
    assert lib.mv_decode_groups_per_cu(96, 2) == 0


def test_prefill_tokens_per_group(lib):
    """Query tokens one prefill work group covers: 16-bit types at head_dim
    64 run 4 row waves of two 16-row tiles (two wave sets), the others 8
    (4 for fp32 at head_dim 128) of one tile; a wave holds
    floor(rows / n_rep) tokens."""
    f = lib.mv_prefill_tokens_per_group
    assert f(14, 2, 64, 2) == 4 * (32 // 7) == 16    # Qwen2-0.5B, bf16
    assert f(12, 2, 64, 1) == 4 * (32 // 6) == 20    # n_rep 6, fp16: 5 tokens per row wave
    assert f(14, 2, 64, 0) == 8 * (16 // 7) == 16    # fp32: one set
    assert f(28, 4, 128, 2) == 8 * (16 // 7) == 16   # head_dim 128: one set
    assert f(8, 8, 64, 2) == 4 * 32 == 128           # MHA
    assert f(14, 2, 128, 0) == 4 * (16 // 7) == 8    # fp32 at head_dim 128: 4 waves
    assert f(17, 1, 64, 2) == 0                      # more than 16 query heads per kv head
    assert f(14, 3, 64, 2) == 0                      # not a whole GQA group
    assert f(14, 2, 96, 2) == 0                      # head_dim


def test_check_workspace_bytes(lib):
    """The slot check needs no workspace up to 4096 tokens (one work group,
    LDS); above, a hash table of 8-byte words, a power of two at least twice
    the tokens. The fused-write check's writer table likewise, at least 64
    words, and nothing beyond MV_WRITE_CHECK_MAX_SEQS sequences."""
    f = lib.mv_kv_slots_check_workspace_bytes
    assert f(0) == f(1) == f(4096) == 0
    assert f(4097) == 16384 * 8
    assert f(32768) == 65536 * 8
    assert f(32769) == 131072 * 8
    g = lib.mv_decode_write_check_workspace_bytes
    assert g(0) == g(1) == g(32) == 64 * 8
    assert g(33) == 128 * 8
    assert g(4096) == 8192 * 8
    assert g(4097) == 0 and g(-1) == 0


def test_checks_reject_bad_arguments_on_host(lib):
    """Argument checks of the two device checks return before any launch
    (dummy or null pointers: nothing is read)."""
    f = lib.mv_kv_slots_check
    assert f(16, 10, 100, None, None, 0, None) == _hip.MV_ERR_INVALID_ARGUMENT  # null status
    assert f(None, 10, 100, 16, None, 0, None) == _hip.MV_ERR_INVALID_ARGUMENT  # null slots
    assert f(16, -1, 100, 16, None, 0, None) == _hip.MV_ERR_INVALID_ARGUMENT
    assert f(16, 1 << 20, 100, 16, None, 0, None) == _hip.MV_ERR_UNSUPPORTED
    assert f(16, 10, 1 << 44, 16, None, 0, None) == _hip.MV_ERR_UNSUPPORTED
    # above 4096 tokens the workspace is required, and its size checked
    need = lib.mv_kv_slots_check_workspace_bytes(5000)
    assert f(16, 5000, 100, 16, None, 0, None) == _hip.MV_ERR_INVALID_ARGUMENT
    assert b"workspace" in lib.mv_last_error()
    assert f(16, 5000, 100, 16, 64, need - 8, None) == _hip.MV_ERR_INVALID_ARGUMENT
    assert f(16, 5000, 100, 16, 68, need, None) == _hip.MV_ERR_INVALID_ARGUMENT  # misaligned
    assert b"aligned" in lib.mv_last_error()

    g = lib.mv_decode_write_check
    need = lib.mv_decode_write_check_workspace_bytes(4)
    assert g(16, 16, 1, 8, 16, 1, 4, 8, 16, None, 64, need, None) == _hip.MV_ERR_INVALID_ARGUMENT
    assert g(16, 16, 1, 8, 16, 1, 4097, 8, 16, 16, 64, 1 << 20, None) == _hip.MV_ERR_UNSUPPORTED
    assert g(16, 16, 1, 8, 16, 1, 4, 8, 12, 16, 64, need, None) == _hip.MV_ERR_UNSUPPORTED
    assert g(16, 16, 1, 8, 16, 1, 4, 8, 1 << 21, 16, 64, need, None) == _hip.MV_ERR_UNSUPPORTED
    assert g(None, 16, 1, 8, 16, 1, 4, 8, 16, 16, 64, need, None) == _hip.MV_ERR_INVALID_ARGUMENT
    assert g(16, 16, 1, 8, 16, 1, 4, 8, 16, 16, None, need, None) == _hip.MV_ERR_INVALID_ARGUMENT
    assert g(16, 16, 1, 8, 16, 1, 4, 8, 16, 16, 64, need - 8, None) == _hip.MV_ERR_INVALID_ARGUMENT
    assert b"workspace" in lib.mv_last_error()


def test_step_check_rejects_bad_arguments_on_host(lib):
    f = lib.mv_decode_step_check
    need = lib.mv_decode_write_check_workspace_bytes(4)

    def call(**kw):
        a = dict(slots=16, bt=16, bt64=1, bts=8, kv=16, kv64=1, n=4, mb=8, bs=16, nb=100,
                 pos=None, cos=None, sin=None, tstride=0, maxpos=0, d=64, dt=2, rc=None, rs=None,
                 st=16, ws=64, wsb=need, stream=None)
        a.update(kw)
        return f(*a.values())

    assert call(st=None) == _hip.MV_ERR_INVALID_ARGUMENT
    assert call(n=4097) == _hip.MV_ERR_UNSUPPORTED
    assert call(bs=12) == _hip.MV_ERR_UNSUPPORTED
    assert call(nb=1 << 41) == _hip.MV_ERR_UNSUPPORTED  # 2^45 slots
    assert call(slots=None) == _hip.MV_ERR_INVALID_ARGUMENT
    assert call(ws=None) == _hip.MV_ERR_INVALID_ARGUMENT
    assert call(wsb=need - 8) == _hip.MV_ERR_INVALID_ARGUMENT
    # positions need the tables, rows, a dtype and whole 16-byte rows, aligned
    assert call(pos=16) == _hip.MV_ERR_INVALID_ARGUMENT
    full = dict(pos=16, cos=64, sin=128, tstride=64, maxpos=100, rc=256, rs=512)
    assert call(**{**full, "d": 4, "dt": 2}) == _hip.MV_ERR_INVALID_ARGUMENT  # 8-byte rows
    assert call(**{**full, "cos": 72}) == _hip.MV_ERR_INVALID_ARGUMENT      # misaligned table
    assert b"aligned" in lib.mv_last_error()
    assert call(**{**full, "tstride": 32}) == _hip.MV_ERR_INVALID_ARGUMENT  # stride < head_dim
    assert call(**{**full, "dt": 9}) == _hip.MV_ERR_INVALID_ARGUMENT


def test_workspace_bytes(lib):
    assert lib.mv_paged_decode_workspace_bytes(64, 14, 64, 1) == 0
    o = 64 * 14 * 8 * 64 * 4
    assert lib.mv_paged_decode_workspace_bytes(64, 14, 64, 8) == -(-o // 256) * 256 + 64 * 14 * 8 * 8


DECODE_PARAMS = [
    "query", "q_stride_tok", "q_stride_head", "key_cache", "value_cache", "work_items",
    "block_ids", "block_ids_capacity", "num_work_groups", "partition_tokens",
    "max_partitions", "counters", "out", "out_stride_tok", "out_stride_head", "scale",
    "num_seqs", "num_q_heads", "num_kv_heads", "head_dim", "block_size", "num_blocks", "dtype",
    "workspace", "workspace_bytes", "stream",
]


def _decode_args(**kw):
    base = dict(query=None, q_stride_tok=0, q_stride_head=0, key_cache=None, value_cache=None,
                work_items=None, block_ids=None, block_ids_capacity=1024,
                num_work_groups=1, partition_tokens=64, max_partitions=1, counters=None, out=None,
                out_stride_tok=0, out_stride_head=0, scale=0.125, num_seqs=1, num_q_heads=14,
                num_kv_heads=2, head_dim=64, block_size=16, num_blocks=10, dtype=2,
                workspace=None, workspace_bytes=0, stream=None)
    base.update(kw)
    return [base[k] for k in DECODE_PARAMS]


def test_block_ids_capacity(lib):
    # kv_heads * num_seqs * (max_blocks + 512 + 16) + 5 * work_capacity (a bound for any piece size)
    assert lib.mv_decode_block_ids_capacity(64, 128, 2, 4096) == 2 * 64 * (128 + 512 + 16) + 5 * 4096
    assert lib.mv_decode_block_ids_capacity(0, 0, 2, 0) == 0
    assert lib.mv_decode_block_ids_capacity(-1, 4, 2, 4) == 0


def test_plan_rejects_small_block_ids_buffer_on_host(lib):
    # dummy addresses: the call fails on the capacity before anything is launched
    rc = lib.mv_decode_plan(16, 1, 16, 1, 8, 4, 8, 16, 100, 2, 3, 256, 0,
                            16, 8, 16, 10, 16, 16, None)
    assert rc == _hip.MV_ERR_INVALID_ARGUMENT
    assert b"block_ids capacity" in lib.mv_last_error()


def test_graph_bounds(lib):
    import ctypes
    out = (ctypes.c_int64 * 3)()
    # c2-like: 64 sequences x 128 entries of 16 tokens, 2 kv heads, 3 groups/CU, 256 CUs
    assert lib.mv_decode_graph_bounds(64, 128, 16, 2, 3, 256, out) == 0
    groups, part, parts = list(out)
    assert part == 511 * 16  # the widest piece: 511 table entries
    assert parts == 128 // 4  # pieces of at least 4 tiles
    # units + max(resident target, units * tiles / widest piece), capped by units * parts;
    # 128 units fit 256 CUs, so the plan aims at 2 groups per CU
    assert groups == min(128 + max(2 * 256, -(-128 * 128 // 511)), 128 * parts)
    # more units than CUs: all 3 slots per CU
    assert lib.mv_decode_graph_bounds(256, 128, 16, 2, 3, 256, out) == 0
    assert list(out)[0] == min(512 + max(3 * 256, -(-512 * 128 // 511)), 512 * 32)
    # tiny tables: at most one piece per sequence
    assert lib.mv_decode_graph_bounds(10, 2, 16, 2, 3, 256, out) == 0
    assert list(out)[0] == 20 and list(out)[2] == 1
    assert lib.mv_decode_graph_bounds(4, 8, 12, 2, 3, 256, out) == _hip.MV_ERR_UNSUPPORTED
    assert lib.mv_decode_graph_bounds(0, 8, 16, 2, 3, 256, out) == _hip.MV_ERR_INVALID_ARGUMENT


def test_decode_param_list_matches_header():
    assert len(DECODE_PARAMS) == len(_hip.SIGNATURES["mv_paged_decode"][1])


def test_decode_rejects_unsupported_shapes_on_host(lib):
    """Argument checks return before any device work (null pointers are fine)."""
    assert lib.mv_paged_decode(*_decode_args(head_dim=96)) == _hip.MV_ERR_UNSUPPORTED
    assert b"head_dim 96" in lib.mv_last_error()
    assert lib.mv_paged_decode(*_decode_args(block_size=12)) == _hip.MV_ERR_UNSUPPORTED
    assert lib.mv_paged_decode(*_decode_args(num_kv_heads=3)) == _hip.MV_ERR_INVALID_ARGUMENT
    assert lib.mv_paged_decode(*_decode_args(num_q_heads=34)) == _hip.MV_ERR_UNSUPPORTED
    assert lib.mv_paged_decode(*_decode_args(dtype=7)) == _hip.MV_ERR_UNSUPPORTED
    assert lib.mv_paged_decode(*_decode_args(partition_tokens=100)) == _hip.MV_ERR_INVALID_ARGUMENT
    # a partition's block ids are staged in LDS: at most 511 blocks per partition
    assert lib.mv_paged_decode(*_decode_args(block_size=1, partition_tokens=512)) == \
        _hip.MV_ERR_INVALID_ARGUMENT
    assert b"spans more than 511 blocks" in lib.mv_last_error()
    assert lib.mv_paged_decode(*_decode_args(block_size=1, partition_tokens=448,
                                             num_work_groups=0)) == _hip.MV_OK
    # the block-id lists of the work items must fit the given capacity
    assert lib.mv_paged_decode(*_decode_args(query=16, key_cache=16, value_cache=16, work_items=16,
                                             block_ids=16, out=16, num_work_groups=300,
                                             block_ids_capacity=1000)) == _hip.MV_ERR_INVALID_ARGUMENT
    assert b"exceed capacity" in lib.mv_last_error()
    # nothing to do is not an error
    assert lib.mv_paged_decode(*_decode_args(num_work_groups=0)) == _hip.MV_OK
    # work to do but null pointers
    assert lib.mv_paged_decode(*_decode_args()) == _hip.MV_ERR_INVALID_ARGUMENT


def test_noalloc_rejects_batches_beyond_its_scratch_on_host(lib):
    """mv_paged_decode_noalloc checks the merge's scratch need against its
    static array before any HIP call: 4096 sequences x 32 query heads x 128
    partitions of head_dim 128 are refused with null pointers, no device
    touched."""
    n, hq, d, parts = 4096, 32, 128, 128
    assert lib.mv_paged_decode_workspace_bytes(n, hq, d, parts) > _hip.MV_DECODE_SCRATCH_BYTES
    rc = lib.mv_paged_decode_noalloc(None, 0, 0, None, None, None, None, 0, 1, 64, parts, None,
                                     None, 0, 0, 0.125, n, hq, 2, d, 16, 1, 2, None)
    assert rc == _hip.MV_ERR_INVALID_ARGUMENT
    assert b"static buffer" in lib.mv_last_error()
    assert lib.mv_paged_decode_noalloc(None, 0, 0, None, None, None, None, 0, 1, 64, 1, None,
                                       None, 0, 0, 0.125, -1, hq, 2, d, 16, 1, 2, None) \
        == _hip.MV_ERR_INVALID_ARGUMENT


def test_write_rejects_bad_sizes_on_host(lib):
    rc = lib.mv_kv_cache_write(None, 0, 0, None, 0, 0, None, None, None,
                               4, 0, 64, 16, 10, 2, None)
    assert rc == _hip.MV_ERR_INVALID_ARGUMENT
    # zero tokens is a no-op, not an error
    assert lib.mv_kv_cache_write(None, 0, 0, None, 0, 0, None, None, None,
                                 0, 2, 64, 16, 10, 2, None) == _hip.MV_OK


def test_check_maps_codes_to_exceptions(lib):
    with pytest.raises(RuntimeError):
        _hip.check(_hip.MV_ERR_UNSUPPORTED, "x")
    with pytest.raises(ValueError):
        _hip.check(_hip.MV_ERR_INVALID_ARGUMENT, "x")
    with pytest.raises(RuntimeError):
        _hip.check(_hip.MV_ERR_HIP, "x")
    _hip.check(_hip.MV_OK, "x")


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="not found"):
        _hip.load(str(tmp_path / "nope.so"))


def test_fast_call_wrappers_match_the_header(lib):
    """The CPython fast-call wrappers (_mvlaunch) are bound to the loaded
    library, take each entry point's parameter count from the header, and
    turn a wrong count or an out-of-range int32 into a Python error before
    any call."""
    from mini_vllm.attention import _mvlaunch

    declared = _declared_functions()
    assert _hip.decode_write is _mvlaunch.decode_write
    assert _hip.decode is _mvlaunch.decode
    assert _hip.cache_write is _mvlaunch.cache_write
    assert _hip.rope_write is _mvlaunch.rope_write
    assert _hip.plan is _mvlaunch.plan
    for fn, name in ((_mvlaunch.decode_write, "mv_paged_decode_write"),
                     (_mvlaunch.decode, "mv_paged_decode"),
                     (_mvlaunch.cache_write, "mv_kv_cache_write"),
                     (_mvlaunch.rope_write, "mv_rope_kv_cache_write"),
                     (_mvlaunch.plan, "mv_decode_plan")):
        n = declared[name]
        with pytest.raises(TypeError, match=f"takes {n} arguments"):
            fn(*([0] * (n - 1)))
    # built against this header's ABI
    assert _mvlaunch.ABI == _hip.ABI_VERSION == lib.mv_abi_version()
    # num_kv_heads (argument 10 of mv_kv_cache_write) beyond int32
    args = [None, 0, 0, None, 0, 0, None, None, None, 0, 1 << 40, 64, 16, 1, 0, None]
    with pytest.raises(OverflowError):
        _mvlaunch.cache_write(*args)


def test_step_words_reach_the_entry_point_in_order(lib):
    """decode_write_step (a step's packed words plus one layer's tensors)
    calls mv_paged_decode_write with exactly the arguments the 35-argument
    fast call passes: the entry point is replaced by a ctypes stand-in of
    the header's signature that records what it receives (no GPU)."""
    from mini_vllm.attention import _mvlaunch

    assert _mvlaunch.STEP_WORDS == _hip.STEP_WORDS
    restype, argtypes = _hip.SIGNATURES["mv_paged_decode_write"]
    seen = []

    def record(*args):
        seen.append(args)
        return 7

    stand_in = ctypes.CFUNCTYPE(restype, *argtypes)(record)
    others = [ctypes.cast(getattr(lib, name), ctypes.c_void_p).value
              for name in ("mv_paged_decode", "mv_kv_cache_write", "mv_rope_kv_cache_write",
                           "mv_decode_plan")]
    step = dict(slots=0x1000, rope_cos=0x2000, rope_sin=None, work=0x3000, ids=0x4000, ids_cap=516,
                groups=510, part_tokens=288, max_parts=8, counters=0x5000, scale=0.125,
                num_seqs=64, hq=14, hkv=2, head_dim=64, block_size=16, num_blocks=9000,
                dtype_code=_hip.MV_DTYPE[torch.bfloat16], ws=0x6000, ws_bytes=1 << 20)
    layer = (0x10, 896, 64, 0x20, 128, 64, 0x30, 256, 64, 0x40, 0x50, 0x60, 896, 64, 0x70)
    try:
        _mvlaunch.bind(ctypes.cast(stand_in, ctypes.c_void_p).value, *others)
        words = _hip.step_words(**step)
        assert len(words) == 8 * _hip.STEP_WORDS
        assert _mvlaunch.decode_write_step(words, *layer) == 7
        full = [0x10, 896, 64, 0x20, 128, 64, 0x30, 256, 64, 0x1000, 0x2000, None, 0x40, 0x50,
                0x3000, 0x4000, 516, 510, 288, 8, 0x5000, 0x60, 896, 64, 0.125, 64, 14, 2, 64, 16,
                9000, _hip.MV_DTYPE[torch.bfloat16], 0x6000, 1 << 20, 0x70]
        assert _mvlaunch.decode_write(*full) == 7
        assert len(seen) == 2 and seen[0] == seen[1]
        # a step of the wrong size, or a 32-bit word out of range, is refused
        with pytest.raises(TypeError, match="STEP_WORDS"):
            _mvlaunch.decode_write_step(words[:-8], *layer)
        with pytest.raises(OverflowError, match="step word 12"):
            _mvlaunch.decode_write_step(_hip.step_words(**{**step, "hq": 1 << 33}), *layer)
        with pytest.raises(TypeError, match="takes 16 arguments"):
            _mvlaunch.decode_write_step(words, *layer[:-1])
        assert len(seen) == 2
    finally:
        _hip._bind_calls(lib)
    assert _hip.decode_write is _mvlaunch.decode_write
    assert _hip.decode_write_step is _mvlaunch.decode_write_step
