"""ctypes binding of libmvattn.so (declarations: include/mvattn.h).

``torch`` is imported first on purpose: torch ships its own
``libamdhip64.so.7``; loading the kernel library afterwards makes the
dynamic linker resolve its HIP dependency to that already-loaded runtime,
so torch tensors, streams and our kernels share one HIP runtime.
"""

from __future__ import annotations

import ctypes
import os
import struct
import threading
import warnings

import torch  # noqa: F401  (must be loaded before the kernel library)

ABI_VERSION = 7

MV_OK = 0
MV_ERR_INVALID_ARGUMENT = -1
MV_ERR_UNSUPPORTED = -2
MV_ERR_HIP = -3

MV_DTYPE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

# status words (mvattn.h)
MV_SLOTS_OUT_OF_RANGE = 0
MV_SLOTS_DUPLICATES = 1
MV_WRITE_CHECK_OWN_SLOT = 0
MV_WRITE_CHECK_SHARED = 1
MV_WRITE_CHECK_MAX_SEQS = 4096
MV_STEP_SLOTS_OUT_OF_RANGE = 0
MV_STEP_SLOTS_DUPLICATES = 1
MV_STEP_WRITE_OWN_SLOT = 2
MV_STEP_WRITE_SHARED = 3
MV_STEP_POSITIONS = 4
MV_STEP_WORDS = 8
MV_PLAN_NUM_ITEMS = 0
MV_PLAN_BAD_KV_LEN = 1
MV_PLAN_INSUFFICIENT = 2
MV_PLAN_BAD_BLOCK = 3
MV_PLAN_MAX_PARTS = 4
MV_PLAN_MIN_KV_LEN = 5
MV_PLAN_PARTITION_TOKENS = 6
MV_PLAN_IDS_PER_ITEM = 7
MV_PLAN_WORDS = 8
MV_DECODE_SCRATCH_BYTES = 16 << 20

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
DEFAULT_LIB_PATH = os.path.join(_PKG_ROOT, "lib", "libmvattn.so")

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t
_F = ctypes.c_float

# name -> (restype, argtypes); must match include/mvattn.h.
SIGNATURES = {
    "mv_abi_version": (ctypes.c_int, []),
    "mv_last_error": (ctypes.c_char_p, []),
    "mv_stream_capture_id": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_uint64)]),
    "mv_decode_chunk_tokens": (ctypes.c_int, [_I32, _I32]),
    "mv_decode_groups_per_cu": (ctypes.c_int, [_I32, _I32]),
    "mv_kv_cache_write": (ctypes.c_int, [
        _P, _I64, _I64,            # key, strides
        _P, _I64, _I64,            # value, strides
        _P, _P, _P,                # key_cache, value_cache, slot_mapping
        _I64, _I32, _I32, _I32,    # num_tokens, num_kv_heads, head_dim, block_size
        _I64, _I32, _P,            # num_blocks, dtype, stream
    ]),
    "mv_kv_slots_check_workspace_bytes": (_SZ, [_I64]),
    "mv_kv_slots_check": (ctypes.c_int, [_P, _I64, _I64, _P, _P, _SZ, _P]),
    "mv_decode_write_check_workspace_bytes": (_SZ, [_I32]),
    "mv_decode_write_check": (ctypes.c_int, [
        _P, _P, _I32, _I64,        # slot_mapping, block_table, bt_is_i64, bt_stride
        _P, _I32, _I32, _I32,      # kv_len, kv_len_is_i64, num_seqs, max_blocks
        _I32, _P, _P, _SZ, _P,     # block_size, status, workspace, workspace_bytes, stream
    ]),
    "mv_decode_step_check": (ctypes.c_int, [
        _P, _P, _I32, _I64,        # slot_mapping, block_table, bt_is_i64, bt_stride
        _P, _I32, _I32, _I32,      # kv_len, kv_len_is_i64, num_seqs, max_blocks
        _I32, _I64,                # block_size, num_blocks
        _P, _P, _P, _I64, _I64,    # positions, cos, sin, table_stride, max_positions
        _I32, _I32, _P, _P,        # head_dim, dtype, cos_rows, sin_rows
        _P, _P, _SZ, _P,           # status, workspace, workspace_bytes, stream
    ]),
    "mv_decode_plan": (ctypes.c_int, [
        _P, _I32, _P, _I32, _I64,  # kv_len, is_i64, block_table, is_i64, bt_stride
        _I32, _I32, _I32, _I64,    # num_seqs, max_blocks, block_size, num_blocks
        _I32, _I32, _I32, _I32,    # num_kv_heads, groups_per_cu, cu_count, fixed_partition_tokens
        _P, _I64, _P, _I64,        # work_items, capacity, block_ids, capacity
        _P, _P, _P,                # counters, status, stream
    ]),
    "mv_decode_plan_step_check": (ctypes.c_int, [
        _P, _I32, _P, _I32, _I64,  # kv_len, is_i64, block_table, is_i64, bt_stride
        _I32, _I32, _I32, _I64,    # num_seqs, max_blocks, block_size, num_blocks
        _I32, _I32, _I32, _I32,    # num_kv_heads, groups_per_cu, cu_count, fixed_partition_tokens
        _P, _I64, _P, _I64,        # work_items, capacity, block_ids, capacity
        _P, _P, _P,                # counters, status, slot_mapping
        _P, _P, _P, _I64, _I64,    # positions, cos, sin, table_stride, max_positions
        _I32, _I32, _P, _P,        # head_dim, dtype, cos_rows, sin_rows
        _P, _P, _SZ, _P,           # step_status, check_workspace, bytes, stream
    ]),
    "mv_decode_graph_bounds": (ctypes.c_int, [_I32, _I32, _I32, _I32, _I32, _I32, _P]),
    "mv_decode_block_ids_capacity": (_I64, [_I32, _I32, _I32, _I64]),
    "mv_paged_decode_workspace_bytes": (_SZ, [_I32, _I32, _I32, _I32]),
    "mv_paged_decode": (ctypes.c_int, [
        _P, _I64, _I64,            # query, strides
        _P, _P,                    # key_cache, value_cache
        _P, _P, _I64, _I32,        # work_items, block_ids, block_ids_capacity, num_work_groups
        _I32, _I32, _P,            # partition_tokens, max_partitions, counters
        _P, _I64, _I64,            # out, strides
        _F, _I32, _I32, _I32, _I32,  # scale, num_seqs, num_q_heads, num_kv_heads, head_dim
        _I32, _I64, _I32,          # block_size, num_blocks, dtype
        _P, _SZ, _P,               # workspace, workspace_bytes, stream
    ]),
    "mv_paged_decode_noalloc": (ctypes.c_int, [
        _P, _I64, _I64,            # query, strides
        _P, _P,                    # key_cache, value_cache
        _P, _P, _I64, _I32,        # work_items, block_ids, block_ids_capacity, num_work_groups
        _I32, _I32, _P,            # partition_tokens, max_partitions, counters
        _P, _I64, _I64,            # out, strides
        _F, _I32, _I32, _I32, _I32,  # scale, num_seqs, num_q_heads, num_kv_heads, head_dim
        _I32, _I64, _I32, _P,      # block_size, num_blocks, dtype, stream
    ]),
    "mv_gather_paged_kv": (ctypes.c_int, [
        _P, _P, _P, _I32, _I64,    # key_cache, value_cache, block_table, bt_is_i64, bt_stride
        _P, _P, _I32, _I64,        # seq_rows, cu_tokens, num_seqs, total_tokens
        _P, _P, _I32, _I32, _I32,  # out_key, out_value, num_kv_heads, head_dim, block_size
        _I64, _I32, _P,            # num_blocks, dtype, stream
    ]),
    "mv_rope_kv_cache_write": (ctypes.c_int, [
        _P, _I64, _I64,            # query, strides
        _P, _I64, _I64,            # query_out, strides
        _P, _I64, _I64,            # key, strides
        _P, _I64, _I64,            # key_out, strides
        _P, _I64, _I64,            # value, strides
        _P, _P, _P,                # key_cache, value_cache, slot_mapping
        _P, _P, _P, _I64, _I64,    # positions, cos, sin, table_stride, max_positions
        _I64, _I32, _I32, _I32,    # num_tokens, num_q_heads, num_kv_heads, head_dim
        _I32, _I64, _I32, _P,      # block_size, num_blocks, dtype, stream
    ]),
    "mv_positions_check": (ctypes.c_int, [_P, _I64, _I64, _P, _P]),
    "mv_paged_decode_write": (ctypes.c_int, [
        _P, _I64, _I64,            # query, strides
        _P, _I64, _I64,            # new_key, strides
        _P, _I64, _I64,            # new_value, strides
        _P, _P, _P,                # slot_mapping, rope_cos_rows, rope_sin_rows
        _P, _P,                    # key_cache, value_cache
        _P, _P, _I64, _I32,        # work_items, block_ids, block_ids_capacity, num_work_groups
        _I32, _I32, _P,            # partition_tokens, max_partitions, counters
        _P, _I64, _I64,            # out, strides
        _F, _I32, _I32, _I32, _I32,  # scale, num_seqs, num_q_heads, num_kv_heads, head_dim
        _I32, _I64, _I32,          # block_size, num_blocks, dtype
        _P, _SZ, _P,               # workspace, workspace_bytes, stream
    ]),
    "mv_prefill_tokens_per_group": (ctypes.c_int, [_I32, _I32, _I32, _I32]),
    "mv_prefill_plan": (ctypes.c_int, [
        _P, _P, _P, _I32, _I64,    # seq_rows, cached_len, query_len, num_seqs, total_query_rows
        _P, _I32, _I64, _I32, _I32,  # block_table, bt_is_i64, bt_stride, bt_rows, max_blocks
        _I32, _I64, _I32, _I32,    # block_size, num_blocks, tokens_per_group, num_kv_heads
        _P, _P, _I32, _P, _P,      # seqs, work_items, work_capacity, status, stream
    ]),
    "mv_paged_prefill": (ctypes.c_int, [
        _P, _I64, _I64,            # query, strides
        _P, _I64, _I64,            # key, strides
        _P, _I64, _I64,            # value, strides
        _P, _P,                    # key_cache, value_cache
        _P, _I32, _I64,            # block_table, bt_is_i64, bt_stride
        _P, _I32, _P, _I32,        # seqs, num_seqs, work_items, num_work_groups
        _P, _I64, _I64,            # out, strides
        _F, _I32, _I32, _I32,      # scale, num_q_heads, num_kv_heads, head_dim
        _I32, _I64, _I32, _P,      # block_size, num_blocks, dtype, stream
    ]),
    "mv_paged_prefill_workspace_bytes": (ctypes.c_size_t, [_I32, _I32, _I32, _I32, _I32, _I32]),
    "mv_paged_prefill_parts": (ctypes.c_int, [
        _P, _I64, _I64,            # query, strides
        _P, _I64, _I64,            # key, strides
        _P, _I64, _I64,            # value, strides
        _P, _P,                    # key_cache, value_cache
        _P, _I32, _I64,            # block_table, bt_is_i64, bt_stride
        _P, _I32, _P, _I32,        # seqs, num_seqs, work_items (8 ints each), num_work_groups
        _I32, _I32,                # num_units, max_parts
        _P, _I64, _I64,            # out, strides
        _F, _I32, _I32, _I32,      # scale, num_q_heads, num_kv_heads, head_dim
        _I32, _I64, _I32,          # block_size, num_blocks, dtype
        _P, ctypes.c_size_t, _P,   # workspace, workspace_bytes, stream
    ]),
}

_lock = threading.Lock()
_lib = None


def library_path() -> str:
    return os.environ.get("MVATTN_LIB", DEFAULT_LIB_PATH)


# The per-layer entry points as called by the wrappers: the CPython
# fast-call wrappers of _mvlaunch (csrc/py_launch.c, built beside this
# module) when it is present, else the ctypes functions. Same arguments in
# the same order, same status codes; set when the library is loaded.
decode_write = None  # mv_paged_decode_write
decode = None        # mv_paged_decode
cache_write = None   # mv_kv_cache_write
rope_write = None    # mv_rope_kv_cache_write
plan = None          # mv_decode_plan
# mv_paged_decode_write from a step's packed words (step_words()) and one
# layer's tensors; None without _mvlaunch (the wrappers then call
# decode_write with all 35 arguments).
decode_write_step = None

# The step words' layout (csrc/py_launch.c): mv_paged_decode_write's
# step-constant arguments in its order, one little-endian 64-bit word each,
# the scale as a double.
STEP_WORDS_FORMAT = "<10qd9q"
STEP_WORDS = 20


def step_words(slots: int, rope_cos: int, rope_sin: int, work: int, ids: int, ids_cap: int,
               groups: int, part_tokens: int, max_parts: int, counters: int, scale: float,
               num_seqs: int, hq: int, hkv: int, head_dim: int, block_size: int,
               num_blocks: int, dtype_code: int, ws: int, ws_bytes: int) -> bytes:
    """The step-constant arguments of mv_paged_decode_write (addresses as
    ints; None or 0 for a null pointer) packed for decode_write_step."""
    return struct.pack(STEP_WORDS_FORMAT, slots or 0, rope_cos or 0, rope_sin or 0, work or 0,
                       ids or 0, ids_cap, groups, part_tokens, max_parts, counters or 0, scale,
                       num_seqs, hq, hkv, head_dim, block_size, num_blocks, dtype_code, ws or 0,
                       ws_bytes)


def _bind_calls(lib: ctypes.CDLL) -> None:
    global decode_write, decode, cache_write, rope_write, plan, decode_write_step
    ctypes_calls = (lib.mv_paged_decode_write, lib.mv_paged_decode, lib.mv_kv_cache_write,
                    lib.mv_rope_kv_cache_write, lib.mv_decode_plan)
    try:
        from . import _mvlaunch
    except ImportError:
        _mvlaunch = None
    if _mvlaunch is not None and getattr(_mvlaunch, "ABI", None) != ABI_VERSION:
        # built against another header: its argument lists may differ
        warnings.warn(f"{_mvlaunch.__file__}: built for ABI {getattr(_mvlaunch, 'ABI', None)}, "
                      f"the library is ABI {ABI_VERSION}; calling through ctypes "
                      f"(rebuild with build_lib.py)", RuntimeWarning, stacklevel=3)
        _mvlaunch = None
    if _mvlaunch is None:
        decode_write, decode, cache_write, rope_write, plan = ctypes_calls
        decode_write_step = None
        return
    _mvlaunch.bind(*(ctypes.cast(fn, ctypes.c_void_p).value for fn in ctypes_calls))
    decode_write, decode, cache_write, rope_write, plan = (
        _mvlaunch.decode_write, _mvlaunch.decode, _mvlaunch.cache_write, _mvlaunch.rope_write,
        _mvlaunch.plan)
    decode_write_step = (_mvlaunch.decode_write_step
                         if getattr(_mvlaunch, "STEP_WORDS", None) == STEP_WORDS else None)


def load(path: str | None = None) -> ctypes.CDLL:
    """Load (once) and type the kernel library; RuntimeError if it is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or library_path()
        if not os.path.exists(p):
            raise RuntimeError(
                f"HIP kernel library not found at {p}; build it with "
                f"`python {os.path.join(_PKG_ROOT, 'build_lib.py')}`"
            )
        lib = ctypes.CDLL(p)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        if lib.mv_abi_version() != ABI_VERSION:
            raise RuntimeError(
                f"{p}: ABI version {lib.mv_abi_version()} != expected {ABI_VERSION}"
            )
        if path is None:
            _bind_calls(lib)
            _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    """Raise for a non-zero return code of a library call."""
    if rc == MV_OK:
        return
    msg = (load().mv_last_error() or b"").decode(errors="replace")
    if rc == MV_ERR_UNSUPPORTED:
        raise RuntimeError(f"{what}: unsupported: {msg}")
    if rc == MV_ERR_INVALID_ARGUMENT:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg} (code {rc})")
