"""HIP paged-attention backend for MI355X (gfx950).

Drop-in for the reference's Triton backend
(mini_vllm/attention/paged_attention_gpu.py): same class name, same methods,
same module-level entry points with the same argument order and the same
error types, all backed by the hand-written kernels of ``libmvattn.so``:

* ``hip_cache_write``  (alias ``triton_cache_write``, reference :90-154)
* ``hip_decode_attention`` (alias ``triton_decode_attention``, reference :252-321)
* ``gather_prefix_kv`` (reference :391-446)
* ``AttentionBackendGPU`` (reference :454-661)

Validation without per-layer stalls: the reference syncs the host twice per
layer (``slot_mapping.unique()`` and ``(kv_len_after < 1).any()``). Here the
checks run as small device kernels whose status words are read back once per
distinct metadata tensor: the 24 layer calls of one engine step pass the
same ``slot_mapping`` / ``kv_len_after`` / block-table tensor objects, so
only the first call of a step synchronises. A tensor is recognised by
object identity plus its in-place version counter, so an in-place update
(``copy_``, ``fill_``, indexing assignment) triggers a fresh check.
"""

from __future__ import annotations

import ctypes
import math
import os
import threading
import weakref
from dataclasses import dataclass, field
from typing import Any, List, Optional, Sequence, Tuple

import torch

from . import _hip
from ..cache.pool import KVCachePool
from ..model_runner.base import AttentionMetadata, ModelConfig
from .backend import AttentionBackend

SUPPORTED_HEAD_DIMS = (64, 128)
MAX_QUERY_HEADS_PER_KV_HEAD = 16
SUPPORTED_DTYPES = tuple(_hip.MV_DTYPE)

__all__ = [
    "AttentionBackendGPU",
    "DecodePlan",
    "check_deferred",
    "clear_deferred",
    "last_capture_id",
    "gather_prefix_kv",
    "hip_cache_write",
    "hip_decode_attention",
    "hip_prefill_attention",
    "hip_rope_kv_cache_write",
    "hip_rotary",
    "plan_decode",
    "triton_cache_write",
    "triton_decode_attention",
]


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


# torch's raw current-stream accessor costs ~0.1 us per call against ~2 us
# for torch.cuda.current_stream(device).cuda_stream.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> int:
    """The current HIP stream of ``device`` as an address (hipStream_t)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return _raw_stream(index)
    return torch.cuda.current_stream(index).cuda_stream


def _is_pow2(v: int) -> bool:
    return v > 0 and (v & (v - 1)) == 0


class _SeenTensors:
    """Identity + in-place version of the tensors a check was run on."""

    __slots__ = ("refs", "versions", "extra")

    def __init__(self, tensors: Sequence[torch.Tensor], extra: tuple) -> None:
        self.refs = tuple(weakref.ref(t) for t in tensors)
        self.versions = tuple(t._version for t in tensors)
        self.extra = extra

    def matches(self, tensors: Sequence[torch.Tensor], extra: tuple) -> bool:
        if extra != self.extra or len(tensors) != len(self.refs):
            return False
        for r, v, t in zip(self.refs, self.versions, tensors):
            if r() is not t or t._version != v:
                return False
        return True


_state = threading.local()


def _cache_get(name: str, tensors: Sequence[torch.Tensor], extra: tuple):
    entry = getattr(_state, name, None)
    if entry is not None and entry[0].matches(tensors, extra):
        return entry[1]
    return None


def _cache_put(name: str, tensors: Sequence[torch.Tensor], extra: tuple, value) -> None:
    setattr(_state, name, (_SeenTensors(tensors, extra), value))


# Decode merge workspaces, per device: the current one and every one it
# replaced. A captured graph holds the raw address of the buffer it was
# captured with, so a workspace is never released once a kernel has used it:
# a larger batch gets a new buffer and the old one stays allocated for the
# graphs that still point at it (its replays keep writing their partials
# there, never into memory that has become another tensor's).
_WORKSPACES: dict = {}
_RETIRED_WORKSPACES: List[torch.Tensor] = []
_WORKSPACE_LOCK = threading.Lock()


def _grow_only(buffers: dict, device: torch.device, nbytes: int) -> torch.Tensor:
    ws = buffers.get(device)
    if ws is not None and ws.numel() >= nbytes:
        return ws
    with _WORKSPACE_LOCK:
        ws = buffers.get(device)
        if ws is None or ws.numel() < nbytes:
            if ws is not None:
                _RETIRED_WORKSPACES.append(ws)
            ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            buffers[device] = ws
    return ws


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Grow-only, never-freed per-device partial buffer of the decode
    merge."""
    return _grow_only(_WORKSPACES, device, nbytes)


# Hash tables of the slot check (above 4096 tokens) and of the fused-write
# check, per device: rebuilt by every call, kept like the merge workspaces
# for the graphs that captured their address.
_CHECK_WORKSPACES: dict = {}


def _check_workspace(device: torch.device, nbytes: int) -> Optional[torch.Tensor]:
    return _grow_only(_CHECK_WORKSPACES, device, nbytes) if nbytes else None


# ----------------------------------------------------------------------------
# Checks inside a captured graph
#
# While a stream is being captured into a HIP graph nothing may wait for the
# device, so the slot, position and plan checks cannot read their status
# words back. They are captured like every other kernel; each records its
# status tensor under the capture's id, and check_deferred() reads them
# after a replay. The per-step caches of plans and checks are keyed by the
# capture id too: a second capture over the same (unmodified) metadata
# tensors records its own plan and check kernels instead of reusing the
# first graph's buffers.
# ----------------------------------------------------------------------------


def _capture_id(device: torch.device) -> int:
    """Id of the graph capture the current stream of ``device`` is in (HIP's
    capture id, nonzero), or 0 when it is not being captured."""
    if not torch.cuda.is_current_stream_capturing():
        return 0
    cid = ctypes.c_uint64(0)
    _hip.check(_hip.load().mv_stream_capture_id(_stream(device), ctypes.byref(cid)),
               "mv_stream_capture_id")
    return cid.value or -1  # capturing: never 0


def _defer(capture: int, raise_fn, status: torch.Tensor) -> None:
    deferred = getattr(_state, "deferred", None)
    if deferred is None:
        deferred = _state.deferred = {}
    deferred.setdefault(capture, []).append((raise_fn, status))
    _state.last_capture = capture


def last_capture_id() -> int:
    """Id of the most recent graph capture (on this thread) that recorded
    deferred checks, 0 if none: read it right after a capture to check that
    graph's replays by id when several graphs are alive."""
    return getattr(_state, "last_capture", 0)


def check_deferred(capture_id: Optional[int] = None) -> None:
    """Raise the first error found by the checks captured into a graph.

    Call after replaying a captured step (it synchronises once): the same
    exceptions as the eager calls (``IndexError`` / ``AssertionError`` for
    slots, ``IndexError`` for positions, ``ValueError`` / ``IndexError`` /
    ``RuntimeError`` for the decode metadata) describe the data of the last
    replay. Only the checks of one capture are read: ``capture_id``
    (``last_capture_id()`` taken right after that capture), by default the
    most recent capture. The kernels themselves skip what the checks report
    (slots and block ids outside the pool, sequences without a valid
    length), so a bad replay produces wrong rows, never an out-of-bounds
    access.
    """
    deferred = getattr(_state, "deferred", None) or {}
    cid = last_capture_id() if capture_id is None else capture_id
    for raise_fn, status in deferred.get(cid, ()):
        raise_fn(status.tolist())


def clear_deferred(capture_id: Optional[int] = None) -> None:
    """Forget the recorded checks of one capture (e.g. when its graph is
    dropped), or of every capture."""
    deferred = getattr(_state, "deferred", None) or {}
    if capture_id is None:
        _state.deferred = {}
        _state.last_capture = 0
    else:
        deferred.pop(capture_id, None)


# The eager (not captured) per-step checks and plans that _cache_get keeps.
_EAGER_CACHES = ("slots", "fused", "plan", "fused_step", "rope_step", "write_step", "rope_rows",
                 "positions", "prefill")


def invalidate_cached_metadata() -> None:
    """Forget this thread's cached metadata checks and plans (eager calls).

    The wrappers validate a step's metadata (slots, block tables, lengths,
    positions) once and reuse the result, and the decode plan, while the
    same tensor objects come back at the same in-place version
    (``t._version``): the other layers of the step. Writes that torch does
    not see leave that version unchanged: through ``tensor.numpy()`` or
    ``torch.from_numpy``, a DLPack alias, or a raw pointer. After such a
    write, call this before the next call (or pass new tensors, as the
    reference's input builder does every step). Plans made while capturing
    a graph belong to that graph and are kept.
    """
    for name in _EAGER_CACHES:
        if hasattr(_state, name):
            delattr(_state, name)


# ============================================================================
# KV-cache write
# ============================================================================


def _check_slots(slot_mapping: torch.Tensor, total_slots: int,
                 capture: Optional[int] = None) -> None:
    """Raise like the reference for out-of-range or duplicate slots.

    Out of range (``< -1`` or ``>= total_slots``): ``IndexError`` with
    "out of range" (reference cache_write.py:61-66). Duplicates among the
    non-(-1) slots: ``AssertionError`` with "Duplicate" (reference
    paged_attention_gpu.py:126-135). Both checks run in one device kernel.
    ``capture``: the current stream's capture id (0: not capturing), when
    the caller already knows it.
    """
    device = slot_mapping.device
    if capture is None:
        capture = _capture_id(device)
    name = "slots_graph" if capture else "slots"
    extra = (total_slots, capture)
    if _cache_get(name, (slot_mapping,), extra) is not None:
        return
    lib = _hip.load()
    status = torch.empty(2, dtype=torch.int32, device=device)
    n = slot_mapping.numel()
    ws_bytes = lib.mv_kv_slots_check_workspace_bytes(n)
    ws = _check_workspace(device, ws_bytes)
    _hip.check(
        lib.mv_kv_slots_check(
            _ptr(slot_mapping), n, total_slots, _ptr(status), _ptr(ws), ws_bytes, _stream(device)
        ),
        "mv_kv_slots_check",
    )

    def raise_slots(st) -> None:
        bad, dups = st
        if bad:
            raise IndexError(
                f"slot_mapping has {bad} slot(s) out of range [0, {total_slots}) "
                f"(-1 marks a skipped token)"
            )
        if dups:
            raise AssertionError(
                f"Duplicate slots in slot_mapping: {dups} duplicate pair(s). "
                f"The HIP cache write forbids duplicate slots."
            )

    if capture:
        _defer(capture, raise_slots, status)
    else:
        raise_slots(status.tolist())
    _cache_put(name, (slot_mapping,), extra, True)


def hip_cache_write(
    key: torch.Tensor,
    value: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    block_size: int,
) -> None:
    """Scatter-write per-token K/V into one layer's paged cache.

    ``key_cache[s // block_size, :, s % block_size, :] = key[t]`` (and the
    same for ``value``) for every token t whose slot ``s = slot_mapping[t]``
    is not -1; bit-exact. Mirrors ``triton_cache_write``
    (reference paged_attention_gpu.py:90-154): ``AssertionError`` for
    mismatched shapes / dtypes / devices and duplicate slots, plus the
    reference write's ``IndexError`` for slots outside the pool
    (cache_write.py:61-66). ``key`` / ``value`` may be strided views (e.g. V
    sliced out of a fused QKV output) as long as ``head_dim`` is
    contiguous; no staging copy is made.
    """
    num_tokens, num_kv_heads, head_dim = key.shape
    assert key.shape == value.shape, f"key {key.shape} != value {value.shape}"
    assert key_cache.shape == value_cache.shape
    assert slot_mapping.shape == (num_tokens,)
    assert key.dtype == key_cache.dtype, f"key dtype {key.dtype} != cache dtype {key_cache.dtype}"
    assert value.dtype == value_cache.dtype
    assert key.device == key_cache.device, f"key device {key.device} != cache device {key_cache.device}"
    assert key.device.type == "cuda", f"key.device must be cuda, got {key.device}"
    assert block_size == key_cache.shape[2], f"block_size {block_size} != cache dim2 {key_cache.shape[2]}"
    assert key_cache.shape[1] == num_kv_heads and key_cache.shape[3] == head_dim, (
        f"key {tuple(key.shape)} does not match cache {tuple(key_cache.shape)}"
    )
    assert key.dtype in SUPPORTED_DTYPES, f"dtype {key.dtype} not supported"
    assert key_cache.is_contiguous() and value_cache.is_contiguous(), "cache must be contiguous"

    num_blocks = key_cache.shape[0]
    # The other layers of an eager step: the checked slots' device copy
    # from one lookup (same tensor, same version).
    device = key.device
    capture = _capture_id(device)
    step_extra = (num_blocks * block_size, device)
    step = None if capture else _cache_get("write_step", (slot_mapping,), step_extra)
    if step is not None:
        slot_mapping = step
    else:
        slots_given = slot_mapping
        if slot_mapping.device != device:
            slot_mapping = slot_mapping.to(device)
        if slot_mapping.dtype != torch.int64:
            slot_mapping = slot_mapping.to(torch.int64)
        slot_mapping = slot_mapping.contiguous()
        _check_slots(slot_mapping, num_blocks * block_size, capture=capture)
        if not capture:
            _cache_put("write_step", (slots_given,), step_extra, slot_mapping)
    if num_tokens == 0:
        return
    if key.stride(2) != 1:
        key = key.contiguous()
    if value.stride(2) != 1:
        value = value.contiguous()
    _hip.load()  # binds _hip.cache_write
    _hip.check(
        _hip.cache_write(
            _ptr(key), key.stride(0), key.stride(1),
            _ptr(value), value.stride(0), value.stride(1),
            _ptr(key_cache), _ptr(value_cache), _ptr(slot_mapping),
            num_tokens, num_kv_heads, head_dim, block_size, num_blocks,
            _hip.MV_DTYPE[key.dtype], _stream(key.device),
        ),
        "mv_kv_cache_write",
    )


# ============================================================================
# Decode
# ============================================================================


@dataclass
class DecodePlan:
    """Device-side per-step decode metadata produced by ``mv_decode_plan``."""

    work: torch.Tensor         # [8 * capacity] int32: one entry per work group
    block_ids: torch.Tensor    # int32: ids_per_item pool blocks per work group
    counters: torch.Tensor     # [num_seqs * num_kv_heads] int32, zero between calls
    num_groups: int
    max_parts: int
    partition_tokens: int
    # merge workspace bytes per query-head count (asked of the library once)
    ws_bytes: dict = field(default_factory=dict)


# The plan aims for as many work groups as the device holds at once (work
# groups per CU from the library, times the CU count), so the whole grid
# runs in one dispatch round and can be balanced over the CUs.
# MVATTN_GROUPS_PER_CU overrides the per-CU figure.
_SPLIT: dict = {}


def _groups_per_cu(device: torch.device, head_dim: int, dtype: torch.dtype) -> Tuple[int, int]:
    """(work groups per CU, CU count) for the decode plan."""
    key = (device, head_dim, dtype)
    split = _SPLIT.get(key)
    if split is None:
        cus = torch.cuda.get_device_properties(device).multi_processor_count
        per_cu = os.environ.get("MVATTN_GROUPS_PER_CU")
        if per_cu is None:
            per_cu = _hip.load().mv_decode_groups_per_cu(head_dim, _hip.MV_DTYPE[dtype])
        split = _SPLIT[key] = (max(1, int(per_cu)), cus)
    return split


_IDS_CAPACITY: dict = {}


def _ids_capacity(num_seqs: int, max_blocks: int, num_kv_heads: int, cap: int) -> int:
    """``mv_decode_block_ids_capacity``, asked of the library once per shape
    (steps of one batch shape share it)."""
    key = (num_seqs, max_blocks, num_kv_heads, cap)
    n = _IDS_CAPACITY.get(key)
    if n is None:
        if len(_IDS_CAPACITY) > 4096:
            _IDS_CAPACITY.clear()
        n = _IDS_CAPACITY[key] = _hip.load().mv_decode_block_ids_capacity(
            num_seqs, max_blocks, num_kv_heads, cap)
    return n


def _decode_metadata(block_table: torch.Tensor, kv_len_after: torch.Tensor,
                     device: torch.device) -> Tuple[torch.Tensor, torch.Tensor]:
    """Block table ``[B, max_blocks]`` and kv lengths ``[B]`` on ``device``
    as int32 or int64 with contiguous rows (copies only where needed)."""
    bt = block_table
    if bt.dim() != 2:
        bt = bt.reshape(kv_len_after.shape[0], -1)
    if bt.device != device:
        bt = bt.to(device)
    if bt.dtype not in (torch.int32, torch.int64):
        bt = bt.to(torch.int64)
    if bt.numel() and bt.stride(1) != 1:
        bt = bt.contiguous()
    kv = kv_len_after
    if kv.device != device:
        kv = kv.to(device)
    if kv.dtype not in (torch.int32, torch.int64):
        kv = kv.to(torch.int64)
    return bt, kv.contiguous()


def _fused_write_ok(slot_mapping: torch.Tensor, block_table: torch.Tensor,
                    kv_len_after: torch.Tensor, block_size: int, device: torch.device,
                    capture: int) -> bool:
    """Whether the decode with the KV write fused is exact for this batch
    (``mv_decode_write_check``): every slot is -1 or the table position of
    its own sequence's token ``kv_len_after - 1``, as the block manager lays
    them out, and no table entry of the batch reads a written slot other
    than its own sequence's last position (blocks shared without
    copy-on-write, as the reference's prefix cache shares a prompt's
    partial last block, break that). Eager: one device check per distinct
    (unmodified) slots / table / lengths, read back. While capturing: True,
    with the check recorded for ``check_deferred()`` (``AssertionError``).
    Batches of more than ``MV_WRITE_CHECK_MAX_SEQS`` sequences are not
    checked and never fused."""
    num_seqs = kv_len_after.shape[0]
    if num_seqs > _hip.MV_WRITE_CHECK_MAX_SEQS:
        return False
    name = "fused_graph" if capture else "fused"
    extra = (block_size, device, capture)
    hit = _cache_get(name, (slot_mapping, block_table, kv_len_after), extra)
    if hit is not None:
        return hit
    bt, kv = _decode_metadata(block_table, kv_len_after, device)
    lib = _hip.load()
    status = torch.empty(2, dtype=torch.int32, device=device)
    ws_bytes = lib.mv_decode_write_check_workspace_bytes(num_seqs)
    ws = _check_workspace(device, ws_bytes)
    _hip.check(
        lib.mv_decode_write_check(
            _ptr(slot_mapping), _ptr(bt) if bt.numel() else None, int(bt.dtype == torch.int64),
            bt.stride(0) if bt.dim() == 2 else 0, _ptr(kv), int(kv.dtype == torch.int64),
            num_seqs, bt.shape[1] if bt.dim() == 2 else 0, block_size, _ptr(status),
            _ptr(ws), ws_bytes, _stream(device),
        ),
        "mv_decode_write_check",
    )

    def raise_fused(st) -> None:
        own, shared = st
        if own:
            raise AssertionError(
                f"decode with the KV write fused: {own} slot(s) are not their sequence's "
                f"position kv_len_after - 1; write the cache and decode in two calls"
            )
        if shared:
            raise AssertionError(
                f"decode with the KV write fused: {shared} block-table entr(y/ies) of the batch "
                f"read a slot this call writes (a block shared between sequences); write the "
                f"cache and decode in two calls"
            )

    if capture:
        _defer(capture, raise_fused, status)
        ok = True
    else:
        ok = not any(status.tolist())
    _cache_put(name, (slot_mapping, block_table, kv_len_after), extra, ok)
    return ok


def plan_decode(
    block_table: torch.Tensor,
    kv_len_after: torch.Tensor,
    block_size: int,
    num_blocks: int,
    device: torch.device,
    head_dim: int,
    dtype: torch.dtype,
    num_kv_heads: int,
    capture: Optional[int] = None,
) -> DecodePlan:
    """Validate decode metadata, pick the partition size, build the work list.

    Raises ``ValueError`` (message contains "kv_len") when a sequence has
    ``kv_len_after < 1`` (reference paged_attention_gpu.py:294-300) and
    ``IndexError`` when a table row cannot cover ``kv_len_after`` tokens or
    one of the entries it needs is not a pool block (reference
    cache_read.py:60-67 raises "insufficient" for the former; the Triton
    kernel silently skips -1 entries). One host synchronisation per
    distinct (block_table, kv_len_after) pair; later calls with the same,
    unmodified tensors (the other layers of the step) reuse the plan.

    While the current stream is being captured into a graph the plan
    cannot be read back: it is enqueued for a launch of fixed size
    (``mv_decode_graph_bounds``), and its checks raise from
    ``check_deferred()`` after a replay instead. ``capture``: the current
    stream's capture id (0: not capturing), when the caller already knows it.
    """
    if device.index is None:  # "cuda" and "cuda:<current>" are one device: one cached plan
        device = torch.device(device.type, torch.cuda.current_device())
    split = _groups_per_cu(device, head_dim, dtype)
    if capture is None:
        capture = _capture_id(device)
    name = "plan_graph" if capture else "plan"
    extra = (block_size, num_blocks, device, head_dim, dtype, num_kv_heads, split, capture)
    cached = _cache_get(name, (block_table, kv_len_after), extra)
    if cached is not None:
        return cached
    pending = _plan_launch(block_table, kv_len_after, block_size, num_blocks, device, head_dim,
                           dtype, num_kv_heads, split, capture)
    if pending.fixed:
        _defer(capture, pending.raise_plan, pending.status)
        plan = _plan_finish(pending, None)
    else:
        plan = _plan_finish(pending, pending.status.tolist())
    _cache_put(name, (block_table, kv_len_after), extra, plan)
    return plan


@dataclass
class _PendingPlan:
    """A plan launched but not yet read back (``_plan_launch``)."""

    work: torch.Tensor
    block_ids: torch.Tensor
    counters: torch.Tensor
    status: torch.Tensor  # MV_PLAN_WORDS words
    extra: Optional[torch.Tensor]  # status words after the plan's, for the caller
    status_all: torch.Tensor  # the plan's words, then the extra ones
    cap: int
    fixed: int
    fixed_parts: int
    raise_plan: Any


def _plan_launch(block_table: torch.Tensor, kv_len_after: torch.Tensor, block_size: int,
                 num_blocks: int, device: torch.device, head_dim: int, dtype: torch.dtype,
                 num_kv_heads: int, split: Tuple[int, int], capture: int,
                 extra_words: int = 0, step_check: Optional[tuple] = None) -> _PendingPlan:
    """Enqueue mv_decode_plan (no read-back). ``extra_words`` status words
    follow the plan's in the same allocation, so a caller that launches
    more checks reads everything back at once. ``step_check``: the step
    check's own arguments (slot_mapping ... sin_rows, then workspace and
    its size) of ``mv_decode_plan_step_check``, which then enqueues the
    step check with the plan, its status in the extra words."""
    lib = _hip.load()
    bt, kv = _decode_metadata(block_table, kv_len_after, device)

    num_seqs = kv.shape[0]
    max_blocks = bt.shape[1] if bt.dim() == 2 else 0
    fixed = 0
    fixed_parts = 0
    if capture and num_seqs > 0 and max_blocks > 0:
        bounds = (ctypes.c_int64 * 3)()
        _hip.check(lib.mv_decode_graph_bounds(num_seqs, max_blocks, block_size, num_kv_heads,
                                              *split, bounds), "mv_decode_graph_bounds")
        cap, fixed, fixed_parts = bounds
        per_item = ((fixed + block_size - 1) // block_size + 1 + 3) // 4 * 4
        ids_cap = max(lib.mv_decode_block_ids_capacity(num_seqs, max_blocks, num_kv_heads, cap),
                      cap * per_item)
    else:
        cap = num_seqs * num_kv_heads * max(1, math.ceil(max_blocks * block_size / 16))
        ids_cap = _ids_capacity(num_seqs, max_blocks, num_kv_heads, cap)
    # one allocation, cut into the work list, block ids, counters and
    # status words (each part 16-byte aligned); the launch takes the parts'
    # addresses, and their views are made while the plan runs
    n_work, n_ids = 8 * max(cap, 1), -(-max(ids_cap, 4) // 4) * 4
    n_units = max(num_seqs * num_kv_heads, 1)
    n_cnt = -(-n_units // 4) * 4
    n_status = _hip.MV_PLAN_WORDS + extra_words
    buf = torch.empty(n_work + n_ids + n_cnt + n_status, dtype=torch.int32, device=device)
    base = buf.data_ptr()
    plan_args = (
        kv.data_ptr(), int(kv.dtype == torch.int64), bt.data_ptr(),
        int(bt.dtype == torch.int64), bt.stride(0) if bt.dim() == 2 else 0, num_seqs,
        max_blocks, block_size, num_blocks, num_kv_heads, split[0], split[1], fixed,
        base, cap, base + 4 * n_work, n_ids, base + 4 * (n_work + n_ids),
        base + 4 * (n_work + n_ids + n_cnt),
    )
    if step_check is None:
        _hip.check(_hip.plan(*plan_args, _stream(device)), "mv_decode_plan")
    else:
        step_status = base + 4 * (n_work + n_ids + n_cnt + _hip.MV_PLAN_WORDS)
        _hip.check(lib.mv_decode_plan_step_check(*plan_args, *step_check[:10], step_status,
                                                 *step_check[10:], _stream(device)),
                   "mv_decode_plan_step_check")
    s0 = n_work + n_ids + n_cnt
    status_all = buf[s0:]

    def raise_plan(st) -> None:
        if st[_hip.MV_PLAN_BAD_KV_LEN]:
            raise ValueError(
                f"kv_len_after must be >= 1 for all decode sequences, "
                f"got min={st[_hip.MV_PLAN_MIN_KV_LEN]}"
            )
        if st[_hip.MV_PLAN_INSUFFICIENT]:
            raise IndexError(
                f"block_table with {max_blocks} blocks per row (block_size={block_size}) is "
                f"insufficient to cover kv_len_after for {st[_hip.MV_PLAN_INSUFFICIENT]} "
                f"sequence(s)"
            )
        if st[_hip.MV_PLAN_BAD_BLOCK]:
            raise IndexError(
                f"block_table has {st[_hip.MV_PLAN_BAD_BLOCK]} entr(ies) within kv_len_after "
                f"that are not pool blocks [0, {num_blocks})"
            )
        if st[_hip.MV_PLAN_NUM_ITEMS] > cap or st[_hip.MV_PLAN_IDS_PER_ITEM] < 0:
            raise RuntimeError(
                f"decode plan: {st[_hip.MV_PLAN_NUM_ITEMS]} work groups exceed the plan "
                f"capacity {cap}"
            )

    return _PendingPlan(
        work=buf[:n_work], block_ids=buf[n_work:n_work + n_ids],
        counters=buf[n_work + n_ids:n_work + n_ids + n_units],
        status=status_all[:_hip.MV_PLAN_WORDS],
        extra=status_all[_hip.MV_PLAN_WORDS:] if extra_words else None, status_all=status_all,
        cap=cap, fixed=fixed, fixed_parts=fixed_parts, raise_plan=raise_plan)


def _plan_finish(p: _PendingPlan, st: Optional[List[int]]) -> DecodePlan:
    """The DecodePlan of a launched plan: of fixed size (graph capture, its
    checks deferred by the caller), or from its status words ``st`` read
    back, raising for bad metadata."""
    if p.fixed:
        return DecodePlan(p.work, p.block_ids, p.counters, p.cap, p.fixed_parts, p.fixed)
    p.raise_plan(st)
    return DecodePlan(p.work, p.block_ids, p.counters, st[_hip.MV_PLAN_NUM_ITEMS],
                      st[_hip.MV_PLAN_MAX_PARTS], st[_hip.MV_PLAN_PARTITION_TOKENS])


def _rope_rows(positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, head_dim: int,
               dtype: torch.dtype, device: torch.device,
               capture: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """The cos / sin table rows at each decode token's position,
    ``[B, head_dim]`` contiguous, for the decode kernel's fused RoPE;
    gathered once per distinct (unmodified) positions / tables (the layers
    of a step share them) after the positions check (``IndexError``, as the
    reference's table lookup raises)."""
    name = "rope_rows_graph" if capture else "rope_rows"
    extra = (head_dim, dtype, device, capture)
    hit = _cache_get(name, (positions, cos, sin), extra)
    if hit is not None:
        return hit
    assert cos.dim() == 2 and cos.shape == sin.shape and cos.shape[1] >= head_dim, (
        f"rotary tables {tuple(cos.shape)} / {tuple(sin.shape)} do not cover head_dim {head_dim}"
    )
    assert cos.dtype == dtype and sin.dtype == dtype, f"rotary tables {cos.dtype} != {dtype}"
    assert cos.device == device and sin.device == device
    pos = positions
    if pos.device != device:
        pos = pos.to(device)
    if pos.dtype != torch.int64:
        pos = pos.to(torch.int64)
    pos = pos.contiguous()
    _check_positions(pos, cos.shape[0])
    # out-of-range positions are reported by the check; clamped here so the
    # gather itself stays inside the tables
    idx = pos.clamp(0, cos.shape[0] - 1)
    rows = (cos.index_select(0, idx)[:, :head_dim].contiguous(),
            sin.index_select(0, idx)[:, :head_dim].contiguous())
    _cache_put(name, (positions, cos, sin), extra, rows)
    return rows


def _fused_step_prepare(block_table: torch.Tensor, kv_len_after: torch.Tensor, block_size: int,
                        num_blocks: int, device: torch.device, head_dim: int, dtype: torch.dtype,
                        num_kv_heads: int, slot_mapping: torch.Tensor,
                        positions: Optional[torch.Tensor], cos: Optional[torch.Tensor],
                        sin: Optional[torch.Tensor], capture: int):
    """A step's plan and checks for the fused decode layer call, launched
    together and read back once (eager; captured: deferred): the plan
    (``plan_decode``, unless the step's tables and lengths already have one)
    and ``mv_decode_step_check`` -- the slot check (``_check_slots``), the
    fused-write precondition (``_fused_write_ok``) and, with RoPE, the
    positions check and the rotary rows (``_rope_rows``). Raises what those
    raise, in that order, and fills their caches so that the step's other
    layers, and the two-call sequence a failed precondition falls back to,
    find them. Returns (plan, slots on the device as int64, whether the
    fused launch is exact, the rotary rows or None)."""
    if slot_mapping.device != device:
        slot_mapping = slot_mapping.to(device)
    if slot_mapping.dtype != torch.int64:
        slot_mapping = slot_mapping.to(torch.int64)
    slots = slot_mapping.contiguous()
    num_seqs = kv_len_after.shape[0]
    rope = positions is not None
    if num_seqs > _hip.MV_WRITE_CHECK_MAX_SEQS:  # not checked: never fused
        plan = plan_decode(block_table, kv_len_after, block_size, num_blocks, device, head_dim,
                           dtype, num_kv_heads, capture=capture)
        _check_slots(slots, num_blocks * block_size, capture=capture)
        return plan, slots, False, None
    if device.index is None:
        device = torch.device(device.type, torch.cuda.current_device())
    lib = _hip.load()
    split = _groups_per_cu(device, head_dim, dtype)
    g = "_graph" if capture else ""
    plan_name = "plan" + g
    plan_extra = (block_size, num_blocks, device, head_dim, dtype, num_kv_heads, split, capture)
    plan = _cache_get(plan_name, (block_table, kv_len_after), plan_extra)
    total_slots = num_blocks * block_size
    # the step's other layers (and a failed precondition's fallback): all
    # of it from the checks' caches, nothing launched
    if plan is not None and _cache_get("slots" + g, (slots,), (total_slots, capture)) is not None:
        fused_ok = _cache_get("fused" + g, (slots, block_table, kv_len_after),
                              (block_size, device, capture))
        rows = None
        if rope:
            rows = _cache_get("rope_rows" + g, (positions, cos, sin), (head_dim, dtype, device, capture))
        if fused_ok is not None and (rows is not None or not rope):
            return plan, slots, fused_ok, rows
    bt, kv = _decode_metadata(block_table, kv_len_after, device)
    pos = rows = None
    max_pos = 0
    if rope:
        assert cos.dim() == 2 and cos.shape == sin.shape and cos.shape[1] >= head_dim, (
            f"rotary tables {tuple(cos.shape)} / {tuple(sin.shape)} do not cover head_dim {head_dim}"
        )
        assert cos.dtype == dtype and sin.dtype == dtype, f"rotary tables {cos.dtype} != {dtype}"
        assert cos.device == device and sin.device == device
        pos = positions
        if pos.device != device:
            pos = pos.to(device)
        if pos.dtype != torch.int64:
            pos = pos.to(torch.int64)
        pos = pos.contiguous()
        tc, ts = cos, sin
        if (tc.stride(1) != 1 or ts.stride(1) != 1 or tc.stride(0) != ts.stride(0)
                or (tc.stride(0) * tc.element_size()) % 16 or tc.data_ptr() % 16
                or ts.data_ptr() % 16):
            tc, ts = tc.contiguous(), ts.contiguous()
        max_pos = tc.shape[0]
        rows = (torch.empty(num_seqs, head_dim, dtype=dtype, device=device),
                torch.empty(num_seqs, head_dim, dtype=dtype, device=device))
    ws_bytes = lib.mv_decode_write_check_workspace_bytes(num_seqs)
    ws = _check_workspace(device, ws_bytes)
    # the step check's own arguments, in mv_decode_plan_step_check's order
    # (its status pointer goes between the rows and the workspace)
    step = (_ptr(slots), _ptr(pos), _ptr(tc) if rope else None, _ptr(ts) if rope else None,
            tc.stride(0) if rope else 0, max_pos, head_dim, _hip.MV_DTYPE[dtype],
            _ptr(rows[0]) if rope else None, _ptr(rows[1]) if rope else None, None,
            _ptr(ws), ws_bytes)
    pending = None
    if plan is None:
        # the plan and the step check enqueued together (one launch for
        # small batches), their status words in one allocation
        pending = _plan_launch(block_table, kv_len_after, block_size, num_blocks, device,
                               head_dim, dtype, num_kv_heads, split, capture,
                               extra_words=_hip.MV_STEP_WORDS, step_check=step[:10] + step[11:])
        status = pending.extra
    else:
        status = torch.empty(_hip.MV_STEP_WORDS, dtype=torch.int32, device=device)
        _hip.check(
            lib.mv_decode_step_check(
                step[0], _ptr(bt) if bt.numel() else None, int(bt.dtype == torch.int64),
                bt.stride(0) if bt.dim() == 2 else 0, _ptr(kv), int(kv.dtype == torch.int64),
                num_seqs, bt.shape[1] if bt.dim() == 2 else 0, block_size, num_blocks,
                *step[1:10], _ptr(status), *step[11:], _stream(device),
            ),
            "mv_decode_step_check",
        )

    def raise_slots(st) -> None:
        bad, dups = st[_hip.MV_STEP_SLOTS_OUT_OF_RANGE], st[_hip.MV_STEP_SLOTS_DUPLICATES]
        if bad:
            raise IndexError(
                f"slot_mapping has {bad} slot(s) out of range [0, {total_slots}) "
                f"(-1 marks a skipped token)"
            )
        if dups:
            raise AssertionError(
                f"Duplicate slots in slot_mapping: {dups} duplicate pair(s). "
                f"The HIP cache write forbids duplicate slots."
            )

    def raise_fused(st) -> None:
        own, shared = st[_hip.MV_STEP_WRITE_OWN_SLOT], st[_hip.MV_STEP_WRITE_SHARED]
        if own:
            raise AssertionError(
                f"decode with the KV write fused: {own} slot(s) are not their sequence's "
                f"position kv_len_after - 1; write the cache and decode in two calls"
            )
        if shared:
            raise AssertionError(
                f"decode with the KV write fused: {shared} block-table entr(y/ies) of the batch "
                f"read a slot this call writes (a block shared between sequences); write the "
                f"cache and decode in two calls"
            )

    def raise_positions(st) -> None:
        if st[_hip.MV_STEP_POSITIONS]:
            raise IndexError(f"{st[_hip.MV_STEP_POSITIONS]} position(s) outside the rotary "
                             f"tables [0, {max_pos})")

    if capture:
        if pending is not None:
            _defer(capture, pending.raise_plan, pending.status)
            plan = _plan_finish(pending, None)
        _defer(capture, raise_slots, status)
        _defer(capture, raise_fused, status)
        if rope:
            _defer(capture, raise_positions, status)
        fused_ok = True
    else:
        st = (pending.status_all if pending is not None else status).tolist()
        if pending is not None:
            plan = _plan_finish(pending, st[:_hip.MV_PLAN_WORDS])
            st = st[_hip.MV_PLAN_WORDS:]
        raise_slots(st)
        if rope:
            raise_positions(st)
        fused_ok = not (st[_hip.MV_STEP_WRITE_OWN_SLOT] or st[_hip.MV_STEP_WRITE_SHARED])
    # the checks' own caches: the step's other layers and the two-call
    # fallback look them up
    if pending is not None:
        _cache_put(plan_name, (block_table, kv_len_after), plan_extra, plan)
    _cache_put("slots" + g, (slots,), (total_slots, capture), True)
    _cache_put("fused" + g, (slots, block_table, kv_len_after), (block_size, device, capture),
               fused_ok)
    if rope:
        _cache_put("positions" + g, (pos,), (max_pos, capture), True)
        _cache_put("rope_rows" + g, (positions, cos, sin), (head_dim, dtype, device, capture), rows)
    return plan, slots, fused_ok, rows


def hip_decode_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    kv_len_after: torch.Tensor,
    block_size: int,
    *,
    new_key: Optional[torch.Tensor] = None,
    new_value: Optional[torch.Tensor] = None,
    slot_mapping: Optional[torch.Tensor] = None,
    positions: Optional[torch.Tensor] = None,
    cos: Optional[torch.Tensor] = None,
    sin: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Paged decode attention on the HIP kernels.

    Args (same order and meaning as ``triton_decode_attention``,
    reference paged_attention_gpu.py:252-321):
        query: ``[total_decode, num_q_heads, head_dim]`` fp16 / bf16 / fp32
        key_cache, value_cache: ``[num_blocks, num_kv_heads, block_size, head_dim]``
        block_table: ``[total_decode, max_blocks]`` int64 or int32, -1 padded
        kv_len_after: ``[total_decode]`` int64 or int32 (tokens to attend)
        block_size: tokens per block (power of 2)

    Returns ``[total_decode, num_q_heads, head_dim]`` in ``query.dtype``.
    Query head h attends kv head ``h // (num_q_heads // num_kv_heads)`` with
    scale ``head_dim ** -0.5``.

    With ``new_key`` / ``new_value`` ``[total_decode, num_kv_heads,
    head_dim]`` and ``slot_mapping`` ``[total_decode]`` the call also does
    the step's KV write of those rows (``triton_cache_write``, with its
    checks): pool and output are those of ``hip_cache_write`` followed by
    this call without them. It is one launch when every slot is -1 or its
    own sequence's position ``kv_len_after - 1`` and no other table entry
    of the batch reads that slot -- the block manager's layout (a
    sequence's last block is its own). A batch that breaks either (slots
    elsewhere, or a written block shared with another sequence that
    attends the slot) is detected on the device and runs as the two calls;
    inside a captured graph it is reported by ``check_deferred()``
    (``AssertionError``) instead.

    With ``positions`` ``[total_decode]`` and the rotary tables ``cos`` /
    ``sin`` (``[max_positions, >= head_dim]``, the query dtype) as well, the
    same launch first applies the rotary embedding to ``query`` and
    ``new_key`` (reference rotary.py:44-82, the reference's rounding): the
    runner's ``q = rope(q); k = rope(k); write_kv_cache(k, v);
    decode_attention(q)`` for the decode rows (qwen_runner.py:164-190), with
    output and pool bit-identical to ``hip_rope_kv_cache_write`` followed by
    this call on the rotated query.
    """
    # (The per-call checks read each attribute once: this wrapper runs once
    # per layer, and its host time exceeds the kernel's when it does not.)
    total_decode, num_q_heads, head_dim = query.shape
    kshape = key_cache.shape
    num_kv_heads = kshape[1]
    dtype = query.dtype
    assert head_dim in SUPPORTED_HEAD_DIMS, f"head_dim {head_dim} not supported (only 64, 128)"
    assert block_size > 0 and _is_pow2(block_size), f"block_size {block_size} must be a power of 2"
    assert num_q_heads % num_kv_heads == 0, (
        f"num_q_heads {num_q_heads} not divisible by num_kv_heads {num_kv_heads}"
    )
    assert num_q_heads // num_kv_heads <= MAX_QUERY_HEADS_PER_KV_HEAD, (
        f"{num_q_heads // num_kv_heads} query heads per kv head (max {MAX_QUERY_HEADS_PER_KV_HEAD})"
    )
    assert dtype in SUPPORTED_DTYPES, f"query dtype {dtype} not supported"
    assert key_cache.dtype == dtype, f"key_cache dtype {key_cache.dtype} != {dtype}"
    assert value_cache.dtype == dtype
    assert query.is_cuda
    assert kshape == value_cache.shape
    assert kshape[2] == block_size and kshape[3] == head_dim
    assert key_cache.is_contiguous() and value_cache.is_contiguous()
    assert block_table.shape[0] == total_decode
    assert kv_len_after.shape == (total_decode,)

    device = query.device
    num_blocks = kshape[0]
    capture = _capture_id(device)
    # The other layers of an eager step with the KV write fused: the plan,
    # the slot check, the fused-write check and the slots' device copy in
    # one lookup (same tensors at the same in-place versions).
    step = None
    step_extra = (block_size, num_blocks, device, head_dim, dtype, num_kv_heads)
    fused = new_key is not None
    rope = positions is not None
    fused_ok = True
    rope_rows = None
    if fused:
        assert new_value is not None and slot_mapping is not None
        nshape = new_key.shape
        assert nshape == (total_decode, num_kv_heads, head_dim), (
            f"new_key {tuple(nshape)} != ({total_decode}, {num_kv_heads}, {head_dim})"
        )
        assert new_value.shape == nshape
        assert new_key.dtype == dtype and new_value.dtype == dtype
        assert new_key.device == device and new_value.device == device
        if rope:
            assert cos is not None and sin is not None
            assert positions.shape == (total_decode,)
        if not capture:
            step = _cache_get("fused_step", (slot_mapping, block_table, kv_len_after), step_extra)
    templates = None
    if step is not None:
        plan, slot_mapping, templates = step
        if _hip.decode_write_step is not None and total_decode and plan.num_groups:
            # the step's packed launch words, for these query heads and
            # rotary rows, while the merge workspace they point at is current
            rows = _rope_rows(positions, cos, sin, head_dim, dtype, device, 0) if rope else None
            words = templates.get((num_q_heads, id(rows[0]) if rope else 0))
            if words is not None and (words[1] is None or _WORKSPACES.get(device) is words[1]):
                return _decode_write_step(words[0], query, new_key, new_value, key_cache,
                                          value_cache, device)
    elif fused:
        # the step's plan and checks: launched together, read back once
        slots_given = slot_mapping
        assert slot_mapping.shape == (total_decode,)
        plan, slot_mapping, fused_ok, rope_rows = _fused_step_prepare(
            block_table, kv_len_after, block_size, num_blocks, device, head_dim, dtype,
            num_kv_heads, slot_mapping, positions, cos, sin, capture)
        if fused_ok and not capture:
            templates = {}
            _cache_put("fused_step", (slots_given, block_table, kv_len_after), step_extra,
                       (plan, slot_mapping, templates))
    else:
        plan = plan_decode(block_table, kv_len_after, block_size, num_blocks, device, head_dim,
                           dtype, num_kv_heads, capture=capture)
    output = torch.empty_like(query, memory_format=torch.contiguous_format)
    if total_decode == 0 or plan.num_groups == 0:
        return output
    if query.stride(2) != 1 or (query.stride(1) * query.element_size()) % 16 or (
        query.stride(0) * query.element_size()
    ) % 16 or query.data_ptr() % 16:
        query = query.contiguous()
    lib = _hip.load()
    ws_bytes = plan.ws_bytes.get(num_q_heads)
    if ws_bytes is None:
        ws_bytes = plan.ws_bytes[num_q_heads] = lib.mv_paged_decode_workspace_bytes(
            total_decode, num_q_heads, head_dim, plan.max_parts)
    ws = _workspace(device, ws_bytes) if ws_bytes else None
    if fused:
        if not fused_ok:
            if rope:  # the unfused sequence: rope + write, then decode of the rotated query
                query, _ = hip_rope_kv_cache_write(query, new_key, new_value, positions, cos, sin,
                                                   key_cache, value_cache, slot_mapping,
                                                   block_size, return_key=False)
            else:
                hip_cache_write(new_key, new_value, key_cache, value_cache, slot_mapping,
                                block_size)
            return hip_decode_attention(query, key_cache, value_cache, block_table, kv_len_after,
                                        block_size)
        rope_cos = rope_sin = None
        if rope:
            rope_cos, rope_sin = rope_rows if rope_rows is not None else _rope_rows(
                positions, cos, sin, head_dim, dtype, device, capture)
        nk, nv = _aligned_rows(new_key), _aligned_rows(new_value)
        if templates is not None and _hip.decode_write_step is not None:
            # the other layers of the step launch from these words
            words = _hip.step_words(
                _ptr(slot_mapping), _ptr(rope_cos), _ptr(rope_sin), _ptr(plan.work),
                _ptr(plan.block_ids), plan.block_ids.numel(), plan.num_groups,
                plan.partition_tokens, plan.max_parts, _ptr(plan.counters),
                float(head_dim ** -0.5), total_decode, num_q_heads, num_kv_heads, head_dim,
                block_size, num_blocks, _hip.MV_DTYPE[dtype], _ptr(ws),
                ws.numel() if ws is not None else 0)
            templates[(num_q_heads, id(rope_cos) if rope else 0)] = (
                words, ws, (rope_cos, rope_sin) if rope else None)
        _hip.check(
            _hip.decode_write(
                _ptr(query), query.stride(0), query.stride(1),
                _ptr(nk), nk.stride(0), nk.stride(1), _ptr(nv), nv.stride(0), nv.stride(1),
                _ptr(slot_mapping), _ptr(rope_cos), _ptr(rope_sin), _ptr(key_cache),
                _ptr(value_cache),
                _ptr(plan.work), _ptr(plan.block_ids), plan.block_ids.numel(), plan.num_groups,
                plan.partition_tokens, plan.max_parts, _ptr(plan.counters),
                _ptr(output), output.stride(0), output.stride(1),
                float(head_dim ** -0.5), total_decode, num_q_heads, num_kv_heads, head_dim,
                block_size, num_blocks, _hip.MV_DTYPE[dtype],
                _ptr(ws), ws.numel() if ws is not None else 0, _stream(device),
            ),
            "mv_paged_decode_write",
        )
        return output
    _hip.check(
        _hip.decode(
            _ptr(query), query.stride(0), query.stride(1),
            _ptr(key_cache), _ptr(value_cache),
            _ptr(plan.work), _ptr(plan.block_ids), plan.block_ids.numel(), plan.num_groups,
            plan.partition_tokens, plan.max_parts, _ptr(plan.counters),
            _ptr(output), output.stride(0), output.stride(1),
            float(head_dim ** -0.5), total_decode, num_q_heads, num_kv_heads, head_dim,
            block_size, num_blocks, _hip.MV_DTYPE[dtype],
            _ptr(ws), ws.numel() if ws is not None else 0, _stream(device),
        ),
        "mv_paged_decode",
    )
    return output


def _row_args(x: torch.Tensor):
    """(x, address, row stride, head stride) with 16-byte aligned,
    head_dim-contiguous rows (a copy only if not)."""
    st = x.stride()
    p = x.data_ptr()
    eb = x.element_size()
    if st[2] != 1 or (st[0] * eb) % 16 or (st[1] * eb) % 16 or p % 16:
        x = x.contiguous()
        st = x.stride()
        p = x.data_ptr()
    return x, p, st[0], st[1]


def _decode_write_step(words: bytes, query: torch.Tensor, new_key: torch.Tensor,
                       new_value: torch.Tensor, key_cache: torch.Tensor,
                       value_cache: torch.Tensor, device: torch.device) -> torch.Tensor:
    """A layer of a step whose fused launch was already made once: the
    step's packed words (plan, slots, rotary rows, sizes, workspace) and
    this layer's tensors."""
    output = torch.empty_like(query, memory_format=torch.contiguous_format)
    q, qp, q_st, q_sh = _row_args(query)
    nk, nkp, nk_st, nk_sh = _row_args(new_key)
    nv, nvp, nv_st, nv_sh = _row_args(new_value)
    o_st = output.stride()
    _hip.check(
        _hip.decode_write_step(words, qp, q_st, q_sh, nkp, nk_st, nk_sh, nvp, nv_st, nv_sh,
                               key_cache.data_ptr(), value_cache.data_ptr(), output.data_ptr(),
                               o_st[0], o_st[1], _stream(device)),
        "mv_paged_decode_write",
    )
    return output


# The reference's tests and benchmarks import these names.
triton_cache_write = hip_cache_write
triton_decode_attention = hip_decode_attention


# ============================================================================
# Rotary embedding (+ KV write)
# ============================================================================


def _check_positions(positions: torch.Tensor, max_positions: int) -> None:
    """``IndexError`` for a position outside the cos / sin tables, as the
    reference's lookup ``self._cos[positions]`` raises
    (mini_vllm/model/rotary.py:64-65). One device check per distinct
    positions tensor (the layers of a step share it)."""
    device = positions.device
    capture = _capture_id(device)
    name = "positions_graph" if capture else "positions"
    extra = (max_positions, capture)
    if _cache_get(name, (positions,), extra) is not None:
        return
    lib = _hip.load()
    status = torch.empty(1, dtype=torch.int32, device=device)
    _hip.check(
        lib.mv_positions_check(_ptr(positions), positions.numel(), max_positions, _ptr(status),
                               _stream(device)),
        "mv_positions_check",
    )

    def raise_positions(st) -> None:
        if st[0]:
            raise IndexError(f"{st[0]} position(s) outside the rotary tables [0, {max_positions})")

    if capture:
        _defer(capture, raise_positions, status)
    else:
        raise_positions(status.tolist())
    _cache_put(name, (positions,), extra, True)


def _rope_operand(x: torch.Tensor) -> torch.Tensor:
    """x with 16-byte aligned, head_dim-contiguous rows (a copy only if not)."""
    eb = x.element_size()
    if (x.stride(2) != 1 or (x.stride(0) * eb) % 16 or (x.stride(1) * eb) % 16
            or x.data_ptr() % 16):
        x = x.contiguous()
    return x


def hip_rope_kv_cache_write(
    query: Optional[torch.Tensor],
    key: torch.Tensor,
    value: Optional[torch.Tensor],
    positions: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    key_cache: Optional[torch.Tensor] = None,
    value_cache: Optional[torch.Tensor] = None,
    slot_mapping: Optional[torch.Tensor] = None,
    block_size: int = 0,
    *,
    return_key: bool = True,
    inplace: bool = False,
) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
    """Fused ``q = rope(q, positions); k = rope(k, positions);
    write_kv_cache(k, v, slot_mapping)`` in one launch.

    Replaces the runner's three calls (reference qwen_runner.py:164-170):
    ``RotaryEmbedding.__call__`` (rotary.py:44-82, tables ``rope.cos`` /
    ``rope.sin`` of ``[max_seq_len, head_dim]`` in the model dtype) on
    ``query`` ``[T, Hq, D]`` and ``key`` ``[T, Hkv, D]``, then
    ``triton_cache_write`` (paged_attention_gpu.py:90-154) of the rotated
    key and of ``value``. Results are bit-identical to the reference's
    eager ops (each product and the sum rounded to the dtype).

    Returns ``(query_rot, key_rot)``: ``query_rot`` is a new tensor, or
    ``query`` itself with ``inplace=True`` (None without a query);
    ``key_rot`` is materialised only with ``return_key=True`` (prefill
    attention reads it), else None. Without ``key_cache`` nothing is
    written to a cache (a plain rotary of query and key). Errors as the
    reference: ``AssertionError`` (shapes, dtypes, duplicate slots),
    ``IndexError`` (slot or position out of range).
    """
    num_tokens, num_kv_heads, head_dim = key.shape
    dtype, device = key.dtype, key.device
    assert device.type == "cuda", f"key.device must be cuda, got {device}"
    assert dtype in SUPPORTED_DTYPES, f"dtype {dtype} not supported"
    assert positions.shape == (num_tokens,), f"positions {tuple(positions.shape)} != ({num_tokens},)"
    assert cos.dim() == 2 and cos.shape == sin.shape and cos.shape[1] >= head_dim, (
        f"rotary tables {tuple(cos.shape)} / {tuple(sin.shape)} do not cover head_dim {head_dim}"
    )
    assert cos.dtype == dtype and sin.dtype == dtype, f"rotary tables {cos.dtype} != {dtype}"
    assert cos.device == device and sin.device == device
    num_q_heads = 0
    if query is not None:
        assert query.dim() == 3 and query.shape[0] == num_tokens and query.shape[2] == head_dim, (
            f"query {tuple(query.shape)} does not match key {tuple(key.shape)}"
        )
        assert query.dtype == dtype and query.device == device
        num_q_heads = query.shape[1]
    write = key_cache is not None
    num_blocks = 0
    if write:
        assert value is not None and value_cache is not None and slot_mapping is not None
        assert key.shape == value.shape, f"key {key.shape} != value {value.shape}"
        assert key_cache.shape == value_cache.shape
        assert value.dtype == dtype and key_cache.dtype == dtype and value_cache.dtype == dtype
        assert key_cache.device == device and value_cache.device == device
        assert slot_mapping.shape == (num_tokens,)
        assert block_size == key_cache.shape[2], f"block_size {block_size} != cache dim2 {key_cache.shape[2]}"
        assert _is_pow2(block_size), f"block_size {block_size} must be a power of 2"
        assert key_cache.shape[1] == num_kv_heads and key_cache.shape[3] == head_dim
        assert key_cache.is_contiguous() and value_cache.is_contiguous(), "cache must be contiguous"
        num_blocks = key_cache.shape[0]
    # The other layers of an eager step: the slot and position checks and
    # their device copies in one lookup (same tensors, same versions).
    capture = _capture_id(device)
    given = (slot_mapping, positions) if write else (positions,)
    step_extra = (num_blocks * block_size, cos.shape[0], device)
    step = None if capture else _cache_get("rope_step", given, step_extra)
    if step is not None:
        slot_mapping, positions = step
    else:
        if write:
            if slot_mapping.device != device:
                slot_mapping = slot_mapping.to(device)
            if slot_mapping.dtype != torch.int64:
                slot_mapping = slot_mapping.to(torch.int64)
            slot_mapping = slot_mapping.contiguous()
            _check_slots(slot_mapping, num_blocks * block_size, capture=capture)
        if positions.device != device:
            positions = positions.to(device)
        if positions.dtype != torch.int64:
            positions = positions.to(torch.int64)
        positions = positions.contiguous()
        _check_positions(positions, cos.shape[0])
        if not capture:
            _cache_put("rope_step", given, step_extra, (slot_mapping, positions))

    q_out = None
    if query is not None:
        query = _rope_operand(query)
        q_out = query if inplace else torch.empty_like(query, memory_format=torch.contiguous_format)
    k_out = torch.empty_like(key, memory_format=torch.contiguous_format) if return_key else None
    if num_tokens == 0:
        return q_out, k_out
    key = _rope_operand(key)
    if write:
        value = _rope_operand(value)
    if cos.stride(1) != 1 or sin.stride(1) != 1 or cos.stride(0) != sin.stride(0):
        cos, sin = cos.contiguous(), sin.contiguous()
    _hip.load()  # binds _hip.rope_write
    _hip.check(
        _hip.rope_write(
            _ptr(query), query.stride(0) if query is not None else 0,
            query.stride(1) if query is not None else 0,
            _ptr(q_out), q_out.stride(0) if q_out is not None else 0,
            q_out.stride(1) if q_out is not None else 0,
            _ptr(key), key.stride(0), key.stride(1),
            _ptr(k_out), k_out.stride(0) if k_out is not None else 0,
            k_out.stride(1) if k_out is not None else 0,
            _ptr(value) if write else None, value.stride(0) if write else 0,
            value.stride(1) if write else 0,
            _ptr(key_cache), _ptr(value_cache), _ptr(slot_mapping) if write else None,
            _ptr(positions), _ptr(cos), _ptr(sin), cos.stride(0), cos.shape[0],
            num_tokens, num_q_heads, num_kv_heads, head_dim, block_size if write else 0,
            num_blocks, _hip.MV_DTYPE[dtype], _stream(device),
        ),
        "mv_rope_kv_cache_write",
    )
    return q_out, k_out


def hip_rotary(x: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor,
               sin: torch.Tensor) -> torch.Tensor:
    """``RotaryEmbedding.__call__`` (reference rotary.py:44-66) on the GPU:
    ``x`` ``[T, H, D]`` rotated at ``positions`` with tables ``cos`` /
    ``sin``; a new tensor, bit-identical to the reference's eager ops."""
    _, out = hip_rope_kv_cache_write(None, x, None, positions, cos, sin, return_key=True)
    return out


# ============================================================================
# Prefill prefix gather
# ============================================================================


def gather_prefix_kv(
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    cached_len_before: Sequence[int],
    seq_indices: Sequence[int],
    block_size: int,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Gather the cached prefix K/V of prefill sequences into contiguous rows.

    Same contract as the reference (paged_attention_gpu.py:391-446): output
    ``[sum(cached_len_before), num_kv_heads, head_dim]`` with sequence i's
    ``cached_len_before[i]`` tokens taken from table row ``seq_indices[i]``.
    Raises ``IndexError`` (message contains "insufficient") when a row
    cannot cover its prefix and when a needed entry is not a pool block.
    """
    num_blocks, num_kv_heads, bs, head_dim = key_cache.shape
    assert bs == block_size, f"block_size {block_size} != cache dim2 {bs}"
    assert key_cache.shape == value_cache.shape and key_cache.dtype == value_cache.dtype
    assert key_cache.is_contiguous() and value_cache.is_contiguous()
    lens = [int(c) for c in cached_len_before]
    rows = [int(s) for s in seq_indices]
    assert len(lens) == len(rows)
    total = sum(lens)
    device = key_cache.device
    out_k = torch.empty(total, num_kv_heads, head_dim, dtype=key_cache.dtype, device=device)
    out_v = torch.empty_like(out_k)
    if total == 0:
        return out_k, out_v
    bt_host = block_table.detach().to("cpu", torch.int64)
    if bt_host.dim() != 2:
        bt_host = bt_host.reshape(-1, bt_host.shape[-1] if bt_host.dim() else 0)
    _check_prefix_tables(bt_host, rows, lens, block_size, num_blocks)
    bt = block_table.to(device)
    if bt.dtype not in (torch.int32, torch.int64):
        bt = bt.to(torch.int64)
    if bt.dim() != 2:
        bt = bt.reshape(bt_host.shape)
    bt = bt.contiguous()
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    meta = torch.tensor([*rows, *cu], dtype=torch.int64).to(device, non_blocking=True)
    lib = _hip.load()
    _hip.check(
        lib.mv_gather_paged_kv(
            _ptr(key_cache), _ptr(value_cache), _ptr(bt), int(bt.dtype == torch.int64),
            bt.stride(0), _ptr(meta), _ptr(meta) + 8 * len(rows), len(rows), total,
            _ptr(out_k), _ptr(out_v), num_kv_heads, head_dim, block_size, num_blocks,
            _hip.MV_DTYPE[key_cache.dtype], _stream(device),
        ),
        "mv_gather_paged_kv",
    )
    return out_k, out_v


# ============================================================================
# Prefill attention
# ============================================================================


def _check_prefix_tables(bt_host: torch.Tensor, rows: Sequence[int], lens: Sequence[int],
                         block_size: int, num_blocks: int) -> None:
    """``IndexError`` ("insufficient") when a table row cannot cover its
    sequence's cached prefix or one of the entries it needs is not a pool
    block (reference cache/cache_read.py:60-67)."""
    for row, n in zip(rows, lens):
        need = -(-n // block_size)
        if not 0 <= row < bt_host.shape[0] or need > bt_host.shape[1]:
            raise IndexError(f"block_table row {row} insufficient to cover {n} tokens")
        ids = bt_host[row, :need]
        if need and (int(ids.min()) < 0 or int(ids.max()) >= num_blocks):
            raise IndexError(
                f"block_table row {row} insufficient: entries {ids.tolist()} are not all pool blocks"
            )


PREFILL_MAX_PARTS = 8     # key parts per prefill unit (mv_paged_prefill_parts)
PREFILL_PART_KEYS = 256   # parts start at multiples of this many keys


def prefill_key_parts(key_ends: Sequence[int], cu_count: int,
                      max_parts: int = PREFILL_MAX_PARTS) -> List[List[Tuple[int, int]]]:
    """Key ranges of the parts of each prefill unit (one (sequence, kv head,
    token block) work group, whose rows see keys ``[0, key_end)``).

    A launch of fewer units than ``cu_count`` leaves CUs idle, so each unit
    is cut at multiples of ``PREFILL_PART_KEYS`` into up to
    ``min(max_parts, cu_count // units)`` parts of at least two such blocks,
    one work group each (``mv_paged_prefill_parts``). Returns
    ``[(first key, end key), ...]`` per unit; ``[(0, key_end)]`` for a unit
    that is not cut.
    """
    n = len(key_ends)
    split = max(1, min(max_parts, cu_count // n)) if 0 < n < cu_count else 1
    out = []
    for ke in key_ends:
        blocks = -(-ke // PREFILL_PART_KEYS)
        parts = max(1, min(split, blocks // 2))
        bounds = [(p * blocks // parts) * PREFILL_PART_KEYS for p in range(parts)] + [ke]
        out.append([(bounds[p], bounds[p + 1]) for p in range(parts)])
    return out


def _prefill_plan(block_table, rows, cached, qlens, block_size, num_blocks, num_q_heads,
                  num_kv_heads, head_dim, dtype, device):
    """Validated table and device work list of one step's prefill, built once:
    the layers of a step pass the same (unmodified) block table and lengths,
    so only the first call validates (one host copy of the table) and
    uploads; the others reuse it.

    Work groups are (sequence, kv head, first token, tokens), the most keys
    first; per sequence (table row, cached, first chunk row, chunk tokens).
    When the units are fewer than the CUs their keys are cut into parts
    (``prefill_key_parts``): the work groups then carry (first key, end key,
    unit, part | parts << 8 | max parts << 16) as well, and the plan its own
    workspace for the merge (counters zero). ``MVATTN_PREFILL_PARTS`` caps
    the parts per unit (1: no cut).
    """
    lib = _hip.load()
    extra = (tuple(rows), tuple(cached), tuple(qlens), block_size, num_blocks, num_q_heads,
             num_kv_heads, head_dim, dtype, device)
    hit = _cache_get("prefill", (block_table,), extra)
    if hit is not None:
        return hit
    tpg = lib.mv_prefill_tokens_per_group(num_q_heads, num_kv_heads, head_dim,
                                          _hip.MV_DTYPE[dtype])
    if tpg == 0:
        raise RuntimeError(
            f"prefill: {num_q_heads} query heads over {num_kv_heads} kv heads not supported"
        )
    bt = block_table
    if bt.dim() != 2:
        bt = bt.reshape(-1, bt.shape[-1] if bt.dim() else 0)
    if any(cached):
        _check_prefix_tables(bt.detach().to("cpu", torch.int64), rows, cached, block_size,
                             num_blocks)
    bt = bt.to(device)
    if bt.dtype not in (torch.int32, torch.int64):
        bt = bt.to(torch.int64)
    if bt.numel() and bt.stride(1) != 1:
        bt = bt.contiguous()
    seqs, items, keys = [], [], []
    start = 0
    for i, (r, c, ql) in enumerate(zip(rows, cached, qlens)):
        seqs.append((r, c, start, ql))
        for t0 in range(0, ql, tpg):
            nt = min(tpg, ql - t0)
            for h in range(num_kv_heads):
                items.append((i, h, t0, nt))
                keys.append(c + t0 + nt)
        start += ql
    cap = int(os.environ.get("MVATTN_PREFILL_PARTS", PREFILL_MAX_PARTS))
    parts = prefill_key_parts(keys, _groups_per_cu(device, head_dim, dtype)[1], cap)
    max_parts = max((len(p) for p in parts), default=1)
    split = None
    if max_parts > 1:
        groups = [(*items[u], k0, k1, u, p | len(pr) << 8 | max_parts << 16)
                  for u, pr in enumerate(parts) for p, (k0, k1) in enumerate(pr)]
        groups.sort(key=lambda g: g[4] - g[5])  # the most keys first
        work = torch.tensor(groups, dtype=torch.int32)
        ws_bytes = lib.mv_paged_prefill_workspace_bytes(len(items), max_parts, num_q_heads,
                                                        num_kv_heads, head_dim,
                                                        _hip.MV_DTYPE[dtype])
        # the plan's own merge workspace: its counters start at zero and every
        # launch leaves them so; the layers of a step share it on one stream
        split = (len(items), max_parts, torch.zeros(ws_bytes, dtype=torch.uint8, device=device))
    else:
        order = sorted(range(len(items)), key=lambda k: -keys[k])
        work = torch.tensor([items[k] for k in order] or [(0, 0, 0, 0)], dtype=torch.int32)
    meta = torch.tensor(seqs or [(0, 0, 0, 0)], dtype=torch.int64)
    plan = (bt, meta.to(device, non_blocking=True), work.to(device, non_blocking=True),
            work.shape[0] if items else 0, split)
    _cache_put("prefill", (block_table,), extra, plan)
    return plan


def _aligned_rows(x: torch.Tensor) -> torch.Tensor:
    """x with 16-byte aligned, head_dim-contiguous rows (a copy only if not)."""
    eb = x.element_size()
    st = x.stride()
    if st[-1] != 1 or (st[0] * eb) % 16 or (st[1] * eb) % 16 or x.data_ptr() % 16:
        x = x.contiguous()
    return x


def _device_i64(x, n: int, device: torch.device) -> torch.Tensor:
    """``x`` (a tensor or a sequence of ints, n entries) as a contiguous
    int64 tensor on ``device``, made by device operations only (usable while
    capturing: a host sequence becomes fill kernels, not a copy)."""
    if isinstance(x, torch.Tensor):
        if x.device != device:
            if torch.cuda.is_current_stream_capturing():
                x = x.tolist()  # a host tensor: its values are known here
            else:
                return x.to(device=device, dtype=torch.int64).contiguous()
        else:
            return x.to(torch.int64).contiguous()
    vals = [int(v) for v in x]
    assert len(vals) == n
    if vals == list(range(n)):
        return torch.arange(n, dtype=torch.int64, device=device)
    t = torch.empty(n, dtype=torch.int64, device=device)
    for i, v in enumerate(vals):
        t[i].fill_(v)
    return t


def _prefill_device_plan(block_table, seq_indices, cached_len_before, query_len, total_rows,
                         block_size, num_blocks, num_q_heads, num_kv_heads, head_dim, dtype,
                         device, capture):
    """Prefill work list built on the device (``mv_prefill_plan``) for a
    launch of fixed size: ``(bt, seqs, work, capacity)``. Used while
    capturing, where the step's lengths cannot be read back; its checks
    raise from ``check_deferred()`` (``IndexError`` "insufficient" for a
    table that cannot cover a prefix, ``ValueError`` for chunk lengths that
    exceed the query rows). Cached per capture and (unmodified) metadata."""
    lib = _hip.load()
    n = len(seq_indices)
    tensors = tuple(x for x in (block_table, cached_len_before, query_len)
                    if isinstance(x, torch.Tensor))
    extra = (tuple(int(r) for r in seq_indices), n, total_rows, block_size, num_blocks,
             num_q_heads, num_kv_heads, head_dim, dtype, device, capture,
             None if isinstance(cached_len_before, torch.Tensor) else tuple(cached_len_before),
             None if isinstance(query_len, torch.Tensor) else tuple(query_len))
    hit = _cache_get("prefill_graph", tensors, extra)
    if hit is not None:
        return hit
    tpg = lib.mv_prefill_tokens_per_group(num_q_heads, num_kv_heads, head_dim,
                                          _hip.MV_DTYPE[dtype])
    if tpg == 0:
        raise RuntimeError(
            f"prefill: {num_q_heads} query heads over {num_kv_heads} kv heads not supported"
        )
    bt = block_table
    if bt.dim() != 2:
        bt = bt.reshape(-1, bt.shape[-1] if bt.dim() else 0)
    if bt.dtype not in (torch.int32, torch.int64):
        bt = bt.to(torch.int64)
    if bt.numel() and bt.stride(1) != 1:
        bt = bt.contiguous()
    rows = _device_i64(list(seq_indices), n, device)
    cached = _device_i64(cached_len_before, n, device)
    qlen = _device_i64(query_len, n, device)
    cap = (-(-total_rows // tpg) + n) * num_kv_heads
    seqs = torch.empty(max(4 * n, 4), dtype=torch.int64, device=device)
    work = torch.empty(4 * max(cap, 1), dtype=torch.int32, device=device)
    status = torch.empty(2, dtype=torch.int32, device=device)
    _hip.check(
        lib.mv_prefill_plan(
            _ptr(rows), _ptr(cached), _ptr(qlen), n, total_rows,
            _ptr(bt) if bt.numel() else None, int(bt.dtype == torch.int64),
            bt.stride(0) if bt.numel() else 0, bt.shape[0] if bt.numel() else 0,
            bt.shape[1] if bt.numel() else 0, block_size, num_blocks, tpg, num_kv_heads,
            _ptr(seqs), _ptr(work), cap, _ptr(status), _stream(device),
        ),
        "mv_prefill_plan",
    )

    def raise_prefill(st) -> None:
        if st[0]:
            raise IndexError(
                f"prefill: {st[0]} sequence(s) with a block_table row insufficient to cover "
                f"their cached prefix (or invalid lengths)"
            )
        if st[1] < 0:
            raise ValueError(
                f"prefill: the chunk lengths exceed the {total_rows} query rows of the launch"
            )

    _defer(capture, raise_prefill, status)
    plan = (bt, seqs, work, cap)
    _cache_put("prefill_graph", tensors, extra, plan)
    return plan


def hip_prefill_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_indices: Sequence[int],
    cached_len_before,
    query_len,
    block_size: int,
) -> torch.Tensor:
    """Chunked-prefill attention over the paged pool in one HIP launch.

    The computation of ``AttentionBackendGPU.prefill_attention`` (reference
    paged_attention_gpu.py:577-661): sequence i (table row
    ``seq_indices[i]``) has ``cached_len_before[i]`` tokens in the pool and
    a chunk of ``query_len[i]`` tokens whose rows in ``query`` / ``key`` /
    ``value`` follow the previous sequences'; chunk token t attends the
    prefix from the pool and chunk keys 0..t from ``key`` / ``value``
    (causal, offset by the prefix), ``scale = head_dim ** -0.5``, query
    head h reads kv head ``h // n_rep``. Returns ``[sum(query_len), Hq, D]``
    in the query dtype. ``IndexError`` (message "insufficient") for a table
    that cannot cover a prefix, as the reference's gather raises. q / k / v
    may be column views of one fused QKV output. ``cached_len_before`` and
    ``query_len`` are sequences of ints or int tensors.

    While the current stream is being captured into a graph the lengths
    may stay on the device: the work list is then built by a device kernel
    for a launch of fixed size (``query.shape[0]`` rows, which the chunks
    must fill), and the checks raise from ``check_deferred()`` after a
    replay. ``seq_indices`` is fixed by the capture.
    """
    total_q, num_q_heads, head_dim = query.shape
    num_blocks, num_kv_heads, bs, _ = key_cache.shape
    assert bs == block_size, f"block_size {block_size} != cache dim2 {bs}"
    assert head_dim in SUPPORTED_HEAD_DIMS, f"head_dim {head_dim} not supported (only 64, 128)"
    assert _is_pow2(block_size), f"block_size {block_size} must be a power of 2"
    assert key.shape[1:] == (num_kv_heads, head_dim) and value.shape == key.shape
    assert query.dtype in SUPPORTED_DTYPES and key.dtype == query.dtype and value.dtype == query.dtype
    assert key_cache.dtype == query.dtype and value_cache.dtype == query.dtype
    assert key_cache.shape == value_cache.shape
    assert key_cache.is_contiguous() and value_cache.is_contiguous()
    assert query.device.type == "cuda"
    device = query.device
    lib = _hip.load()
    capture = _capture_id(device)
    rows = [int(r) for r in seq_indices]
    if capture:
        assert key.shape[0] >= total_q and value.shape[0] >= total_q
        out = torch.empty(total_q, num_q_heads, head_dim, dtype=query.dtype, device=device)
        if total_q == 0 or not rows:
            return out
        bt, meta, work, n_work = _prefill_device_plan(
            block_table, rows, cached_len_before, query_len, total_q, block_size, num_blocks,
            num_q_heads, num_kv_heads, head_dim, query.dtype, device, capture)
        split = None
    else:
        def host_ints(x):
            return x.tolist() if isinstance(x, torch.Tensor) else x

        cached = [int(c) for c in host_ints(cached_len_before)]
        qlens = [int(q) for q in host_ints(query_len)]
        assert len(rows) == len(cached) == len(qlens)
        total = sum(qlens)
        assert total <= total_q and total <= key.shape[0], (
            f"{total} chunk tokens, query has {total_q} rows, key {key.shape[0]}"
        )
        out = torch.empty(total, num_q_heads, head_dim, dtype=query.dtype, device=device)
        if total == 0:
            return out
        bt, meta, work, n_work, split = _prefill_plan(block_table, rows, cached, qlens,
                                                      block_size, num_blocks, num_q_heads,
                                                      num_kv_heads, head_dim, query.dtype, device)

    q = _aligned_rows(query)
    k = _aligned_rows(key)
    v = _aligned_rows(value)
    head = (_ptr(q), q.stride(0), q.stride(1), _ptr(k), k.stride(0), k.stride(1),
            _ptr(v), v.stride(0), v.stride(1), _ptr(key_cache), _ptr(value_cache),
            _ptr(bt) if bt.numel() else None, int(bt.dtype == torch.int64),
            bt.stride(0) if bt.numel() else 0, _ptr(meta), len(rows), _ptr(work), n_work)
    tail = (_ptr(out), out.stride(0), out.stride(1), float(head_dim ** -0.5), num_q_heads,
            num_kv_heads, head_dim, block_size, num_blocks, _hip.MV_DTYPE[query.dtype])
    if split is None:
        _hip.check(lib.mv_paged_prefill(*head, *tail, _stream(device)), "mv_paged_prefill")
    else:
        units, max_parts, ws = split
        _hip.check(lib.mv_paged_prefill_parts(*head, units, max_parts, *tail, _ptr(ws), ws.numel(),
                                              _stream(device)), "mv_paged_prefill_parts")
    return out


# ============================================================================
# Backend class
# ============================================================================


def _find_group(attn_metadata: Any, kind: Tuple[str, ...]):
    for g in attn_metadata.groups:
        if g.attention_type in kind:
            return g
    return None


class AttentionBackendGPU(AttentionBackend):
    """HIP backend (reference class: paged_attention_gpu.py:454-661)."""

    def __init__(self, config: ModelConfig) -> None:
        self._config = config
        self._pool: Optional[KVCachePool] = None
        self._block_size = 0
        hd = config.head_dim
        if hd not in SUPPORTED_HEAD_DIMS:
            raise RuntimeError(
                f"AttentionBackendGPU: head_dim={hd} not supported (only 64, 128). "
                f"Use the upstream reference backend for arbitrary head_dim."
            )
        if config.num_heads and config.num_kv_heads:
            n_rep = config.num_heads // config.num_kv_heads
            if config.num_heads % config.num_kv_heads or n_rep > MAX_QUERY_HEADS_PER_KV_HEAD:
                raise RuntimeError(
                    f"AttentionBackendGPU: {config.num_heads} query heads over "
                    f"{config.num_kv_heads} kv heads not supported (integer ratio <= "
                    f"{MAX_QUERY_HEADS_PER_KV_HEAD})"
                )
        if not torch.cuda.is_available():
            raise RuntimeError(
                "attention_backend='hip' requires a ROCm GPU, but none is available."
            )
        _hip.load()  # RuntimeError if the kernel library is missing

    def allocate_pool(
        self,
        num_layers: int,
        num_blocks: int,
        block_size: int,
        num_kv_heads: int,
        head_dim: int,
        dtype: torch.dtype,
        device: torch.device,
    ) -> KVCachePool:
        if not _is_pow2(block_size):
            raise RuntimeError(
                f"AttentionBackendGPU: block_size={block_size} must be a positive power of 2."
            )
        if dtype not in SUPPORTED_DTYPES:
            raise RuntimeError(f"AttentionBackendGPU: dtype {dtype} not supported")
        pool = KVCachePool.allocate(
            num_layers, num_blocks, block_size, num_kv_heads, head_dim, dtype, device
        )
        self._pool = pool
        self._block_size = block_size
        return pool

    def write_kv_cache(
        self,
        layer_idx: int,
        key: torch.Tensor,
        value: torch.Tensor,
        slot_mapping: torch.Tensor,
    ) -> None:
        pool = self._pool
        assert pool is not None, "allocate_pool must be called first"
        hip_cache_write(
            key, value, pool.key_caches[layer_idx], pool.value_caches[layer_idx],
            slot_mapping, pool.block_size,
        )

    def rope_write_kv_cache(
        self,
        layer_idx: int,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        positions: torch.Tensor,
        rope: Any,
        slot_mapping: torch.Tensor,
        return_key: bool = False,
    ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        """Fused replacement of the runner's ``q = rope(q, positions);
        k = rope(k, positions); write_kv_cache(layer, k, v, slot_mapping)``
        (reference qwen_runner.py:164-170). ``rope`` is the runner's
        ``RotaryEmbedding`` (its ``cos`` / ``sin`` tables). Returns the
        rotated query and, with ``return_key``, the rotated key (the prefill
        chunk's attention reads it)."""
        pool = self._pool
        assert pool is not None, "allocate_pool must be called first"
        return hip_rope_kv_cache_write(
            query, key, value, positions, rope.cos, rope.sin,
            pool.key_caches[layer_idx], pool.value_caches[layer_idx], slot_mapping,
            pool.block_size, return_key=return_key,
        )

    def decode_attention(
        self,
        layer_idx: int,
        query: torch.Tensor,
        attn_metadata: AttentionMetadata,
        pool: KVCachePool,
    ) -> torch.Tensor:
        if query.shape[0] == 0:
            return query
        group = _find_group(attn_metadata, ("decode_gpu",))
        if group is None:
            return query
        # Rows of decode_block_tables are decode sequences 0..B-1 in query
        # order (the runner rebases seq_indices, qwen_runner.py:213-251).
        return hip_decode_attention(
            query, pool.key_caches[layer_idx], pool.value_caches[layer_idx],
            attn_metadata.decode_block_tables, group.kv_len_after, pool.block_size,
        )

    def decode_attention_with_write(
        self,
        layer_idx: int,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        slot_mapping: torch.Tensor,
        attn_metadata: AttentionMetadata,
        pool: KVCachePool,
    ) -> torch.Tensor:
        """``write_kv_cache(layer, key, value, slot_mapping)`` of the decode
        tokens and ``decode_attention(layer, query, ...)`` in one launch
        (the runner's two calls, qwen_runner.py:168-190, for the decode
        rows). ``key`` / ``value`` / ``slot_mapping`` are the decode rows
        (``k[num_prefill:]`` ...). Output and pool are bit-identical to the
        two calls: a batch whose slots do not lie at their own sequence's
        last position, or that another sequence attends (a block shared
        without copy-on-write), is found on the device and run as the two
        calls (``hip_decode_attention``; inside a captured graph it is
        reported by ``check_deferred()``)."""
        if query.shape[0] == 0:
            return query
        group = _find_group(attn_metadata, ("decode_gpu",))
        if group is None:
            self.write_kv_cache(layer_idx, key, value, slot_mapping)
            return query
        return hip_decode_attention(
            query, pool.key_caches[layer_idx], pool.value_caches[layer_idx],
            attn_metadata.decode_block_tables, group.kv_len_after, pool.block_size,
            new_key=key, new_value=value, slot_mapping=slot_mapping,
        )

    def decode_attention_with_rope_write(
        self,
        layer_idx: int,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        positions: torch.Tensor,
        rope: Any,
        slot_mapping: torch.Tensor,
        attn_metadata: AttentionMetadata,
        pool: KVCachePool,
    ) -> torch.Tensor:
        """The whole attention sub-layer of the decode rows in one launch:
        ``q = rope(q, positions); k = rope(k, positions);
        write_kv_cache(layer, k, v, slot_mapping); decode_attention(layer,
        q, ...)`` (the runner's calls, qwen_runner.py:164-190, for the decode
        rows ``q[P:]``, ``k[P:]`` ... with their positions and slots). ``query``
        and ``key`` are not yet rotated; ``rope`` is the runner's
        ``RotaryEmbedding`` (its ``cos`` / ``sin`` tables). Output and pool
        are bit-identical to those calls."""
        if query.shape[0] == 0:
            return query
        group = _find_group(attn_metadata, ("decode_gpu",))
        if group is None:
            self.rope_write_kv_cache(layer_idx, query, key, value, positions, rope, slot_mapping)
            return query
        return hip_decode_attention(
            query, pool.key_caches[layer_idx], pool.value_caches[layer_idx],
            attn_metadata.decode_block_tables, group.kv_len_after, pool.block_size,
            new_key=key, new_value=value, slot_mapping=slot_mapping,
            positions=positions, cos=rope.cos, sin=rope.sin,
        )

    def prefill_attention(
        self,
        layer_idx: int,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        attn_metadata: AttentionMetadata,
        pool: KVCachePool,
    ) -> torch.Tensor:
        """Prefill over the pool in one HIP launch (``hip_prefill_attention``).

        Same contract as the reference's GPU prefill
        (paged_attention_gpu.py:577-661): the cached prefix comes from the
        pool, the current chunk's K/V from the arguments, and query i of a
        chunk starting at position P sees key positions <= P + i; the
        outputs of all prefill groups, in order, in one tensor.
        """
        if query.shape[0] == 0:
            return query
        groups = [g for g in attn_metadata.groups
                  if g.attention_type in ("prefill_gpu", "prefill_ref")]
        rows: List[int] = [int(s) for g in groups for s in g.seq_indices]
        if not rows:
            return query
        # Lengths stay tensors: read on the host per step (eager), or planned
        # on the device inside a captured graph. One group's tensors are
        # passed as they are, so the layers of a step share one plan.
        if len(groups) == 1:
            cached, qlens = groups[0].cached_len_before, groups[0].query_len
        else:
            cached = torch.cat([g.cached_len_before.reshape(-1) for g in groups])
            qlens = torch.cat([g.query_len.reshape(-1) for g in groups])
        return hip_prefill_attention(
            query, key, value, pool.key_caches[layer_idx], pool.value_caches[layer_idx],
            attn_metadata.prefill_block_tables, rows, cached, qlens, pool.block_size,
        )
