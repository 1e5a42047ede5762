"""mv_paged_decode_noalloc (no device allocation) against mv_paged_decode.

Both entry points run the same kernels on the same plan; the no-allocation
one keeps its split-K partials in the library's static per-GPU scratch
array instead of a caller's workspace, so the outputs must be bit-identical.
Two calls in a row, the second on a smaller batch (the array keeps the
first call's partials), each through the C ABI; device free memory is the
same before and after a call. (A batch whose merge needs more than the
array holds is rejected in host code before anything is launched: that is
tested without a GPU, in test_capi.py.)
"""

import ctypes

import pytest
import torch

from benchmarks.paged_decode_workloads import WorkloadSpec, make_case
from gpu_util import DEV, bits, say, to_device
from mini_vllm.attention import _hip
from mini_vllm.attention.paged_attention_gpu import _stream, hip_cache_write, plan_decode

pytestmark = pytest.mark.gpu


def _args(d, plan, out):
    spec = d.layout.spec
    q = d.query
    return [
        q.data_ptr(), q.stride(0), q.stride(1), d.key_cache.data_ptr(), d.value_cache.data_ptr(),
        plan.work.data_ptr(), plan.block_ids.data_ptr(), plan.block_ids.numel(), plan.num_groups,
        plan.partition_tokens, plan.max_parts, plan.counters.data_ptr(),
        out.data_ptr(), out.stride(0), out.stride(1), float(spec.head_dim ** -0.5),
        q.shape[0], spec.num_q_heads, spec.num_kv_heads, spec.head_dim, spec.block_size,
        d.key_cache.shape[0], _hip.MV_DTYPE[spec.dtype],
    ]


def _both(case):
    lib = _hip.load()
    d = to_device(case)
    spec = case.layout.spec
    # the step's new tokens first (their slots hold NaN until written)
    hip_cache_write(d.new_key, d.new_value, d.key_cache, d.value_cache, d.slot_mapping,
                    spec.block_size)
    plan = plan_decode(d.block_table, d.kv_len, spec.block_size, d.key_cache.shape[0], DEV,
                       spec.head_dim, spec.dtype, spec.num_kv_heads)
    assert plan.max_parts > 1, "the case must split sequences, so the scratch is used"
    ws_bytes = lib.mv_paged_decode_workspace_bytes(len(case.kv_len), spec.num_q_heads,
                                                   spec.head_dim, plan.max_parts)
    assert 0 < ws_bytes <= _hip.MV_DECODE_SCRATCH_BYTES
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    ref = torch.empty_like(d.query)
    got = torch.full_like(d.query, float("nan"))
    stream = _stream(torch.device("cuda", torch.cuda.current_device()))
    _hip.check(lib.mv_paged_decode(*_args(d, plan, ref), ws.data_ptr(), ws_bytes, stream),
               "mv_paged_decode")
    # the first call on the device looks the scratch address up (set-up);
    # the second is measured: it must not change the device's free memory
    got_first = torch.full_like(d.query, float("nan"))
    _hip.check(lib.mv_paged_decode_noalloc(*_args(d, plan, got_first), stream),
               "mv_paged_decode_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(bits(ref.cpu()), bits(got_first.cpu()))
    # Free device memory is a device-wide figure that another process can
    # move: a call passes when one of up to three readings around it is
    # unchanged. torch's own allocator statistics must not move at all.
    torch_before = torch.cuda.memory_stats()["allocated_bytes.all.current"]
    readings = []
    for _ in range(3):
        free_before = torch.cuda.mem_get_info()[0]
        _hip.check(lib.mv_paged_decode_noalloc(*_args(d, plan, got), stream),
                   "mv_paged_decode_noalloc")
        torch.cuda.synchronize()
        free_after = torch.cuda.mem_get_info()[0]
        readings.append((free_before, free_after))
        if free_before == free_after:
            break
    assert torch.cuda.memory_stats()["allocated_bytes.all.current"] == torch_before
    return ref, got, readings


def test_noalloc_matches_decode_on_two_calls():
    big = make_case("c2", seed=3, nan_fill=True)
    small = make_case(WorkloadSpec("noalloc-small", 14, 2, 64, 16, torch.bfloat16, 5,
                                   ("fixed", [3000, 17, 1500, 640, 2222])), seed=4, nan_fill=True)
    for tag, case in (("c2", big), ("smaller", small)):
        say("noalloc decode", tag)
        ref, got, readings = _both(case)
        assert torch.equal(bits(ref.cpu()), bits(got.cpu())), tag
        assert not torch.isnan(got.float()).any(), tag
        assert any(a == b for a, b in readings), (tag, readings)
