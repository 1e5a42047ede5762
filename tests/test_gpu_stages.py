"""Three tile stages and two give the same bits.

For 16-bit data at head_dim 64, mv_paged_decode keeps three tile buffers
per wave instead of two when a launch cuts a large batch into short
pieces (the c2 shape). The stages only change how far ahead the tiles are
copied, not the order of the arithmetic, so on the same pieces both forms
must agree bit for bit. One work list runs twice through the C ABI: with
its own piece bound (three stages) and announced with a longer bound (two
stages: the same entries, their id lists copied to that bound's stride).
"""

import pytest
import torch

from benchmarks.paged_decode_workloads import SPECS, WorkloadSpec, make_case
from gpu_util import DEV, TOL, bits, cached_case, oracle_step, say, to_device
from mini_vllm.attention import _hip
from mini_vllm.attention.paged_attention_gpu import _stream, hip_cache_write, plan_decode

pytestmark = pytest.mark.gpu


def _ids_per_item(part_tokens, block_size):
    n = (part_tokens + block_size - 1) // block_size + 1
    return (n + 3) // 4 * 4


def _decode(lib, d, spec, work, ids, num_groups, part_tokens, max_parts, counters, ws, out):
    q = d.query
    stream = _stream(torch.device("cuda", torch.cuda.current_device()))
    _hip.check(lib.mv_paged_decode(
        q.data_ptr(), q.stride(0), q.stride(1), d.key_cache.data_ptr(), d.value_cache.data_ptr(),
        work.data_ptr(), ids.data_ptr(), ids.numel(), num_groups, part_tokens, max_parts,
        counters.data_ptr(), out.data_ptr(), out.stride(0), out.stride(1),
        float(spec.head_dim ** -0.5), q.shape[0], spec.num_q_heads, spec.num_kv_heads,
        spec.head_dim, spec.block_size, d.key_cache.shape[0], _hip.MV_DTYPE[spec.dtype],
        ws.data_ptr(), ws.numel(), stream), "mv_paged_decode")


@pytest.mark.parametrize("spec", [
    SPECS["c2"],
    WorkloadSpec("stages-f16", 8, 8, 64, 32, torch.float16, 12, ("uniform", 60, 900)),
], ids=["c2", "f16-8x8"])
def test_three_and_two_stages_agree(spec):
    say("stages", spec.name)
    lib = _hip.load()
    if spec.name in SPECS:
        case, (want, _, _) = cached_case(spec.name)
    else:
        case = make_case(spec, seed=5, nan_fill=True)
        want, _, _ = oracle_step(case)
    d = to_device(case)
    bs = spec.block_size
    hip_cache_write(d.new_key, d.new_value, d.key_cache, d.value_cache, d.slot_mapping, bs)
    plan = plan_decode(d.block_table, d.kv_len, bs, d.key_cache.shape[0], DEV, spec.head_dim,
                       spec.dtype, spec.num_kv_heads)
    units = len(case.kv_len) * spec.num_kv_heads
    # the launch takes three stages: short pieces, two or more per unit, a
    # batch of at least 64 units (the library's rule)
    assert plan.partition_tokens <= 512 and plan.num_groups >= 2 * units and units >= 64, (
        plan.partition_tokens, plan.num_groups, units)
    n = plan.num_groups
    s1 = _ids_per_item(plan.partition_tokens, bs)
    long_tokens = 1024
    s2 = _ids_per_item(long_tokens, bs)
    ids2 = torch.full((n, s2), -1, dtype=torch.int32, device=DEV)
    ids2[:, :s1] = plan.block_ids[:n * s1].view(n, s1)
    ws_bytes = lib.mv_paged_decode_workspace_bytes(len(case.kv_len), spec.num_q_heads,
                                                   spec.head_dim, plan.max_parts)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
    three = torch.full_like(d.query, float("nan"))
    two = torch.full_like(d.query, float("nan"))
    _decode(lib, d, spec, plan.work, plan.block_ids, n, plan.partition_tokens, plan.max_parts,
            plan.counters, ws, three)
    _decode(lib, d, spec, plan.work, ids2, n, long_tokens, plan.max_parts, plan.counters, ws, two)
    torch.cuda.synchronize()
    assert torch.equal(bits(three.cpu()), bits(two.cpu()))
    assert (three.float().cpu() - want).abs().max().item() <= TOL[spec.dtype]
