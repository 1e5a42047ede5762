"""Paged decode on the GPU against the oracle (fp32 torch restatement of
AttentionBackendRef.decode_attention) on identical inputs.

Tolerances (max-abs, against the fp32 oracle run on the kernel's own
rounded inputs): fp32 1e-5, bf16 2e-2, fp16 1e-2. Pools are NaN outside
the attended tokens, so a read past kv_len or a missing KV write shows up
as NaN.
"""

import pytest
import torch

from benchmarks.paged_decode_workloads import SPECS, WorkloadSpec, make_case
from gpu_util import DEV, TOL, bits, cached_case, oracle_step, say, to_device
from mini_vllm.attention import AttentionBackend
from mini_vllm.attention.paged_attention_gpu import (
    gather_prefix_kv,
    hip_cache_write,
    hip_decode_attention,
    triton_decode_attention,
)
from mini_vllm.model_runner.base import AttentionGroup, AttentionMetadata, ModelConfig
from oracle import paged_ref

pytestmark = pytest.mark.gpu


def _step_on_gpu(case, dtype=None):
    d = to_device(case)
    bs = case.layout.spec.block_size
    hip_cache_write(d.new_key, d.new_value, d.key_cache, d.value_cache, d.slot_mapping, bs)
    out = hip_decode_attention(d.query, d.key_cache, d.value_cache, d.block_table, d.kv_len, bs)
    torch.cuda.synchronize()
    return out.float().cpu(), d


def _check(out, ref, dtype, what):
    assert not torch.isnan(out).any(), f"{what}: NaN in output"
    err = (out - ref).abs().max().item()
    assert err <= TOL[dtype], f"{what}: max abs err {err} > {TOL[dtype]}"
    return err


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5"])
def test_workload_matches_oracle(name):
    say("decode workload", name)
    case, (ref, _, _) = cached_case(name)
    out, _ = _step_on_gpu(case)
    err = _check(out, ref, SPECS[name].dtype, name)
    say(f"  {name} max abs err {err:.3g}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("name", ["c2", "c5"])
def test_workload_other_dtypes(name, dtype):
    say("decode workload", name, dtype)
    case, (ref, _, _) = cached_case(name, dtype=dtype)
    out, _ = _step_on_gpu(case)
    _check(out, ref, dtype, f"{name}/{dtype}")


def test_c1_golden_fixture():
    """fp32 at 1e-5 against the committed c1 fixture (write + decode)."""
    import os

    import numpy as np

    say("decode golden c1")
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "c1_decode.npz"))
    kc_post = torch.from_numpy(z["key_cache"])
    vc_post = torch.from_numpy(z["value_cache"])
    slots = torch.from_numpy(z["slot_mapping"])
    kc, vc = kc_post.clone(), vc_post.clone()
    for s in slots.tolist():  # the slots the write fills were NaN before it
        kc[s // 16, :, s % 16] = float("nan")
        vc[s // 16, :, s % 16] = float("nan")
    kd, vd = kc.to(DEV), vc.to(DEV)
    hip_cache_write(torch.from_numpy(z["new_key"]).to(DEV), torch.from_numpy(z["new_value"]).to(DEV),
                    kd, vd, slots.to(DEV), 16)
    out = hip_decode_attention(torch.from_numpy(z["query"]).to(DEV), kd, vd,
                               torch.from_numpy(z["block_table"]).to(DEV),
                               torch.from_numpy(z["kv_len"]).to(DEV), 16)
    torch.cuda.synchronize()
    assert torch.equal(bits(kd.cpu()), bits(kc_post)) and torch.equal(bits(vd.cpu()), bits(vc_post))
    err = (out.cpu() - torch.from_numpy(z["out"])).abs().max().item()
    assert err <= 1e-5, err


def _random_case(hq, hkv, d, bs, lens, dtype, seed, table_dtype=torch.int64, len_dtype=torch.int64):
    spec = WorkloadSpec("t", hq, hkv, d, bs, dtype, len(lens), ("fixed", list(lens)))
    c = make_case(spec, seed=seed, nan_fill=True)
    c.block_table = c.block_table.to(table_dtype)
    c.kv_len = c.kv_len.to(len_dtype)
    return c


LENS = [1, 2, 15, 16, 17, 255, 256, 257, 511, 513, 1000]


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 4), (14, 2), (16, 1), (28, 4), (12, 1), (6, 2)])
@pytest.mark.parametrize("d", [64, 128])
def test_group_sizes(hq, hkv, d):
    for dtype in (torch.bfloat16, torch.float32):
        say("decode groups", hq, hkv, d, dtype)
        c = _random_case(hq, hkv, d, 16, LENS, dtype, seed=hq * 7 + d)
        ref, _, _ = oracle_step(c)
        out, _ = _step_on_gpu(c)
        _check(out, ref, dtype, f"hq={hq} hkv={hkv} d={d} {dtype}")


@pytest.mark.parametrize("bs", [1, 2, 8, 32, 64, 256])
def test_block_sizes(bs):
    for dtype in (torch.float16, torch.float32):
        say("decode block size", bs, dtype)
        c = _random_case(14, 2, 64, bs, LENS, dtype, seed=bs)
        ref, _, _ = oracle_step(c)
        out, _ = _step_on_gpu(c)
        _check(out, ref, dtype, f"bs={bs} {dtype}")


def test_int32_metadata():
    """int32 block tables and kv_len (the reference's GPU tests pass int32
    kv_len_after, test_paged_attention_gpu.py:268)."""
    say("decode int32 metadata")
    c = _random_case(14, 2, 64, 16, LENS, torch.bfloat16, 3, torch.int32, torch.int32)
    ref, _, _ = oracle_step(c)
    out, _ = _step_on_gpu(c)
    _check(out, ref, torch.bfloat16, "int32 metadata")


def _ramp(shape, base, dtype=torch.float16):
    n = 1
    for s in shape:
        n *= s
    return (base + torch.arange(n, dtype=torch.float32)).view(*shape).to(dtype)


@pytest.mark.parametrize("lens,qh", [([7], 4), ([10, 15], 4), ([3, 23], 4), ([19], 4), ([40], 4),
                                     ([16] * 4, 4), ([32] * 8, 4), ([5, 17, 32, 50], 4),
                                     ([1, 3, 7, 15, 16, 17, 31, 32], 4), ([8, 24], 8)])
def test_reference_gpu_suite_ramp_inputs(lens, qh):
    """The reference GPU suite's cases (test_paged_attention_gpu.py:263-687):
    fp16, block 16, ramp inputs base + i (near one-hot softmax), sequence
    i at slots i*512.., compared at atol = rtol = 1e-2 as there."""
    say("decode ramp", lens, qh)
    bs, hkv, d = 16, 2, 64
    kc = torch.full((512, hkv, bs, d), float("nan"), dtype=torch.float16)
    vc = kc.clone()
    rows = []
    for i, n in enumerate(lens):
        slots = torch.arange(i * 512, i * 512 + n)
        paged_ref.write_to_paged_cache(_ramp((n, hkv, d), 10.0 + i * 100),
                                       _ramp((n, hkv, d), 1010.0 + i * 100), kc, vc, slots, bs)
        rows.append(list(range(i * 32, i * 32 + -(-n // bs))))
    mb = max(len(r) for r in rows)
    bt = torch.tensor([r + [-1] * (mb - len(r)) for r in rows])
    kv = torch.tensor(lens, dtype=torch.int32)
    q = _ramp((len(lens), qh, d), 50.0)
    ref = paged_ref.decode_from_tables(q.float(), kc.float(), vc.float(), bt, kv, bs)
    out = triton_decode_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), kv.to(DEV), bs)
    assert torch.allclose(out.float().cpu(), ref, atol=1e-2, rtol=1e-2)


def _split_ranges(lens, first, gap):
    """Sequence i holds min(n, first) tokens from slot i*512 and the rest from
    slot i*512 + gap, written in sequence order (a later sequence may
    overwrite an earlier one's second range, as in the reference's own
    setup); returns (kc, vc, table)."""
    bs, hkv, d = 16, 2, 64
    kc = torch.full((512, hkv, bs, d), float("nan"), dtype=torch.float16)
    vc = kc.clone()
    rows = []
    for i, n in enumerate(lens):
        k = _ramp((n, hkv, d), 10.0 + i * 100)
        v = _ramp((n, hkv, d), 1010.0 + i * 100)
        a = min(n, first)
        row = []
        for lo, hi, s0 in ((0, a, i * 512), (a, n, i * 512 + gap)):
            if hi > lo:
                paged_ref.write_to_paged_cache(k[lo:hi], v[lo:hi], kc, vc,
                                               torch.arange(s0, s0 + hi - lo), bs)
                row += list(range(s0 // bs, s0 // bs + -(-(hi - lo) // bs)))
        rows.append(row)
    mb = max(len(r) for r in rows)
    return kc, vc, torch.tensor([r + [-1] * (mb - len(r)) for r in rows])


@pytest.mark.parametrize("lens,gap", [([32] * 4, 256), ([7, 19, 33, 48], 512)])
def test_reference_gpu_suite_split_ranges(lens, gap):
    """Each sequence's blocks in two separate ranges of the pool
    (test_paged_attention_gpu.py:562-646: batch 4 non-contiguous, batch 4
    ragged non-contiguous); fp16 ramp inputs, atol = rtol = 1e-2 as there."""
    say("decode split ranges", lens, gap)
    kc, vc, bt = _split_ranges(lens, 16, gap)
    kv = torch.tensor(lens, dtype=torch.int32)
    q = _ramp((len(lens), 4, 64), 50.0)
    ref = paged_ref.decode_from_tables(q.float(), kc.float(), vc.float(), bt, kv, 16)
    out = triton_decode_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), kv.to(DEV), 16)
    assert torch.allclose(out.float().cpu(), ref, atol=1e-2, rtol=1e-2)


def test_noncontiguous_table_10_50():
    """Table [[10, 50]] with 19 tokens (test_paged_attention_gpu.py:357-381)."""
    say("decode [[10,50]]")
    kc = torch.full((64, 2, 16, 64), float("nan"), dtype=torch.float16)
    vc = kc.clone()
    paged_ref.write_to_paged_cache(_ramp((16, 2, 64), 10.0), _ramp((16, 2, 64), 1000.0), kc, vc,
                                   torch.arange(160, 176), 16)
    paged_ref.write_to_paged_cache(_ramp((3, 2, 64), 50.0), _ramp((3, 2, 64), 5000.0), kc, vc,
                                   torch.arange(800, 803), 16)
    q = _ramp((1, 4, 64), 99.0)
    bt = torch.tensor([[10, 50]])
    kv = torch.tensor([19], dtype=torch.int32)
    ref = paged_ref.decode_from_tables(q.float(), kc.float(), vc.float(), bt, kv, 16)
    out = hip_decode_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), kv.to(DEV), 16)
    assert torch.allclose(out.float().cpu(), ref, atol=1e-2, rtol=1e-2)


def test_split_merges_in_a_row_are_deterministic():
    """Sequences split into many partitions, several calls in a row with
    different layouts (batch, partitions per sequence): each matches the
    oracle and is bit-identical when repeated (the partials are merged in
    partition order, whichever work group merges)."""
    for seed, lens, dtype in ((31, [4000, 40, 9000, 700], torch.bfloat16),
                              (32, [20000, 3], torch.float32),
                              (33, [900] * 24 + [5000], torch.float16)):
        say("decode split merges", seed, lens, dtype)
        c = _random_case(14, 2, 64, 16, lens, dtype, seed)
        ref, _, _ = oracle_step(c)
        out, _ = _step_on_gpu(c)
        _check(out, ref, dtype, f"split merges seed {seed}")
        again, _ = _step_on_gpu(c)  # whichever work group merges, the same bits
        assert torch.equal(bits(out), bits(again))
        _assert_counters_at_rest(c)


def _assert_counters_at_rest(c):
    """Every merge put its (sequence, kv head) counter back to zero: the
    plan's counters are zero between calls, as the next call of the step
    (which does not replan) needs them."""
    from mini_vllm.attention import paged_attention_gpu as pg

    d = to_device(c)
    spec = c.layout.spec
    plan = pg.plan_decode(d.block_table, d.kv_len, spec.block_size, d.key_cache.shape[0], DEV,
                          spec.head_dim, spec.dtype, spec.num_kv_heads)
    for _ in range(2):
        hip_decode_attention(d.query, d.key_cache, d.value_cache, d.block_table, d.kv_len,
                             spec.block_size)
        torch.cuda.synchronize()
        # the call ran on this plan (the same cached object)
        assert pg.plan_decode(d.block_table, d.kv_len, spec.block_size, d.key_cache.shape[0], DEV,
                              spec.head_dim, spec.dtype, spec.num_kv_heads) is plan
        assert int(torch.count_nonzero(plan.counters)) == 0


def test_block_size_one_long_id_lists():
    """Block size 1 with many long sequences: pieces of up to 496 tokens
    span up to 497 table entries, more than the 256 the first id copy
    holds, so each work group fetches the rest of its list once the work
    item is known."""
    from mini_vllm.attention.paged_attention_gpu import plan_decode

    say("decode block size 1, long id lists")
    c = _random_case(14, 2, 64, 1, [900 + (7 * i) % 200 for i in range(300)], torch.bfloat16, 41)
    ref, _, _ = oracle_step(c)
    out, d = _step_on_gpu(c)
    plan = plan_decode(d.block_table, d.kv_len, 1, d.key_cache.shape[0], d.key_cache.device, 64,
                       torch.bfloat16, 2)
    assert plan.partition_tokens + 1 > 256, plan.partition_tokens  # the second copy ran
    _check(out, ref, torch.bfloat16, "block size 1")


def test_invalid_metadata_raises():
    say("decode invalid metadata")
    q = torch.randn(1, 4, 64).half().to(DEV)
    kc = torch.zeros(8, 2, 16, 64, dtype=torch.float16, device=DEV)
    with pytest.raises(ValueError, match="kv_len"):
        hip_decode_attention(q, kc, kc, torch.full((1, 1), -1, device=DEV),
                             torch.tensor([0], dtype=torch.int32, device=DEV), 16)
    with pytest.raises(IndexError, match="insufficient"):
        hip_decode_attention(q, kc, kc, torch.tensor([[0]], device=DEV),
                             torch.tensor([17], device=DEV), 16)
    with pytest.raises(IndexError, match="pool blocks"):
        hip_decode_attention(q, kc, kc, torch.tensor([[0, -1, 2]], device=DEV),
                             torch.tensor([40], device=DEV), 16)
    with pytest.raises(IndexError, match="pool blocks"):
        hip_decode_attention(q, kc, kc, torch.tensor([[8]], device=DEV),
                             torch.tensor([4], device=DEV), 16)


def test_padding_after_needed_blocks_is_ignored():
    say("decode padding")
    c = _random_case(14, 2, 64, 16, [5, 40], torch.bfloat16, 11)
    c.block_table = torch.cat([c.block_table, torch.full((2, 3), -1)], dim=1)
    ref, _, _ = oracle_step(c)
    out, _ = _step_on_gpu(c)
    _check(out, ref, torch.bfloat16, "padded table")


def test_plan_reused_and_refreshed():
    """Same metadata tensors -> cached plan; in-place edit -> new plan."""
    say("decode plan cache")
    c = _random_case(14, 2, 64, 16, [300, 40, 700], torch.bfloat16, 12)
    d = to_device(c)
    bs = 16
    hip_cache_write(d.new_key, d.new_value, d.key_cache, d.value_cache, d.slot_mapping, bs)
    a = hip_decode_attention(d.query, d.key_cache, d.value_cache, d.block_table, d.kv_len, bs)
    b = hip_decode_attention(d.query, d.key_cache, d.value_cache, d.block_table, d.kv_len, bs)
    assert torch.equal(a, b)
    d.kv_len[1] = 20  # still covered by the table, slots before 40 are live
    e = hip_decode_attention(d.query, d.key_cache, d.value_cache, d.block_table, d.kv_len, bs)
    ref = paged_ref.decode_from_tables(d.query.float().cpu(), d.key_cache.float().cpu(),
                                       d.value_cache.float().cpu(), c.block_table, d.kv_len.cpu(), bs)
    _check(e.float().cpu(), ref, torch.bfloat16, "refreshed plan")


def test_strided_query_view():
    """Query as the decode rows of a larger [T, Hq, D] tensor (runner passes
    q[num_prefill:], qwen_runner.py:185-190)."""
    say("decode strided query")
    c = _random_case(14, 2, 64, 16, [33, 300], torch.bfloat16, 13)
    ref, _, _ = oracle_step(c)
    d = to_device(c)
    big = torch.randn(5, 14, 64, device=DEV).to(torch.bfloat16)
    big[3:] = d.query
    hip_cache_write(d.new_key, d.new_value, d.key_cache, d.value_cache, d.slot_mapping, 16)
    out = hip_decode_attention(big[3:], d.key_cache, d.value_cache, d.block_table, d.kv_len, 16)
    _check(out.float().cpu(), ref, torch.bfloat16, "strided query")


def test_empty_batch():
    q = torch.empty(0, 14, 64, dtype=torch.bfloat16, device=DEV)
    kc = torch.zeros(4, 2, 16, 64, dtype=torch.bfloat16, device=DEV)
    out = hip_decode_attention(q, kc, kc, torch.empty(0, 1, dtype=torch.long, device=DEV),
                               torch.empty(0, dtype=torch.long, device=DEV), 16)
    assert out.shape == (0, 14, 64)


# -------------------------------------------------------------- backend --


def _meta(bt, cached):
    g = AttentionGroup(list(range(len(cached))), "decode_gpu", cached,
                       torch.ones_like(cached), cached + 1)
    return AttentionMetadata(groups=[g], decode_block_tables=bt, block_size=16)


def test_backend_runner_sequence_three_layers():
    """The runner's per-layer order (qwen_runner.py:150-197): write the step's
    K/V with slot_mapping, then decode from the pool, for several layers of
    one pool with different data per layer."""
    say("backend runner sequence")
    spec = SPECS["c2"]
    cfg = ModelConfig(num_layers=3, num_heads=14, num_kv_heads=2, head_dim=64, dtype=torch.bfloat16)
    be = AttentionBackend.create(cfg, backend="hip")
    assert type(be).__name__ == "AttentionBackendGPU"
    assert type(AttentionBackend.create(cfg, backend="triton")) is type(be)
    base = make_case(spec, seed=0, nan_fill=True)
    lay = base.layout  # one block manager: the same tables for every layer
    pool = be.allocate_pool(3, lay.num_blocks, 16, 2, 64, torch.bfloat16, DEV)
    meta = _meta(base.block_table.to(DEV), base.kv_len.to(DEV) - 1)
    slots = base.slot_mapping.to(DEV)
    layers = []
    for layer in range(3):  # per-layer values: shifted/scaled copies (NaN stays NaN)
        c = make_case(spec, seed=0, nan_fill=True)
        c.key_cache = (c.key_cache.float() * (1 + 0.5 * layer)).to(torch.bfloat16)
        c.value_cache = (c.value_cache.float() + layer).to(torch.bfloat16)
        c.new_key = (c.new_key.float() - layer).to(torch.bfloat16)
        c.new_value = (c.new_value.float() * (1 + layer)).to(torch.bfloat16)
        pool.key_caches[layer].copy_(c.key_cache.to(DEV))
        pool.value_caches[layer].copy_(c.value_cache.to(DEV))
        layers.append(c)
    for layer, c in enumerate(layers):
        be.write_kv_cache(layer, c.new_key.to(DEV), c.new_value.to(DEV), slots)
        out = be.decode_attention(layer, c.query.to(DEV), meta, pool)
        ref, _, _ = oracle_step(c)
        _check(out.float().cpu(), ref, torch.bfloat16, f"layer {layer}")


def test_backend_no_decode_group_and_empty_query():
    cfg = ModelConfig(num_heads=14, num_kv_heads=2, head_dim=64)
    be = AttentionBackend.create(cfg, backend="hip")
    pool = be.allocate_pool(1, 16, 16, 2, 64, torch.bfloat16, DEV)
    q = torch.randn(2, 14, 64, device=DEV).to(torch.bfloat16)
    assert be.decode_attention(0, q, AttentionMetadata(), pool) is q
    e = q[:0]
    assert be.decode_attention(0, e, _meta(torch.zeros(0, 1, dtype=torch.long), torch.zeros(0, dtype=torch.long)), pool) is e
    with pytest.raises(RuntimeError, match="block_size"):
        be.allocate_pool(1, 16, 12, 2, 64, torch.bfloat16, DEV)


def test_gather_prefix_matches_oracle_gather():
    """gather_prefix_kv (reference :391-446) against the oracle gather,
    including table [[10, 50]] and an empty prefix."""
    say("gather prefix")
    g = torch.Generator().manual_seed(21)
    kc = torch.randn(64, 2, 16, 64, generator=g).half()
    vc = torch.randn(64, 2, 16, 64, generator=g).half()
    bt = torch.tensor([[10, 50, -1], [3, 4, 5], [7, -1, -1]])
    lens, rows = [20, 40, 0], [0, 1, 2]
    k, v = gather_prefix_kv(kc.to(DEV), vc.to(DEV), bt.to(DEV), lens, rows, 16)
    ks, vs = [], []
    for r, n in zip(rows, lens):
        ids = [b for b in bt[r].tolist() if b != -1]
        a, b = paged_ref.gather_paged_kv(kc, vc, ids, n, 16)
        ks.append(a)
        vs.append(b)
    assert torch.equal(k.cpu(), torch.cat(ks)) and torch.equal(v.cpu(), torch.cat(vs))
    with pytest.raises(IndexError, match="insufficient"):
        gather_prefix_kv(kc.to(DEV), vc.to(DEV), bt.to(DEV), [60], [0], 16)


def test_backend_prefill_matches_oracle_prefill():
    """prefill_attention: cached prefix from the pool + chunk K/V, offset
    causal mask (reference paged_attention_ref.py:167-244)."""
    say("backend prefill")
    cfg = ModelConfig(num_heads=8, num_kv_heads=2, head_dim=64)
    be = AttentionBackend.create(cfg, backend="hip")
    pool = be.allocate_pool(1, 32, 4, 2, 64, torch.float32, DEV)
    g = torch.Generator().manual_seed(22)
    cached, qlens, rows = [0, 8, 5], [4, 2, 3], [[0, -1, -1], [4, 5, 6], [9, 2, -1]]
    kc = torch.randn(32, 2, 4, 64, generator=g)
    vc = torch.randn(32, 2, 4, 64, generator=g)
    total = sum(qlens)
    q = torch.randn(total, 8, 64, generator=g)
    k = torch.randn(total, 2, 64, generator=g)
    v = torch.randn(total, 2, 64, generator=g)
    slots, off = [], 0
    for r, c, ql in zip(rows, cached, qlens):
        for p in range(c, c + ql):
            slots.append(r[p // 4] * 4 + p % 4)
    paged_ref.write_to_paged_cache(k, v, kc, vc, torch.tensor(slots), 4)  # write-first
    pool.key_caches[0].copy_(kc.to(DEV))
    pool.value_caches[0].copy_(vc.to(DEV))
    grp = AttentionGroup([0, 1, 2], "prefill_gpu", torch.tensor(cached), torch.tensor(qlens),
                         torch.tensor(cached) + torch.tensor(qlens))
    meta = AttentionMetadata(groups=[grp], prefill_block_tables=torch.tensor(rows).to(DEV), block_size=4)
    out = be.prefill_attention(0, q.to(DEV), k.to(DEV), v.to(DEV), meta, pool)
    ref = paged_ref.prefill_attention(q, kc, vc, torch.tensor(rows), [0, 1, 2], cached, qlens, 4)
    assert (out.cpu() - ref).abs().max().item() < 1e-5


# ---- the softmax reference: tiles kept as computed, or redone exactly

SHARP_LENS = [1, 17, 300, 1000, 2048]


def _sharp_case(dtype, seed):
    return _random_case(14, 2, 64, 16, SHARP_LENS, dtype, seed=seed)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=str)
@pytest.mark.parametrize("d", [64, 128])
def test_sharp_scores(dtype, d):
    """Q x 4: tile sums leave [2^-12, 2^12], so those tiles are computed
    exactly (reference moved, O rescaled)."""
    say("decode sharp scores", dtype, d)
    c = _random_case(14, 2, d, 16, SHARP_LENS, dtype, seed=21)
    c.query = (c.query.float() * 4).to(c.query.dtype)
    ref, _, _ = oracle_step(c)
    out, _ = _step_on_gpu(c)
    say("  max abs err", _check(out, ref, dtype, f"sharp {dtype}"))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_late_key_with_a_far_higher_score(dtype):
    """Keys of each sequence's sixth block (tokens 80-95) x 12: their tile
    overflows the range, the reference moves up by tens of units, and later
    tiles are kept as computed again (sums far below 1, l above)."""
    say("decode late high key", dtype)
    c = _sharp_case(dtype, seed=22)
    kc = c.key_cache.float()
    for b, n in enumerate(c.kv_len.tolist()):
        if n > 96:
            blk = int(c.block_table[b, 5])
            kc[blk] = kc[blk] * 12
    c.key_cache = kc.to(c.key_cache.dtype)
    ref, _, _ = oracle_step(c)
    out, _ = _step_on_gpu(c)
    say("  max abs err", _check(out, ref, dtype, f"late key {dtype}"))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_scores_far_below_zero(dtype):
    """Every score near -60 in the exponent's units: the first tile's sums
    fall below 2^-12 and are computed exactly, which moves the reference
    down to the head's maximum."""
    say("decode negative scores", dtype)
    c = _sharp_case(dtype, seed=23)
    c.query = (c.query.float().abs() * 2 + 1).to(c.query.dtype)
    c.key_cache = (-(c.key_cache.float().abs() * 2 + 1)).to(c.key_cache.dtype)
    c.new_key = (-(c.new_key.float().abs() * 2 + 1)).to(c.new_key.dtype)
    ref, _, _ = oracle_step(c)
    out, _ = _step_on_gpu(c)
    say("  max abs err", _check(out, ref, dtype, f"negative {dtype}"))
