"""The per-step decode plan (mv_decode_plan) on the GPU.

* Structure, read back from the device: every (sequence, kv head) unit is
  cut into pieces that tile [0, kv_len) exactly once, in order; the launch
  slots form a complete list; each slot's block ids are its table entries
  (-1 past its last block, to a multiple of 4); pieces respect the
  reported bounds.
* Parity on the plan's three paths: groups dealt over the CUs (one
  dispatch round), more groups than can be dealt (natural order), and a
  skewed batch whose one-round split would need oversized pieces (fair
  pieces in several rounds).
"""

import pytest
import torch

from benchmarks.paged_decode_workloads import WorkloadSpec, make_case
from gpu_util import DEV, TOL, oracle_step, say, to_device
from mini_vllm.attention.paged_attention_gpu import hip_cache_write, hip_decode_attention, plan_decode

pytestmark = pytest.mark.gpu


def _cus():
    return torch.cuda.get_device_properties(DEV).multi_processor_count


def _check_plan(case):
    spec = case.layout.spec
    bt = case.block_table.to(DEV)
    kv = case.kv_len.to(DEV)
    plan = plan_decode(bt, kv, spec.block_size, case.layout.num_blocks, DEV, spec.head_dim,
                       spec.dtype, spec.num_kv_heads)
    torch.cuda.synchronize()
    g = plan.num_groups
    work = plan.work[: 8 * g].view(g, 8).cpu().tolist()
    bs = spec.block_size
    kv_l = case.kv_len.tolist()
    table = case.block_table.tolist()
    pieces = {}
    for slot, (b, h, j, np_, t0, t1, z0, z1) in enumerate(work):
        assert 0 <= b < len(kv_l) and 0 <= h < spec.num_kv_heads and 0 <= j < np_, (slot, b, h, j, np_)
        assert (z0, z1) == (0, 0)
        assert 0 <= t0 < t1 <= kv_l[b], (slot, t0, t1, kv_l[b])
        assert t0 % 16 == 0
        assert t1 - t0 <= plan.partition_tokens
        assert np_ <= plan.max_parts
        pieces.setdefault((b, h), {})[j] = (np_, t0, t1, slot)
    for b, n in enumerate(kv_l):
        for h in range(spec.num_kv_heads):
            ps = pieces[(b, h)]
            np_ = next(iter(ps.values()))[0]
            assert sorted(ps) == list(range(np_)), (b, h, sorted(ps))
            pos = 0
            for j in range(np_):
                assert ps[j][0] == np_
                assert ps[j][1] == pos, (b, h, j, ps[j], pos)
                pos = ps[j][2]
            assert pos == n
    assert len(work) == sum(len(v) for v in pieces.values())
    # block ids per slot
    ids = plan.block_ids.cpu()
    stride = None
    for slot, (b, h, j, np_, t0, t1, _, _) in enumerate(work):
        first, last = t0 // bs, (t1 - 1) // bs
        if stride is None:
            # the stride is at least the span of the widest piece, a multiple of 4
            stride = ((plan.partition_tokens + bs - 1) // bs + 1 + 3) // 4 * 4
            assert stride * g <= ids.numel()
        # entries [0, span) are the piece's blocks, -1 fills its last group of
        # four; the decode reads nothing past that, and the plan writes nothing
        span4 = min(stride, (last - first + 1 + 3) // 4 * 4)
        row = ids[slot * stride:slot * stride + span4].tolist()
        want = [table[b][first + k] if first + k <= last else -1 for k in range(span4)]
        assert row == want, (slot, row[:8], want[:8])
    return plan


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5"])
def test_plan_structure_on_workloads(name):
    say("plan structure", name)
    case = make_case(name, seed=0)
    plan = _check_plan(case)
    spec = case.layout.spec
    units = len(case.layout.kv_lens) * spec.num_kv_heads
    assert plan.num_groups >= units


def _run_and_check(spec, seed=0):
    case = make_case(spec, seed=seed, nan_fill=True)
    plan = _check_plan(case)
    d = to_device(case)
    bs = spec.block_size
    hip_cache_write(d.new_key, d.new_value, d.key_cache, d.value_cache, d.slot_mapping, bs)
    out = hip_decode_attention(d.query, d.key_cache, d.value_cache, d.block_table, d.kv_len, bs)
    torch.cuda.synchronize()
    ref, _, _ = oracle_step(case)
    out = out.float().cpu()
    assert not torch.isnan(out).any()
    err = (out - ref).abs().max().item()
    assert err <= TOL[spec.dtype], err
    return plan, err


def test_many_units_are_not_dealt():
    """700 sequences x 2 kv heads: more work groups than one sort holds."""
    lens = [1 + (7 * i) % 40 for i in range(700)]
    spec = WorkloadSpec("many", 14, 2, 64, 16, torch.bfloat16, len(lens), ("fixed", lens))
    say("plan: many units", len(lens))
    plan, err = _run_and_check(spec)
    assert plan.num_groups > 1024
    say(f"  groups {plan.num_groups} max abs err {err:.3g}")


def test_batch_beyond_the_plan_length_cache():
    """5000 sequences (more than the 4096 lengths the plan kernel keeps in
    shared memory): lengths are read from memory in every pass, the block
    search runs over the whole work group, and the groups are not dealt."""
    lens = [1 + (13 * i) % 37 for i in range(5000)]
    spec = WorkloadSpec("huge-batch", 14, 2, 64, 16, torch.bfloat16, len(lens), ("fixed", lens))
    say("plan: 5000 sequences")
    plan, err = _run_and_check(spec)
    assert plan.num_groups >= 2 * len(lens)
    say(f"  groups {plan.num_groups} P {plan.partition_tokens} max abs err {err:.3g}")


def test_skewed_batch_uses_fair_pieces():
    """One-tile sequences filling all but 2 of the slots LDS allows (2 kv
    heads each; the plan's resident target is at most that) and one sequence
    of 16000 tokens: fitting one dispatch round would leave the long
    sequence at most one piece of 1000 tiles per kv head, far over twice the
    fair share, so the plan cuts fair pieces and runs more groups than
    resident slots."""
    from mini_vllm.attention import _hip

    per_cu = _hip.load().mv_decode_groups_per_cu(64, _hip.MV_DTYPE[torch.bfloat16])
    slots = per_cu * _cus()
    lens = [16] * (slots // 2 - 1) + [16000]
    spec = WorkloadSpec("skew", 14, 2, 64, 16, torch.bfloat16, len(lens), ("fixed", lens))
    say("plan: skewed batch", len(lens), "sequences,", slots, "slots")
    plan, err = _run_and_check(spec)
    assert plan.num_groups > slots
    say(f"  groups {plan.num_groups} P {plan.partition_tokens} max abs err {err:.3g}")


def test_dealt_plan_fills_slots_round_robin():
    """A batch that fits one round is dealt: sizes never increase within
    the first round of slots (biggest pieces first)."""
    case = make_case("c2", seed=1)
    plan = _check_plan(case)
    cus = _cus()
    g = plan.num_groups
    assert g <= 2 * cus
    work = plan.work[: 8 * g].view(g, 8).cpu()
    sizes = ((work[:, 5] - work[:, 4] + 15) // 16).tolist()  # the plan sorts by 16-token tiles
    first_round = sorted(sizes[:min(g, cus)], reverse=True)
    second = sizes[cus:]
    # every piece of the first round is at least as big as every later one
    if second:
        assert min(first_round) >= max(second)


def test_bad_entry_in_a_second_id_pass_raises():
    """Block size 1 and 16 sequences of 5000 tokens: pieces span over 300
    table entries, so a slot's id list is written in two passes of 256.
    One entry outside the pool, 300 entries into a piece (the second
    pass), is counted and raises; the same table without it runs."""
    n, kv_len, hkv = 16, 5000, 2
    pool = n * kv_len + 8
    bt = torch.arange(n * kv_len, dtype=torch.int32, device=DEV).view(n, kv_len)
    kv = torch.full((n,), kv_len, dtype=torch.int32, device=DEV)
    plan = plan_decode(bt, kv, 1, pool, DEV, 64, torch.bfloat16, hkv)
    g = plan.num_groups
    work = plan.work[: 8 * g].view(g, 8).cpu().tolist()
    long = [(w[0], w[4], w[5]) for w in work if w[5] - w[4] > 300]
    say("plan: bad entry in the second id pass,", g, "groups, P", plan.partition_tokens)
    assert long, "no piece spans over 300 table entries"
    b, t0, _ = long[0]
    q = torch.randn(n, 14, 64, device=DEV).to(torch.bfloat16)
    kc = torch.zeros(pool, hkv, 1, 64, dtype=torch.bfloat16, device=DEV)
    out = hip_decode_attention(q, kc, kc, bt, kv, 1)
    assert torch.isfinite(out.float()).all()
    bt[b, t0 + 300] = pool
    with pytest.raises(IndexError, match="pool blocks"):
        hip_decode_attention(q, kc, kc, bt, kv, 1)


@pytest.mark.parametrize("seed", range(12))
def test_small_batch_plans_on_random_shapes(seed):
    """Batches of up to 64 sequences (the wave plan, in one launch or two
    by table size) on random lengths, block sizes 1-64 and 1-8 kv heads,
    some pieces over 64 tiles (buckets wider than one tile): every unit is
    cut into pieces that tile [0, kv_len) once, the slots form a complete
    list, and the id lists are the table entries."""
    import random
    import types

    from benchmarks.paged_decode_workloads import make_layout

    rnd = random.Random(1000 + seed)
    bs = rnd.choice([1, 4, 16, 64])
    hkv = rnd.choice([1, 2, 4, 8])
    n = rnd.randint(1, 64)
    top = rnd.choice([40, 300, 2048, 6000])
    lens = [rnd.randint(1, top) for _ in range(n)]
    spec = WorkloadSpec("small-random", 8 * hkv, hkv, 64, bs, torch.bfloat16, n, ("fixed", lens))
    layout = make_layout(spec, seed)
    case = types.SimpleNamespace(layout=layout, block_table=layout.block_table(),
                                 kv_len=torch.tensor(layout.kv_lens, dtype=torch.int64))
    say("plan: random small batch", seed, n, bs, hkv, max(lens))
    plan = _check_plan(case)
    assert plan.num_groups >= n * hkv


def _plan_lists(bt, kv, bs, pool, hkv):
    plan = plan_decode(bt, kv, bs, pool, DEV, 64, torch.bfloat16, hkv)
    torch.cuda.synchronize()
    g = plan.num_groups
    stride = ((plan.partition_tokens + bs - 1) // bs + 1 + 3) // 4 * 4
    work = plan.work[: 8 * g].view(g, 8).cpu()
    ids = []
    for slot, w in enumerate(work.tolist()):
        span4 = min(stride, ((w[5] - 1) // bs - w[4] // bs + 1 + 3) // 4 * 4)
        ids.append(plan.block_ids[slot * stride:slot * stride + span4].cpu())
    return plan, work, ids


@pytest.mark.parametrize("hkv,max_kv", [(2, 2048), (16, 100)])
def test_one_launch_plan_matches_two_launches(hkv, max_kv):
    """Up to 64 sequences over a table of at most 8192 entries, the plan
    and the id lists are one launch (decode_plan_wave_kernel with its id
    groups); the same lengths over a wider table (unused columns of -1)
    take the plan kernel followed by decode_ids_kernel. Both give the same
    work list and the same id lists, dealt (2 kv heads, c2-like lengths)
    and in natural order (16 kv heads: more groups than the resident
    target); a table entry outside the pool raises on both."""
    g = torch.Generator().manual_seed(7)
    n, bs = 64, 16
    kv = torch.randint(1, max_kv + 1, (n,), generator=g, dtype=torch.int32)
    width = (max_kv + bs - 1) // bs
    pad = max(1, 8192 // n + 1 - width)  # the wide table holds over 8192 entries
    assert n * width <= 8192 < n * (width + pad)
    pool = n * width + 3
    bt = torch.randperm(pool, generator=g)[: n * width].view(n, width).to(torch.int32)
    wide = torch.cat([bt, torch.full((n, pad), -1, dtype=torch.int32)], dim=1)
    say("plan: one launch against two,", n, "sequences,", hkv, "kv heads")
    one = _plan_lists(bt.to(DEV), kv.to(DEV), bs, pool, hkv)
    two = _plan_lists(wide.to(DEV), kv.to(DEV), bs, pool, hkv)
    assert (one[0].num_groups, one[0].partition_tokens, one[0].max_parts) == \
        (two[0].num_groups, two[0].partition_tokens, two[0].max_parts)
    assert torch.equal(one[1], two[1])
    assert all(torch.equal(x, y) for x, y in zip(one[2], two[2]))
    dealt = one[0].num_groups <= 2 * _cus()
    say(f"  groups {one[0].num_groups} P {one[0].partition_tokens} dealt {dealt}")
    assert dealt == (hkv == 2)
    for table in (bt, wide):
        bad = table.clone()
        bad[5, 0] = pool
        with pytest.raises(IndexError, match="pool blocks"):
            plan_decode(bad.to(DEV), kv.to(DEV), bs, pool, DEV, 64, torch.bfloat16, hkv)


def test_write_through_dlpack_alias_needs_invalidation():
    """A length written through a DLPack alias leaves the tensor's in-place
    version unchanged, so the step's cached plan is reused as it is;
    invalidate_cached_metadata() makes the next call plan the new length."""
    from mini_vllm.attention.paged_attention_gpu import invalidate_cached_metadata

    bt = torch.arange(8, dtype=torch.int32, device=DEV).view(2, 4)
    kv = torch.tensor([40, 20], dtype=torch.int32, device=DEV)
    p1 = plan_decode(bt, kv, 16, 64, DEV, 64, torch.bfloat16, 2)
    alias = torch.from_dlpack(kv)
    alias[0] = 60
    torch.cuda.synchronize()
    assert plan_decode(bt, kv, 16, 64, DEV, 64, torch.bfloat16, 2) is p1
    invalidate_cached_metadata()
    p2 = plan_decode(bt, kv, 16, 64, DEV, 64, torch.bfloat16, 2)
    assert p2 is not p1
    g = p2.num_groups
    work = p2.work[: 8 * g].view(g, 8).cpu().tolist()
    ends = {(w[0], w[1]): max(x[5] for x in work if (x[0], x[1]) == (w[0], w[1])) for w in work}
    assert ends[(0, 0)] == 60 and ends[(1, 0)] == 20, ends


def _smallest_fitting_bound(kv_lens, hkv, bs, groups_per_cu, cus):
    """The plan's piece bound L (16-token tiles) from its rules, by brute
    force: the smallest L from the search's lower end whose groups fit the
    resident target, the fair share when even the widest L does not fit
    (several rounds), and twice the fair share when the fitting L is over
    that (skewed batches)."""
    tiles = [(k + 15) // 16 for k in kv_lens if k >= 1]
    units = len(tiles) * hkv
    total, most = sum(tiles), max(tiles)
    per_cu = min(2, max(1, groups_per_cu)) if units <= cus else min(3, max(1, groups_per_cu))
    target = per_cu * max(1, cus)
    l_cap = max(1, ((512 - 1) * bs) // 16)
    l_min = min(l_cap, max(4, -(-most // 128)))
    l_top = min(l_cap, max(l_min, most))
    l_fair = min(l_cap, max(l_min, -(-(total * hkv) // target)))

    def groups(l):
        return hkv * sum(-(-t // l) for t in tiles)

    if groups(l_top) > target:
        return l_fair
    l = min(l_fair, l_top)
    while groups(l) > target:
        l += 1
    return max(l_min, min(l_cap, 2 * l_fair)) if l > 2 * l_fair else l


@pytest.mark.parametrize("batch,hkv,ctx,seed", [
    (64, 2, ("uniform", 128, 2048), 0),     # the c2 shape (one launch, waves)
    (16, 8, ("uniform", 8192, 32768), 1),   # long contexts (waves, then the id kernel)
    (65, 2, ("uniform", 16, 4000), 2),      # the 1024-thread plan from here on
    (128, 4, ("uniform", 512, 4096), 3),
    (200, 1, ("lognormal", 300, 1.0, 1, 8192), 4),
    (256, 2, ("lognormal", 300, 1.0, 1, 8192), 5),
    (300, 2, ("uniform", 1, 3000), 6),      # past the one-wave search: block sums
    (1000, 8, ("uniform", 1, 600), 7),
])
def test_piece_bound_is_the_smallest_that_fits(batch, hkv, ctx, seed):
    """Both plan kernels search the piece bound (the wave plan up to 64
    sequences, the 1024-thread plan above: one wave's binary search up to
    256 sequences, block sums past that); the bound they return must be the
    one the rules define, and the groups the ones it cuts."""
    from benchmarks.paged_decode_workloads import make_layout
    from mini_vllm.attention import paged_attention_gpu as pag

    spec = WorkloadSpec("bound", 2 * hkv, hkv, 64, 16, torch.bfloat16, batch, ctx)
    lay = make_layout(spec, seed)
    say("plan bound", batch, hkv, ctx, seed)
    bt = lay.block_table().to(DEV)
    kv = torch.tensor(lay.kv_lens, dtype=torch.int64, device=DEV)
    plan = plan_decode(bt, kv, 16, lay.num_blocks, DEV, 64, torch.bfloat16, hkv)
    gpc, cus = pag._groups_per_cu(DEV, 64, torch.bfloat16)
    want = _smallest_fitting_bound(lay.kv_lens, hkv, 16, gpc, cus)
    assert plan.partition_tokens == 16 * want, (plan.partition_tokens, 16 * want)
    tiles = [(k + 15) // 16 for k in lay.kv_lens]
    assert plan.num_groups == hkv * sum(-(-t // want) for t in tiles)
