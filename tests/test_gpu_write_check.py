"""The fused write+decode's precondition check (mv_decode_write_check) and
the O(T) slot check (mv_kv_slots_check), through the C ABI.

The fused launch (mv_paged_decode_write) is exact only when no table entry
of the batch reads a slot the call writes, other than each sequence's own
slot at its own last position. The reference's block manager can break
that: its prefix cache registers a prompt's partial last block and a later
identical prompt shares it, with no copy-on-write in ensure_block
(reference mini_vllm/cache/prefix_cache.py:42-51, cache/manager.py:140-172,
218-225). Then one sequence's decode slot lies in a block another sequence
attends. The two calls of the reference's runner (qwen_runner.py:168-190)
write first and read after; the fused launch would read a pool row while
another work group rewrites it.

Both status words are checked against a brute force written from their
definitions (a loop over every writer for every table entry, not the
kernel's per-block minimum), on layouts with shared blocks, repeated
blocks, duplicate slots, off-table and -1 slots; then the backend's fused
call on the prefix-cache layout is checked to run as the two calls, eager,
and to be reported by check_deferred() when captured.
"""

import ctypes

import numpy as np
import pytest
import torch

from benchmarks.paged_decode_workloads import make_case
from gpu_util import DEV, bits, say
from mini_vllm.attention import _hip
from mini_vllm.attention import paged_attention_gpu as pg

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None and t.numel() else None


def brute_counts(slots, bt, kv, bs):
    """(own-slot failures, shared-read entries) by definition."""
    slots, bt, kv = (np.asarray(x, dtype=np.int64) for x in (slots, bt, kv))
    nseq, max_blocks = bt.shape
    own_bad = 0
    by_block = {}  # block -> [(writer, offset)]
    for b in range(nseq):
        s = int(slots[b])
        if s == -1:
            continue
        k = int(kv[b])
        e = (k - 1) // bs
        ok = k >= 1 and e < max_blocks
        if ok:
            blk = int(bt[b, e])
            ok = 0 <= blk < 0xFFFFFFFF and s == blk * bs + (k - 1) % bs
        if not ok:
            own_bad += 1
            continue
        by_block.setdefault(s // bs, []).append((b, s % bs))
    shared = 0
    for c in range(nseq):
        k = int(kv[c])
        if k < 1:
            continue
        n = min((k + bs - 1) // bs, max_blocks)
        e_c = (k - 1) // bs
        for j in range(n):
            lim = min(bs, k - j * bs)
            for w, off in by_block.get(int(bt[c, j]), ()):
                if off < lim and not (w == c and j == e_c):
                    shared += 1
                    break
    return own_bad, shared


def device_counts(slots, bt, kv, bs):
    lib = _hip.load()
    slots = torch.as_tensor(slots, dtype=torch.int64).to(DEV)
    bt, kv = bt.to(DEV), kv.to(DEV)
    n = kv.shape[0]
    status = torch.full((2,), -7, dtype=torch.int32, device=DEV)
    nbytes = lib.mv_decode_write_check_workspace_bytes(n)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _hip.check(lib.mv_decode_write_check(
        _ptr(slots), _ptr(bt), int(bt.dtype == torch.int64), bt.stride(0), _ptr(kv),
        int(kv.dtype == torch.int64), n, bt.shape[1], bs, _ptr(status), _ptr(ws), nbytes,
        stream), "mv_decode_write_check")
    torch.cuda.synchronize()
    return tuple(status.tolist())


def shared_layout(seed, nseq, bs, max_blocks, pool_blocks):
    """Tables drawn from a small pool (blocks shared and repeated), slots
    mostly at each sequence's own last position, some -1, some elsewhere,
    some duplicated."""
    g = np.random.default_rng(seed)
    kv = g.integers(1, max_blocks * bs + 1, size=nseq)
    bt = np.full((nseq, max_blocks), -1, dtype=np.int64)
    for b in range(nseq):
        n = (kv[b] + bs - 1) // bs
        bt[b, :n] = g.integers(0, pool_blocks, size=n)
    last = kv - 1
    slots = bt[np.arange(nseq), last // bs] * bs + last % bs
    r = g.random(nseq)
    slots[r < 0.1] = -1
    elsewhere = (r >= 0.1) & (r < 0.15)
    slots[elsewhere] = g.integers(0, pool_blocks * bs, size=int(elsewhere.sum()))
    dup = g.integers(0, nseq, size=max(1, nseq // 50))
    slots[dup] = slots[g.integers(0, nseq, size=dup.size)]
    return slots, bt, kv


@pytest.mark.parametrize("seed,nseq,bs,max_blocks,pool", [
    (0, 8, 16, 4, 6), (1, 64, 16, 8, 40), (2, 200, 4, 16, 300), (3, 33, 1, 40, 64),
    (4, 256, 32, 6, 120), (5, 1000, 16, 12, 2500), (6, 4096, 16, 3, 3000),
])
@pytest.mark.parametrize("idx", [torch.int64, torch.int32])
def test_counts_match_brute_force(seed, nseq, bs, max_blocks, pool, idx):
    say("write check: random shared layout", seed, nseq, bs, idx)
    slots, bt, kv = shared_layout(seed, nseq, bs, max_blocks, pool)
    want = brute_counts(slots, bt, kv, bs)
    got = device_counts(slots, torch.from_numpy(bt).to(idx), torch.from_numpy(kv).to(idx), bs)
    assert got == want


def test_prefix_cache_partial_block():
    """Two identical prompts of 20 tokens (block 16): the second shares the
    first's blocks X0 (full) and X1 (4 prompt tokens). The first has
    generated 2 tokens (kv 22, writes X1 offset 5), the second 1 (kv 21,
    writes X1 offset 4, which the first attends)."""
    bs = 16
    bt = np.array([[7, 3, -1], [7, 3, -1], [11, 12, 13]])
    kv = np.array([22, 21, 40])
    slots = np.array([3 * bs + 5, 3 * bs + 4, 13 * bs + 7])
    assert brute_counts(slots, bt, kv, bs) == (0, 1)
    assert device_counts(slots, torch.from_numpy(bt), torch.from_numpy(kv), bs) == (0, 1)
    # the first sequence alone writes: the second reads offsets 0..4 only
    slots2 = slots.copy()
    slots2[1] = -1
    assert device_counts(slots2, torch.from_numpy(bt), torch.from_numpy(kv), bs) == (0, 0)
    # a block repeated in one table: read at its first entry, written at the last
    bt3 = np.array([[5, 9, 5], [11, 12, -1]])
    kv3 = np.array([40, 20])
    slots3 = np.array([5 * bs + 7, 12 * bs + 3])
    assert device_counts(slots3, torch.from_numpy(bt3), torch.from_numpy(kv3), bs) == (0, 1)
    # a duplicated slot: each of the two reads the other's write
    slots4 = np.array([3 * bs + 4, 3 * bs + 4])
    bt4, kv4 = np.array([[7, 3], [7, 3]]), np.array([21, 21])
    assert brute_counts(slots4, bt4, kv4, bs) == (0, 2)
    assert device_counts(slots4, torch.from_numpy(bt4), torch.from_numpy(kv4), bs) == (0, 2)


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5"])
def test_workloads_fuse(name):
    """The bench workloads (c4 shares its full prefix blocks among groups of
    8) pass both checks: their layer call is the fused launch."""
    say("write check: workload", name)
    c = make_case(name, seed=0, nan_fill=False)
    bs = c.layout.spec.block_size
    assert device_counts(c.slot_mapping, c.block_table, c.kv_len, bs) == (0, 0)


def _prefix_case(dtype=torch.bfloat16):
    """A c2-shaped batch where sequence 1 re-uses sequence 0's blocks as the
    prefix cache lays them out (sequence 0 one token ahead)."""
    case = make_case("c2", seed=5, nan_fill=False, dtype=dtype)
    bs = case.layout.spec.block_size
    bt, kv = case.block_table.clone(), case.kv_len.clone()
    kv[1] = kv[0] - 1
    bt[1] = bt[0]
    last = kv - 1
    case.slot_mapping = bt[torch.arange(len(kv)), last // bs] * bs + last % bs
    case.block_table, case.kv_len = bt, kv
    assert brute_counts(case.slot_mapping, bt, kv, bs) == (0, 1)
    return case


def test_eager_fused_call_runs_as_two_calls():
    say("write check: eager fused call on a shared partial block")
    from gpu_util import to_device

    case = _prefix_case()
    d = to_device(case)
    bs = case.layout.spec.block_size
    pg.invalidate_cached_metadata()
    assert not pg._fused_write_ok(d.slot_mapping, d.block_table, d.kv_len, bs, DEV, 0)
    kc1, vc1 = d.key_cache.clone(), d.value_cache.clone()
    pg.hip_cache_write(d.new_key, d.new_value, kc1, vc1, d.slot_mapping, bs)
    out1 = pg.hip_decode_attention(d.query, kc1, vc1, d.block_table, d.kv_len, bs)
    for _ in range(3):
        kc2, vc2 = d.key_cache.clone(), d.value_cache.clone()
        out2 = pg.hip_decode_attention(d.query, kc2, vc2, d.block_table, d.kv_len, bs,
                                       new_key=d.new_key, new_value=d.new_value,
                                       slot_mapping=d.slot_mapping)
        torch.cuda.synchronize()
        for x, y in ((out1, out2), (kc1, kc2), (vc1, vc2)):
            assert torch.equal(bits(x.cpu()), bits(y.cpu()))


def test_captured_fused_call_reports_a_shared_slot():
    """A captured fused call replays fine on the block manager's layout and
    reports, from check_deferred(), a replay whose slot another sequence
    attends."""
    say("write check: captured fused call")
    from gpu_util import to_device

    good = make_case("c2", seed=5, nan_fill=False)
    bad = _prefix_case()
    bs = good.layout.spec.block_size
    g, b = to_device(good), to_device(bad)
    st = {k: getattr(g, k).clone() for k in ("query", "key_cache", "value_cache", "new_key",
                                             "new_value", "slot_mapping", "block_table", "kv_len")}

    def step():
        return pg.hip_decode_attention(st["query"], st["key_cache"], st["value_cache"],
                                       st["block_table"], st["kv_len"], bs, new_key=st["new_key"],
                                       new_value=st["new_value"], slot_mapping=st["slot_mapping"])

    pg.clear_deferred()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    gid = pg.last_capture_id()
    for tag, src, raises in (("good", g, False), ("shared", b, True), ("good again", g, False)):
        say("write check: replay", tag)
        for k in ("slot_mapping", "block_table", "kv_len"):
            st[k].copy_(getattr(src, k))
        graph.replay()
        torch.cuda.synchronize()
        if raises:
            with pytest.raises(AssertionError, match="read a slot this call writes"):
                pg.check_deferred(gid)
        else:
            pg.check_deferred(gid)
    del graph
    pg.clear_deferred()


def _slots_status(slots, total):
    lib = _hip.load()
    slots = slots.to(DEV)
    n = slots.numel()
    nbytes = lib.mv_kv_slots_check_workspace_bytes(n)
    ws = torch.empty(max(nbytes, 8), dtype=torch.uint8, device=DEV)
    status = torch.full((2,), -7, dtype=torch.int32, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _hip.check(lib.mv_kv_slots_check(_ptr(slots), n, total, _ptr(status), _ptr(ws), nbytes, stream),
               "mv_kv_slots_check")
    torch.cuda.synchronize()
    return tuple(status.tolist())


def _brute_slots(slots, total):
    s = slots.numpy()
    bad = int(((s < -1) | (s >= total)).sum())
    ok = s[(s >= 0) & (s < total)]
    _, counts = np.unique(ok, return_counts=True)
    return bad, int((counts * (counts - 1) // 2).sum())


@pytest.mark.parametrize("n", [0, 1, 255, 4096, 4097, 32768, 100000])
def test_slot_check_counts(n):
    """Out-of-range slots and duplicate pairs, exactly, in one work group up
    to 4096 tokens and over a grid above; a 32k-token list with duplicates
    at both ends."""
    say("slot check", n)
    g = torch.Generator().manual_seed(n)
    total = 4 * n + 100
    slots = torch.randperm(total, generator=g)[:n].to(torch.int64)
    assert _slots_status(slots, total) == (0, 0)
    if n < 4:
        return
    s = slots.clone()
    s[-1] = s[0]            # both ends
    s[n // 2] = s[0]        # a triple: 3 pairs
    s[1] = -1
    s[2] = total            # out of range
    s[3] = -5
    assert _slots_status(s, total) == _brute_slots(s, total) == (2, 3)
    # many repeats of few values
    few = torch.randint(-1, 50, (n,), generator=g)
    assert _slots_status(few, total) == _brute_slots(few, total)


def test_slot_check_in_the_write_wrapper_at_32k_tokens():
    say("slot check: hip_cache_write at 32768 tokens")
    n, hkv, d, bs = 32768, 2, 64, 16
    nb = 2 * n // bs
    g = torch.Generator().manual_seed(11)
    slots = torch.randperm(nb * bs, generator=g)[:n]
    k = torch.randn(n, hkv, d, generator=g).to(torch.bfloat16).to(DEV)
    kc = torch.zeros(nb, hkv, bs, d, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    pg.hip_cache_write(k, k, kc, vc, slots.to(DEV), bs)
    torch.cuda.synchronize()
    rows = kc.permute(0, 2, 1, 3).reshape(nb * bs, hkv, d)[slots.to(DEV)]
    assert torch.equal(bits(rows.cpu()), bits(k.cpu()))
    dup = slots.clone()
    dup[-1] = dup[0]
    with pytest.raises(AssertionError, match="Duplicate"):
        pg.hip_cache_write(k, k, kc, vc, dup.to(DEV), bs)


def _separate(slots, bt, kv, bs, nb, pos, max_pos):
    """The three separate checks' words, through their own entry points."""
    lib = _hip.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    s = _slots_status(slots, nb * bs)
    w = device_counts(slots, bt, kv, bs)
    st = torch.full((1,), -7, dtype=torch.int32, device=DEV)
    p = pos.to(DEV)
    _hip.check(lib.mv_positions_check(_ptr(p), p.numel(), max_pos, _ptr(st), stream),
               "mv_positions_check")
    torch.cuda.synchronize()
    return list(s) + list(w) + [int(st.item())]


@pytest.mark.parametrize("seed,nseq,bs,max_blocks,pool,idx,dt,d", [
    (0, 64, 16, 8, 60, torch.int64, torch.bfloat16, 64),
    (1, 256, 16, 6, 300, torch.int32, torch.float16, 128),
    (2, 33, 4, 20, 90, torch.int64, torch.float32, 64),
    (3, 4096, 16, 3, 3000, torch.int64, torch.bfloat16, 128),
])
def test_step_check_equals_the_separate_checks(seed, nseq, bs, max_blocks, pool, idx, dt, d):
    """mv_decode_step_check (one work group, then the shared-read grid)
    gives the words of mv_kv_slots_check, mv_decode_write_check and
    mv_positions_check on the same inputs, and rows equal to the tables'
    rows at the clamped positions (bit for bit)."""
    say("step check", seed, nseq, bs, idx, dt, d)
    slots, bt, kv = shared_layout(seed, nseq, bs, max_blocks, pool)
    g = torch.Generator().manual_seed(seed)
    max_pos = 4000
    pos = torch.randint(0, max_pos, (nseq,), generator=g)
    pos[:3] = torch.tensor([-1, max_pos, max_pos + 9])[: min(3, nseq)]
    slots = torch.as_tensor(slots)
    slots[0] = pool * bs + 5  # out of the pool
    cos = torch.randn(max_pos, d + 32, generator=g).to(dt).to(DEV)  # a wider table row
    sin = torch.randn(max_pos, d + 32, generator=g).to(dt).to(DEV)
    btt, kvt = torch.from_numpy(bt).to(idx).to(DEV), torch.from_numpy(kv).to(idx).to(DEV)
    want = _separate(slots, btt, kvt, bs, pool, pos, max_pos)
    lib = _hip.load()
    sd, pd = slots.to(DEV), pos.to(DEV)
    rows_c = torch.full((nseq, d), float("nan"), dtype=dt, device=DEV)
    rows_s = torch.full((nseq, d), float("nan"), dtype=dt, device=DEV)
    st = torch.full((_hip.MV_STEP_WORDS,), -7, dtype=torch.int32, device=DEV)
    nbytes = lib.mv_decode_write_check_workspace_bytes(nseq)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _hip.check(lib.mv_decode_step_check(
        _ptr(sd), _ptr(btt), int(idx == torch.int64), btt.stride(0), _ptr(kvt),
        int(idx == torch.int64), nseq, max_blocks, bs, pool, _ptr(pd), _ptr(cos), _ptr(sin),
        cos.stride(0), max_pos, d, _hip.MV_DTYPE[dt], _ptr(rows_c), _ptr(rows_s), _ptr(st),
        _ptr(ws), nbytes, stream), "mv_decode_step_check")
    torch.cuda.synchronize()
    got = st.tolist()
    assert got[:5] == want, (got, want)
    assert got[1] > 0 and got[4] == min(3, nseq) and got[0] >= 1  # the planted cases count
    idx_c = pd.clamp(0, max_pos - 1)
    assert torch.equal(bits(rows_c.cpu()), bits(cos.index_select(0, idx_c)[:, :d].cpu()))
    assert torch.equal(bits(rows_s.cpu()), bits(sin.index_select(0, idx_c)[:, :d].cpu()))
    # without positions: no rows, word 4 zero
    st2 = torch.full((_hip.MV_STEP_WORDS,), -7, dtype=torch.int32, device=DEV)
    _hip.check(lib.mv_decode_step_check(
        _ptr(sd), _ptr(btt), int(idx == torch.int64), btt.stride(0), _ptr(kvt),
        int(idx == torch.int64), nseq, max_blocks, bs, pool, None, None, None, 0, 0, d,
        _hip.MV_DTYPE[dt], None, None, _ptr(st2), _ptr(ws), nbytes, stream), "mv_decode_step_check")
    torch.cuda.synchronize()
    assert st2.tolist()[:5] == want[:4] + [0]


def _plan_buffers(nseq, max_blocks, bs, hkv):
    lib = _hip.load()
    cap = nseq * hkv * max(1, -(-max_blocks * bs // 16))
    ids_cap = lib.mv_decode_block_ids_capacity(nseq, max_blocks, hkv, cap)
    return (torch.full((8 * cap,), -9, dtype=torch.int32, device=DEV),
            torch.full((max(ids_cap, 4),), -9, dtype=torch.int32, device=DEV),
            torch.full((nseq * hkv,), -9, dtype=torch.int32, device=DEV),
            torch.full((_hip.MV_PLAN_WORDS,), -9, dtype=torch.int32, device=DEV), cap, ids_cap)


@pytest.mark.parametrize("seed,nseq,bs,max_blocks,pool,idx", [
    (0, 64, 16, 8, 60, torch.int64),    # one launch: plan, id lists and step check
    (2, 33, 4, 20, 90, torch.int32),    # one launch
    (1, 256, 16, 6, 300, torch.int64),  # over 64 sequences: the separate launches
])
def test_plan_step_check_equals_the_two_calls(seed, nseq, bs, max_blocks, pool, idx):
    """mv_decode_plan_step_check gives mv_decode_plan's work list, id lists
    and status words, and mv_decode_step_check's status words and rotary
    rows, on the same inputs with out-of-pool slots, shared-slot reads and
    out-of-range positions planted."""
    say("plan + step check", seed, nseq, bs, idx)
    lib = _hip.load()
    hkv, d, dt, max_pos = 2, 64, torch.bfloat16, 4000
    slots, bt, kv = shared_layout(seed, nseq, bs, max_blocks, pool)
    g = torch.Generator().manual_seed(seed)
    pos = torch.randint(0, max_pos, (nseq,), generator=g)
    pos[:2] = torch.tensor([-1, max_pos])
    slots = torch.as_tensor(slots)
    slots[0] = pool * bs + 5
    cos = torch.randn(max_pos, d, generator=g).to(dt).to(DEV)
    sin = torch.randn(max_pos, d, generator=g).to(dt).to(DEV)
    btt, kvt = torch.from_numpy(bt).to(idx).to(DEV), torch.from_numpy(kv).to(idx).to(DEV)
    sd, pd = slots.to(DEV), pos.to(DEV)
    i64 = int(idx == torch.int64)
    cus = torch.cuda.get_device_properties(DEV).multi_processor_count
    nbytes = lib.mv_decode_write_check_workspace_bytes(nseq)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = []
    for combined in (False, True):
        work, ids, cnt, st, cap, ids_cap = _plan_buffers(nseq, max_blocks, bs, hkv)
        step = torch.full((_hip.MV_STEP_WORDS,), -7, dtype=torch.int32, device=DEV)
        rows = [torch.full((nseq, d), float("nan"), dtype=dt, device=DEV) for _ in range(2)]
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        plan = (_ptr(kvt), i64, _ptr(btt), i64, btt.stride(0), nseq, max_blocks, bs, pool, hkv, 2, cus, 0,
                _ptr(work), cap, _ptr(ids), ids_cap, _ptr(cnt), _ptr(st))
        chk = (_ptr(pd), _ptr(cos), _ptr(sin), cos.stride(0), max_pos, d, _hip.MV_DTYPE[dt],
               _ptr(rows[0]), _ptr(rows[1]))
        if combined:
            _hip.check(lib.mv_decode_plan_step_check(*plan, _ptr(sd), *chk, _ptr(step), _ptr(ws), nbytes,
                                                     stream), "mv_decode_plan_step_check")
        else:
            _hip.check(lib.mv_decode_plan(*plan, stream), "mv_decode_plan")
            _hip.check(lib.mv_decode_step_check(_ptr(sd), _ptr(btt), i64, btt.stride(0), _ptr(kvt), i64, nseq,
                                                max_blocks, bs, pool, *chk, _ptr(step), _ptr(ws), nbytes,
                                                stream), "mv_decode_step_check")
        torch.cuda.synchronize()
        s = st.tolist()
        n = s[_hip.MV_PLAN_NUM_ITEMS]
        per = s[_hip.MV_PLAN_IDS_PER_ITEM]
        w = work[: 8 * n].view(n, 8).cpu()
        lists = []
        for slot, e in enumerate(w.tolist()):
            span4 = min(per, ((e[5] - 1) // bs - e[4] // bs + 1 + 3) // 4 * 4)
            lists.append(ids[slot * per:slot * per + span4].cpu())
        out.append((s, w, lists, cnt.cpu(), step.tolist()[:5], [bits(r.cpu()) for r in rows]))
    (s0, w0, l0, c0, t0, r0), (s1, w1, l1, c1, t1, r1) = out
    assert s0 == s1
    # the same groups with the same id lists (the 1024-thread plan kernel of
    # the larger batch orders groups of one size by arrival)
    m0 = {tuple(e): l.tolist() for e, l in zip(w0.tolist(), l0)}
    m1 = {tuple(e): l.tolist() for e, l in zip(w1.tolist(), l1)}
    assert m0 == m1 and len(m0) == s1[_hip.MV_PLAN_NUM_ITEMS]
    if nseq <= 64:
        assert torch.equal(w0, w1)
    assert torch.equal(c0, c1) and not c1.any()
    assert t0 == t1, (t0, t1)
    assert t1[0] >= 1 and t1[4] == 2  # the planted slot and positions count
    assert all(torch.equal(x, y) for x, y in zip(r0, r1))
