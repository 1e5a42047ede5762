"""Decode layer call with the KV write fused in (mv_paged_decode_write).

It must leave the pool and the output bit-identical to the two calls it
replaces: hip_cache_write of the step's new rows, then hip_decode_attention.
In the NaN-filled cases every slot about to be written holds NaN, so a
fused call that read the new token from the pool, or skipped the write,
would not match.
"""

import pytest
import torch

from benchmarks.paged_decode_workloads import make_case
from gpu_util import DEV, TOL, bits, oracle_step, say, to_device
from mini_vllm.attention import AttentionBackend
from mini_vllm.attention.paged_attention_gpu import hip_cache_write, hip_decode_attention
from mini_vllm.model_runner.base import AttentionGroup, AttentionMetadata, ModelConfig

pytestmark = pytest.mark.gpu


def _both(case, slots=None, new_k=None, new_v=None):
    d = to_device(case)
    bs = case.layout.spec.block_size
    slots = d.slot_mapping if slots is None else slots.to(DEV)
    nk = d.new_key if new_k is None else new_k
    nv = d.new_value if new_v is None else new_v
    kc1, vc1 = d.key_cache.clone(), d.value_cache.clone()
    hip_cache_write(nk, nv, kc1, vc1, slots, bs)
    out1 = hip_decode_attention(d.query, kc1, vc1, d.block_table, d.kv_len, bs)
    kc2, vc2 = d.key_cache.clone(), d.value_cache.clone()
    out2 = hip_decode_attention(d.query, kc2, vc2, d.block_table, d.kv_len, bs,
                                new_key=nk, new_value=nv, slot_mapping=slots)
    torch.cuda.synchronize()
    return (out1, kc1, vc1), (out2, kc2, vc2)


def _same(a, b):
    for x, y in zip(a, b):
        assert torch.equal(bits(x.cpu()), bits(y.cpu()))


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5"])
def test_fused_equals_write_then_decode(name):
    say("decode+write", name)
    case = make_case(name, seed=0, nan_fill=True)
    ref, fused = _both(case)
    _same(ref, fused)
    out = fused[0].float().cpu()
    want, _, _ = oracle_step(case)
    assert not torch.isnan(out).any()
    assert (out - want).abs().max().item() <= TOL[case.layout.spec.dtype]


def test_slot_off_the_table_and_skipped_slot():
    """Sequence 0's slot is a free block's row (not its table position) and
    sequence 1's is -1: the fused call reads those sequences' last tokens
    from the pool and writes (or skips) exactly as the two calls do."""
    say("decode+write: off-table and -1 slots")
    case = make_case("c2", seed=1, nan_fill=False)
    lay = case.layout
    slots = case.slot_mapping.clone()
    used = set(int(x) for x in case.block_table.flatten().tolist() if x >= 0)
    free = next(b for b in range(lay.num_blocks) if b not in used)
    slots[0] = free * lay.spec.block_size + 3
    slots[1] = -1
    ref, fused = _both(case, slots=slots)
    _same(ref, fused)


def test_strided_new_rows():
    """New K / V as column views of one [B, 2 Hkv D] buffer."""
    say("decode+write: strided rows")
    case = make_case("c2", seed=2, nan_fill=True)
    b, hkv, d = case.new_key.shape
    kv = torch.cat([case.new_key.reshape(b, -1), case.new_value.reshape(b, -1)], dim=1).to(DEV)
    nk = kv[:, : hkv * d].view(b, hkv, d)
    nv = kv[:, hkv * d:].view(b, hkv, d)
    ref, fused = _both(case, new_k=nk, new_v=nv)
    _same(ref, fused)


def test_backend_method():
    say("decode+write: backend method")
    case = make_case("c1", seed=3, nan_fill=True)
    spec, lay = case.layout.spec, case.layout
    cfg = ModelConfig(num_layers=1, num_heads=spec.num_q_heads, num_kv_heads=spec.num_kv_heads,
                      head_dim=spec.head_dim, dtype=spec.dtype)
    be = AttentionBackend.create(cfg, backend="hip")
    pool = be.allocate_pool(1, lay.num_blocks, spec.block_size, spec.num_kv_heads, spec.head_dim,
                            spec.dtype, DEV)
    d = to_device(case)
    pool.key_caches[0].copy_(d.key_cache)
    pool.value_caches[0].copy_(d.value_cache)
    kv = d.kv_len
    group = AttentionGroup(list(range(len(kv))), "decode_gpu", kv - 1, torch.ones_like(kv), kv)
    meta = AttentionMetadata(groups=[group], decode_block_tables=d.block_table,
                             decode_slot_mapping=d.slot_mapping, block_size=spec.block_size,
                             num_kv_heads=spec.num_kv_heads, head_dim=spec.head_dim)
    out = be.decode_attention_with_write(0, d.query, d.new_key, d.new_value, d.slot_mapping, meta, pool)
    ref, _ = _both(case)
    torch.cuda.synchronize()
    _same(ref, (out, pool.key_caches[0], pool.value_caches[0]))


def test_slot_at_an_earlier_position_of_its_own_sequence():
    """Sequence 0's slot is one of its own earlier attended positions (token
    5), sequence 2's another sequence's attended row: the fused launch would
    read those rows while it writes them, so the call detects the layout on
    the device and runs as the two calls. Pool and output equal the two
    calls bit for bit, and the oracle's write-then-decode within tolerance."""
    say("decode+write: slot at an earlier attended position")
    case = make_case("c2", seed=4, nan_fill=False)
    bs = case.layout.spec.block_size
    slots = case.slot_mapping.clone()
    slots[0] = int(case.block_table[0, 5 // bs]) * bs + 5 % bs
    slots[2] = int(case.block_table[3, 0]) * bs + 1
    case.slot_mapping = slots
    ref, fused = _both(case)
    _same(ref, fused)
    want, kc_ref, vc_ref = oracle_step(case)
    assert (fused[0].float().cpu() - want).abs().max().item() <= TOL[case.layout.spec.dtype]
    assert torch.equal(bits(fused[1].float().cpu()), bits(kc_ref))


def test_fused_precondition_is_checked_in_a_captured_graph():
    """Captured, the fused call cannot fall back: its check is recorded and
    check_deferred() raises AssertionError after a replay whose slots break
    the layout; a replay with the block manager's slots passes."""
    from mini_vllm.attention import paged_attention_gpu as pg

    say("decode+write: captured precondition check")
    case = make_case("c1", seed=5, nan_fill=False)
    d = to_device(case)
    bs = case.layout.spec.block_size
    kc, vc = d.key_cache.clone(), d.value_cache.clone()
    slots = d.slot_mapping.clone()
    pg.clear_deferred()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # eager warm-up
        hip_decode_attention(d.query, kc.clone(), vc.clone(), d.block_table, d.kv_len, bs,
                             new_key=d.new_key, new_value=d.new_value, slot_mapping=slots)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        hip_decode_attention(d.query, kc, vc, d.block_table, d.kv_len, bs,
                             new_key=d.new_key, new_value=d.new_value, slot_mapping=slots)
    gid = pg.last_capture_id()
    assert gid != 0
    graph.replay()
    torch.cuda.synchronize()
    pg.check_deferred(gid)
    slots[1] = int(case.block_table[1, 0]) * bs  # sequence 1's first token, not its last
    graph.replay()
    torch.cuda.synchronize()
    with pytest.raises(AssertionError, match="kv_len_after - 1"):
        pg.check_deferred(gid)
    del graph
    pg.clear_deferred()


def test_step_cache_sees_in_place_slot_edits():
    """Layers of one step reuse the plan and the slot and fused-write checks
    (one cached entry for the same slot, table and length tensors). An
    in-place edit of the slots between layers must be checked again: a
    slot moved to an earlier attended position of its own sequence runs as
    the two calls (equal to them bit for bit), and a duplicate slot
    raises."""
    say("decode+write: step cache and in-place slot edits")
    case = make_case("c2", seed=5, nan_fill=False)
    bs = case.layout.spec.block_size
    d = to_device(case)
    slots = d.slot_mapping.clone()

    def fused(kc, vc):
        return hip_decode_attention(d.query, kc, vc, d.block_table, d.kv_len, bs,
                                    new_key=d.new_key, new_value=d.new_value, slot_mapping=slots)

    for _ in range(2):  # the second call hits the step's cached entry
        kc, vc = d.key_cache.clone(), d.value_cache.clone()
        out = fused(kc, vc)
    kc1, vc1 = d.key_cache.clone(), d.value_cache.clone()
    hip_cache_write(d.new_key, d.new_value, kc1, vc1, slots, bs)
    ref = hip_decode_attention(d.query, kc1, vc1, d.block_table, d.kv_len, bs)
    _same((ref, kc1, vc1), (out, kc, vc))

    slots[0] = int(case.block_table[0, 5 // bs]) * bs + 5 % bs  # in place: a new version
    kc, vc = d.key_cache.clone(), d.value_cache.clone()
    out = fused(kc, vc)
    kc1, vc1 = d.key_cache.clone(), d.value_cache.clone()
    hip_cache_write(d.new_key, d.new_value, kc1, vc1, slots, bs)
    ref = hip_decode_attention(d.query, kc1, vc1, d.block_table, d.kv_len, bs)
    torch.cuda.synchronize()
    _same((ref, kc1, vc1), (out, kc, vc))

    slots[1] = slots[2]
    with pytest.raises(AssertionError, match="Duplicate"):
        fused(d.key_cache.clone(), d.value_cache.clone())


def test_ctypes_route_matches_the_fast_calls(monkeypatch):
    """Without the fast-call extension the wrappers call the same entry
    points through ctypes: the fused layer call, the decode and the write
    give the same bits either way."""
    from mini_vllm.attention import _hip

    say("decode+write: ctypes route against the fast calls")
    case = make_case("c2", seed=6, nan_fill=False)
    bs = case.layout.spec.block_size
    d = to_device(case)

    def run():
        kc, vc = d.key_cache.clone(), d.value_cache.clone()
        fused = hip_decode_attention(d.query, kc, vc, d.block_table, d.kv_len, bs,
                                     new_key=d.new_key, new_value=d.new_value,
                                     slot_mapping=d.slot_mapping)
        kc2, vc2 = d.key_cache.clone(), d.value_cache.clone()
        hip_cache_write(d.new_key, d.new_value, kc2, vc2, d.slot_mapping, bs)
        dec = hip_decode_attention(d.query, kc2, vc2, d.block_table, d.kv_len, bs)
        torch.cuda.synchronize()
        return fused, kc, vc, dec, kc2, vc2

    fast = run()
    lib = _hip.load()
    monkeypatch.setattr(_hip, "decode_write", lib.mv_paged_decode_write)
    monkeypatch.setattr(_hip, "decode_write_step", None)
    monkeypatch.setattr(_hip, "decode", lib.mv_paged_decode)
    monkeypatch.setattr(_hip, "cache_write", lib.mv_kv_cache_write)
    slow = run()
    _same(fast, slow)


@pytest.mark.parametrize("rope", [False, True])
def test_layers_of_a_step_launch_from_the_step_words(monkeypatch, rope):
    """After a step's first fused layer call its other layers launch from
    the step's packed words (decode_write_step: plan, slots, rotary rows,
    sizes and workspace packed once, then only the layer's tensors). Every
    layer -- its own query, new rows and pool -- is bit-identical to its
    two calls, including a layer after the merge workspace grew (the words
    then point at a retired buffer and are rebuilt)."""
    from mini_vllm.attention import _hip
    from mini_vllm.attention import paged_attention_gpu as pg
    from oracle.rotary_ref import RotaryTables
    from mini_vllm.attention.paged_attention_gpu import hip_rope_kv_cache_write

    if _hip.load() is None or _hip.decode_write_step is None:
        pytest.skip("fast-call extension not built")
    say("decode+write: step words", "rope" if rope else "no rope")
    real = _hip.decode_write_step
    calls = []

    def counted(*args):
        calls.append(args[0])
        return real(*args)

    monkeypatch.setattr(_hip, "decode_write_step", counted)
    case = make_case("c2", seed=8, nan_fill=False)
    spec = case.layout.spec
    bs = spec.block_size
    d = to_device(case)
    pos = d.kv_len - 1
    tables = RotaryTables(spec.head_dim, 1000000.0, 4096, spec.dtype)
    cos, sin = tables.cos.to(DEV), tables.sin.to(DEV)
    extra = dict(positions=pos, cos=cos, sin=sin) if rope else {}
    g = torch.Generator(device=DEV).manual_seed(8)

    def layer(i):
        q = torch.randn(d.query.shape, device=DEV, generator=g).to(spec.dtype)
        nk = torch.randn(d.new_key.shape, device=DEV, generator=g).to(spec.dtype)
        nv = torch.randn(d.new_value.shape, device=DEV, generator=g).to(spec.dtype)
        kc1, vc1 = d.key_cache.clone(), d.value_cache.clone()
        if rope:
            q_rot, _ = hip_rope_kv_cache_write(q, nk, nv, pos, cos, sin, kc1, vc1,
                                               d.slot_mapping, bs, return_key=False)
        else:
            q_rot = q
            hip_cache_write(nk, nv, kc1, vc1, d.slot_mapping, bs)
        ref = hip_decode_attention(q_rot, kc1, vc1, d.block_table, d.kv_len, bs)
        kc2, vc2 = d.key_cache.clone(), d.value_cache.clone()
        out = hip_decode_attention(q, kc2, vc2, d.block_table, d.kv_len, bs, new_key=nk,
                                   new_value=nv, slot_mapping=d.slot_mapping, **extra)
        torch.cuda.synchronize()
        _same((ref, kc1, vc1), (out, kc2, vc2))

    for i in range(3):
        layer(i)
    assert len(calls) == 2, "layers 2 and 3 of the step launch from its words"
    # a larger batch elsewhere grows the merge workspace (here: asking for
    # one byte more than it holds); the step's words are rebuilt
    dev = d.query.device
    ws0 = pg._WORKSPACES.get(dev)
    assert ws0 is not None
    ws = pg._workspace(dev, ws0.numel() + 1)
    assert ws is not ws0
    layer(3)
    layer(4)
    assert len(calls) == 3 and calls[1] == calls[0] and calls[2] != calls[1]
    assert pg._WORKSPACES.get(dev) is ws
