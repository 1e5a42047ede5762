"""Fused RoPE + KV write (mv_rope_kv_cache_write) against the oracle.

The oracle is the runner's own sequence on CPU (oracle/rotary_ref.py:
rope_then_write, restating qwen_runner.py:164-170): rotate q, rotate k with
eager torch ops in the dtype, then the per-token KV write. The kernel must
match it bit for bit: the rotated query, the rotated key, and every cache
row (written or untouched; free rows hold NaN).
"""

import pytest
import torch

from gpu_util import DEV, bits, say
from mini_vllm.attention import AttentionBackend
from mini_vllm.attention.paged_attention_gpu import hip_rope_kv_cache_write, hip_rotary
from mini_vllm.model_runner.base import ModelConfig
from oracle.rotary_ref import RotaryTables, rope_then_write, rotary

pytestmark = pytest.mark.gpu

MAX_POS = 4096


def _tables(d, dtype, theta=1000000.0):
    return RotaryTables(d, theta, MAX_POS, dtype)


def _case(hq, hkv, d, t, bs, dtype, fused, seed=0, num_blocks=64):
    g = torch.Generator().manual_seed(seed)
    if fused:  # q / k / v as column views of one QKV projection output
        qkv = torch.randn(t, (hq + 2 * hkv) * d, generator=g).to(dtype)
        q = qkv[:, : hq * d].view(t, hq, d)
        k = qkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
        v = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
    else:
        q = torch.randn(t, hq, d, generator=g).to(dtype)
        k = torch.randn(t, hkv, d, generator=g).to(dtype)
        v = torch.randn(t, hkv, d, generator=g).to(dtype)
    total = num_blocks * bs
    slots = torch.randperm(total, generator=g)[:t].to(torch.int64)
    slots[::7] = -1  # skipped tokens (prefix-cache hits)
    pos = torch.randint(0, MAX_POS, (t,), generator=g)
    pos[0], pos[-1] = 0, MAX_POS - 1
    kc = torch.full((num_blocks, hkv, bs, d), float("nan")).to(dtype)
    vc = torch.full((num_blocks, hkv, bs, d), float("nan")).to(dtype)
    return q, k, v, slots, pos, kc, vc


SHAPES = [(14, 2, 64, 16, 64), (28, 4, 128, 16, 37), (14, 2, 64, 256, 300)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("fused", [True, False])
def test_matches_runner_sequence_bitwise(dtype, shape, fused):
    hq, hkv, d, bs, t = shape
    say("rope+write", dtype, shape, "fused" if fused else "contiguous")
    q, k, v, slots, pos, kc, vc = _case(hq, hkv, d, t, bs, dtype, fused)
    tables = _tables(d, dtype)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    q_ref, k_ref = rope_then_write(q, k, v, pos, tables, kc_ref, vc_ref, slots, bs)

    if fused:  # views of one device QKV buffer, as the projection leaves them
        qkv = torch.cat([q.reshape(t, -1), k.reshape(t, -1), v.reshape(t, -1)], dim=1).to(DEV)
        qd = qkv[:, : hq * d].view(t, hq, d)
        kd = qkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
        vd = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
        assert not qd.is_contiguous()
    else:
        qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    q_rot, k_rot = hip_rope_kv_cache_write(qd, kd, vd, pos.to(DEV), tables.cos.to(DEV),
                                           tables.sin.to(DEV), kc_d, vc_d, slots.to(DEV), bs)
    torch.cuda.synchronize()
    assert torch.equal(bits(q_rot.cpu()), bits(q_ref))
    assert torch.equal(bits(k_rot.cpu()), bits(k_ref))
    assert torch.equal(bits(kc_d.cpu()), bits(kc_ref))
    assert torch.equal(bits(vc_d.cpu()), bits(vc_ref))


def test_inplace_query_and_no_key_copy():
    say("rope+write in place")
    q, k, v, slots, pos, kc, vc = _case(14, 2, 64, 64, 16, torch.bfloat16, False, seed=1)
    tables = _tables(64, torch.bfloat16)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    q_ref, _ = rope_then_write(q, k, v, pos, tables, kc_ref, vc_ref, slots, 16)
    qd, kc_d, vc_d = q.to(DEV), kc.to(DEV), vc.to(DEV)
    q_rot, k_rot = hip_rope_kv_cache_write(qd, k.to(DEV), v.to(DEV), pos.to(DEV), tables.cos.to(DEV),
                                           tables.sin.to(DEV), kc_d, vc_d, slots.to(DEV), 16,
                                           return_key=False, inplace=True)
    torch.cuda.synchronize()
    assert q_rot is qd and k_rot is None
    assert torch.equal(bits(qd.cpu()), bits(q_ref))
    assert torch.equal(bits(kc_d.cpu()), bits(kc_ref))
    assert torch.equal(bits(vc_d.cpu()), bits(vc_ref))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_plain_rotary(dtype):
    say("rotary", dtype)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(50, 5, 128, generator=g).to(dtype)
    pos = torch.randint(0, MAX_POS, (50,), generator=g)
    tables = _tables(128, dtype, theta=10000.0)
    out = hip_rotary(x.to(DEV), pos.to(DEV), tables.cos.to(DEV), tables.sin.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(bits(out.cpu()), bits(rotary(x, pos, tables)))


def test_errors_like_the_reference():
    say("rope+write errors")
    q, k, v, slots, pos, kc, vc = _case(14, 2, 64, 8, 16, torch.bfloat16, False, seed=2)
    tables = _tables(64, torch.bfloat16)
    args = [t.to(DEV) for t in (q, k, v)]
    cos, sin = tables.cos.to(DEV), tables.sin.to(DEV)
    bad_pos = pos.clone()
    bad_pos[3] = MAX_POS  # one past the tables (the reference's lookup raises IndexError)
    with pytest.raises(IndexError):
        hip_rope_kv_cache_write(*args, bad_pos.to(DEV), cos, sin, kc.to(DEV), vc.to(DEV),
                                slots.to(DEV), 16)
    dup = slots.clone()
    dup[1] = dup[2] = 5
    with pytest.raises(AssertionError):
        hip_rope_kv_cache_write(*args, pos.to(DEV), cos, sin, kc.to(DEV), vc.to(DEV), dup.to(DEV), 16)


def test_backend_method_replaces_runner_calls():
    say("backend rope_write_kv_cache")
    cfg = ModelConfig(num_layers=2, hidden_size=896, num_heads=14, num_kv_heads=2, head_dim=64,
                      dtype=torch.bfloat16)
    be = AttentionBackend.create(cfg, backend="hip")
    pool = be.allocate_pool(2, 32, 16, 2, 64, torch.bfloat16, DEV)
    q, k, v, slots, pos, _, _ = _case(14, 2, 64, 20, 16, torch.bfloat16, False, seed=4, num_blocks=32)
    tables = _tables(64, torch.bfloat16)
    kc_ref = pool.key_caches[1].cpu().clone()
    vc_ref = pool.value_caches[1].cpu().clone()
    q_ref, k_ref = rope_then_write(q, k, v, pos, tables, kc_ref, vc_ref, slots, 16)

    class Rope:  # the runner's RotaryEmbedding exposes .cos / .sin
        cos = tables.cos.to(DEV)
        sin = tables.sin.to(DEV)

    q_rot, k_rot = be.rope_write_kv_cache(1, q.to(DEV), k.to(DEV), v.to(DEV), pos.to(DEV), Rope,
                                          slots.to(DEV), return_key=True)
    torch.cuda.synchronize()
    assert torch.equal(bits(q_rot.cpu()), bits(q_ref))
    assert torch.equal(bits(k_rot.cpu()), bits(k_ref))
    assert torch.equal(bits(pool.key_caches[1].cpu()), bits(kc_ref))
    assert torch.equal(bits(pool.value_caches[1].cpu()), bits(vc_ref))


# ---- the whole decode sub-layer in one launch: RoPE + KV write + decode ----

@pytest.mark.parametrize("name,dtype", [("c1", torch.float32), ("c2", torch.bfloat16),
                                        ("c2", torch.float16), ("c3", torch.bfloat16),
                                        ("c4", torch.bfloat16), ("c5", torch.bfloat16),
                                        ("c5", torch.float32)])
def test_decode_with_fused_rope_equals_rope_write_then_decode(name, dtype):
    """hip_decode_attention with new rows, slots and positions/cos/sin does
    RoPE of q and the new k, the KV write and the decode in one launch; pool
    and output are bit-identical to hip_rope_kv_cache_write followed by the
    decode of the rotated query, and the decode matches the oracle (rotate,
    write, decode on the CPU) within the dtype tolerance. q, k and v are
    column views of one fused QKV buffer; unread and about-to-be-written
    pool rows hold NaN."""
    from benchmarks.paged_decode_workloads import make_case
    from gpu_util import TOL, to_device
    from mini_vllm.attention.paged_attention_gpu import hip_decode_attention
    from oracle import paged_ref

    say("decode + fused rope + write", name, dtype)
    case = make_case(name, seed=6, dtype=dtype, nan_fill=True)
    d = to_device(case)
    spec = case.layout.spec
    b, hq, hd = d.query.shape
    hkv = spec.num_kv_heads
    qkv = torch.cat([d.query.reshape(b, -1), d.new_key.reshape(b, -1),
                     d.new_value.reshape(b, -1)], dim=1)
    q = qkv[:, : hq * hd].view(b, hq, hd)
    k = qkv[:, hq * hd:(hq + hkv) * hd].view(b, hkv, hd)
    v = qkv[:, (hq + hkv) * hd:].view(b, hkv, hd)
    pos = (d.kv_len - 1).clamp(max=MAX_POS - 1)
    tables = _tables(hd, dtype)
    cos, sin = tables.cos.to(DEV), tables.sin.to(DEV)
    bs = spec.block_size
    # two calls: fused RoPE + write, then decode of the rotated query
    kc1, vc1 = d.key_cache.clone(), d.value_cache.clone()
    q_rot, _ = hip_rope_kv_cache_write(q, k, v, pos, cos, sin, kc1, vc1, d.slot_mapping, bs,
                                       return_key=False)
    out1 = hip_decode_attention(q_rot, kc1, vc1, d.block_table, d.kv_len, bs)
    # one launch
    kc2, vc2 = d.key_cache.clone(), d.value_cache.clone()
    out2 = hip_decode_attention(q, kc2, vc2, d.block_table, d.kv_len, bs, new_key=k, new_value=v,
                                slot_mapping=d.slot_mapping, positions=pos, cos=cos, sin=sin)
    torch.cuda.synchronize()
    for x, y in ((out1, out2), (kc1, kc2), (vc1, vc2)):
        assert torch.equal(bits(x.cpu()), bits(y.cpu()))
    # the oracle: the runner's rotate / rotate / write / decode on the CPU
    kc_ref, vc_ref = case.key_cache.float().clone(), case.value_cache.float().clone()
    cpu_tab = _tables(hd, dtype)
    q_r = rotary(case.query, pos.cpu(), cpu_tab).float()
    k_r = rotary(case.new_key, pos.cpu(), cpu_tab).float()
    paged_ref.write_to_paged_cache(k_r, case.new_value.float(), kc_ref, vc_ref, case.slot_mapping,
                                   bs)
    want = paged_ref.decode_from_tables(q_r, kc_ref, vc_ref, case.block_table, case.kv_len, bs)
    got = out2.float().cpu()
    assert not torch.isnan(got).any()
    assert (got - want).abs().max().item() <= TOL[dtype]
    assert torch.equal(bits(kc2.cpu().float()), bits(kc_ref))


def test_backend_sub_layer_method():
    """AttentionBackendGPU.decode_attention_with_rope_write: the runner's
    rope / rope / write / decode of the decode rows in one call."""
    from benchmarks.paged_decode_workloads import make_case
    from gpu_util import to_device
    from mini_vllm.attention.paged_attention_gpu import hip_decode_attention
    from mini_vllm.model_runner.base import AttentionGroup, AttentionMetadata

    say("backend decode_attention_with_rope_write")
    case = make_case("c1", seed=7, dtype=torch.bfloat16, nan_fill=True)
    d = to_device(case)
    spec = case.layout.spec
    dt = case.query.dtype
    cfg = ModelConfig(num_layers=1, num_heads=spec.num_q_heads, num_kv_heads=spec.num_kv_heads,
                      head_dim=spec.head_dim, dtype=dt)
    be = AttentionBackend.create(cfg, backend="hip")
    pool = be.allocate_pool(1, case.layout.num_blocks, spec.block_size, spec.num_kv_heads,
                            spec.head_dim, dt, DEV)
    pool.key_caches[0].copy_(d.key_cache)
    pool.value_caches[0].copy_(d.value_cache)
    kv = d.kv_len
    meta = AttentionMetadata(
        groups=[AttentionGroup(list(range(len(kv))), "decode_gpu", kv - 1, torch.ones_like(kv), kv)],
        decode_block_tables=d.block_table, decode_slot_mapping=d.slot_mapping,
        block_size=spec.block_size, num_kv_heads=spec.num_kv_heads, head_dim=spec.head_dim)
    tables = _tables(spec.head_dim, dt)
    tables.cos, tables.sin = tables.cos.to(DEV), tables.sin.to(DEV)
    pos = kv - 1
    out = be.decode_attention_with_rope_write(0, d.query, d.new_key, d.new_value, pos, tables,
                                              d.slot_mapping, meta, pool)
    kc, vc = d.key_cache.clone(), d.value_cache.clone()
    q_rot, _ = hip_rope_kv_cache_write(d.query, d.new_key, d.new_value, pos, tables.cos,
                                       tables.sin, kc, vc, d.slot_mapping, spec.block_size,
                                       return_key=False)
    ref = hip_decode_attention(q_rot, kc, vc, d.block_table, kv, spec.block_size)
    torch.cuda.synchronize()
    for x, y in ((ref, out), (kc, pool.key_caches[0]), (vc, pool.value_caches[0])):
        assert torch.equal(bits(x.cpu()), bits(y.cpu()))
