"""KV-cache write on the GPU: bit-exact against the oracle's write.

Mirrors the reference's Triton write tests (tests/test_paged_attention_gpu.py:159-207)
and its CPU write tests (tests/test_cache_write.py), comparing whole pools
bit for bit (NaN patterns included).
"""

import pytest
import torch

from gpu_util import DEV, bits, cached_case, say, to_device
from mini_vllm.attention.paged_attention_gpu import hip_cache_write, triton_cache_write
from oracle.paged_ref import write_to_paged_cache

pytestmark = pytest.mark.gpu


def _pool(nb, hkv, bs, d, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    kc = torch.randn(nb, hkv, bs, d, generator=g).to(dtype)
    vc = torch.randn(nb, hkv, bs, d, generator=g).to(dtype)
    return kc, vc


def _write_both(k, v, kc, vc, slots, bs):
    """GPU write into device copies; oracle write into CPU copies; compare."""
    kd, vd = kc.to(DEV), vc.to(DEV)
    hip_cache_write(k.to(DEV) if k.device.type != "cuda" else k,
                    v.to(DEV) if v.device.type != "cuda" else v, kd, vd, slots.to(DEV), bs)
    torch.cuda.synchronize()
    kr, vr = kc.clone(), vc.clone()
    write_to_paged_cache(k.cpu(), v.cpu(), kr, vr, slots.cpu(), bs)
    assert torch.equal(bits(kd.cpu()), bits(kr)), "key_cache differs"
    assert torch.equal(bits(vd.cpu()), bits(vr)), "value_cache differs"


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5"])
def test_workload_write_bit_exact(name):
    say("write", name)
    c, (_, kref, vref) = cached_case(name)
    d = to_device(c)
    hip_cache_write(d.new_key, d.new_value, d.key_cache, d.value_cache, d.slot_mapping,
                    c.layout.spec.block_size)
    torch.cuda.synchronize()
    assert torch.equal(bits(d.key_cache.cpu().float()), bits(kref))
    assert torch.equal(bits(d.value_cache.cpu().float()), bits(vref))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bs,d", [(16, 64), (16, 128), (1, 64), (8, 128), (32, 64), (4, 40), (4, 7)])
def test_shapes_and_dtypes(dtype, bs, d):
    say("write shape", dtype, bs, d)
    hkv, nb = 2, 64
    kc, vc = _pool(nb, hkv, bs, d, dtype)
    g = torch.Generator().manual_seed(bs * 100 + d)
    n = min(50, nb * bs)
    slots = torch.randperm(nb * bs, generator=g)[:n]
    slots[3::5] = -1
    k = torch.randn(n, hkv, d, generator=g).to(dtype)
    v = torch.randn(n, hkv, d, generator=g).to(dtype)
    _write_both(k, v, kc, vc, slots, bs)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_strided_views_of_fused_qkv(dtype):
    """K and V as column views of a fused [T, (Hq + 2 Hkv) * D] projection
    (reference qkv_proj.py:57-61); V stays non-contiguous."""
    say("write strided", dtype)
    t, hq, hkv, d, bs = 37, 14, 2, 64, 16
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(t, (hq + 2 * hkv) * d, generator=g).to(dtype).to(DEV)
    k = qkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
    assert not v.is_contiguous()
    kc, vc = _pool(16, hkv, bs, d, dtype)
    slots = torch.randperm(16 * bs, generator=g)[:t]
    _write_both(k, v, kc, vc, slots, bs)


def test_reference_known_answers():
    """Single token at slot 5, non-contiguous slots, block boundary, -1 skip
    (test_paged_attention_gpu.py:167-197)."""
    say("write known answers")
    for bs, nb, slots in [(16, 64, [5]), (16, 32, [0, 17, 33, 50, 99]), (4, 8, [7, 8]),
                          (16, 64, [0, -1, 15])]:
        kc, vc = _pool(nb, 2, bs, 64, torch.float16)
        n = len(slots)
        k = (10.0 + torch.arange(n * 2 * 64, dtype=torch.float32)).view(n, 2, 64).half()
        v = (500.0 + torch.arange(n * 2 * 64, dtype=torch.float32)).view(n, 2, 64).half()
        _write_both(k, v, kc, vc, torch.tensor(slots), bs)


def test_duplicate_slots_raise_and_write_nothing():
    say("write duplicates")
    kc, vc = _pool(64, 2, 16, 64, torch.float16)
    kd, vd = kc.to(DEV), vc.to(DEV)
    k = torch.randn(2, 2, 64).half().to(DEV)
    with pytest.raises(AssertionError, match="Duplicate"):
        triton_cache_write(k, k, kd, vd, torch.tensor([5, 5], device=DEV), 16)
    torch.cuda.synchronize()
    assert torch.equal(bits(kd.cpu()), bits(kc))


@pytest.mark.parametrize("slot", [64 * 16, -2, 10**12])
def test_out_of_range_raises_and_writes_nothing(slot):
    say("write out of range", slot)
    kc, vc = _pool(64, 2, 16, 64, torch.bfloat16)
    kd, vd = kc.to(DEV), vc.to(DEV)
    k = torch.randn(2, 2, 64).to(torch.bfloat16).to(DEV)
    with pytest.raises(IndexError, match="out of range"):
        hip_cache_write(k, k, kd, vd, torch.tensor([3, slot], device=DEV), 16)
    torch.cuda.synchronize()
    assert torch.equal(bits(kd.cpu()), bits(kc)) and torch.equal(bits(vd.cpu()), bits(vc))


def test_many_tokens_duplicate_detection_across_tiles():
    """2000 tokens (8 check tiles): a duplicate pair far apart is found; a
    permutation passes."""
    say("write many tokens")
    nb, bs = 256, 16
    kc, vc = _pool(nb, 2, bs, 64, torch.bfloat16)
    g = torch.Generator().manual_seed(9)
    slots = torch.randperm(nb * bs, generator=g)[:2000]
    k = torch.randn(2000, 2, 64, generator=g).to(torch.bfloat16)
    _write_both(k, k.clone(), kc, vc, slots, bs)
    dup = slots.clone()
    dup[1999] = dup[3]
    with pytest.raises(AssertionError, match="Duplicate"):
        hip_cache_write(k.to(DEV), k.to(DEV), kc.to(DEV), vc.to(DEV), dup.to(DEV), bs)


def test_validation_is_redone_after_in_place_update():
    """The slot check is cached per tensor object + version: the same
    tensor passes again without a check, an in-place edit is re-checked."""
    say("write check cache")
    kc, vc = _pool(8, 2, 4, 64, torch.float16)
    kd, vd = kc.to(DEV), vc.to(DEV)
    k = torch.randn(3, 2, 64).half().to(DEV)
    slots = torch.tensor([1, 2, 3], device=DEV)
    for _ in range(3):
        hip_cache_write(k, k, kd, vd, slots, 4)
    slots[2] = 1
    with pytest.raises(AssertionError, match="Duplicate"):
        hip_cache_write(k, k, kd, vd, slots, 4)


def test_empty_write_is_a_no_op():
    kc, vc = _pool(8, 2, 4, 64, torch.float16)
    kd, vd = kc.to(DEV), vc.to(DEV)
    e = torch.empty(0, 2, 64, dtype=torch.float16, device=DEV)
    hip_cache_write(e, e, kd, vd, torch.empty(0, dtype=torch.long, device=DEV), 4)
    torch.cuda.synchronize()
    assert torch.equal(bits(kd.cpu()), bits(kc))
