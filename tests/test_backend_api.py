"""Plugin API and pool behaviour that needs no GPU.

Mirrors the reference's tests/test_no_silent_fallback.py and
tests/test_kv_cache_pool.py for this package's backend and pool.
"""

import pytest
import torch

from mini_vllm.attention import AttentionBackend, AttentionBackendGPU
from mini_vllm.attention.paged_attention_gpu import hip_cache_write, hip_decode_attention
from mini_vllm.cache.pool import MIN_BLOCKS, KVCachePool, compute_num_gpu_blocks
from mini_vllm.model_runner.base import AttentionGroup, AttentionMetadata, ModelConfig


def _cfg(**kw):
    base = dict(num_layers=1, hidden_size=256, num_heads=4, num_kv_heads=2, head_dim=64,
                dtype=torch.float16)
    base.update(kw)
    return ModelConfig(**base)


def test_unknown_backend_raises_value_error():
    with pytest.raises(ValueError, match="Unknown"):
        AttentionBackend.create(_cfg(), backend="nonexistent")


def test_reference_backend_not_shipped_here_import_error_propagates():
    # This package does not ship the reference's PyTorch backend module, so
    # the reference's lazy import fails loudly (no fallback to the GPU).
    for name in ("reference", "ref"):
        with pytest.raises(ImportError, match="paged_attention_ref"):
            AttentionBackend.create(_cfg(), backend=name)


def test_reference_backend_branch_imports_sibling_module(monkeypatch):
    # Dropped into the reference tree, create("reference") returns the
    # reference's AttentionBackendRef (reference backend.py:106-108,
    # tests/test_no_silent_fallback.py:88-94): stand in a module for it.
    import sys
    import types

    class AttentionBackendRef:
        def __init__(self, config):
            self.config = config

    mod = types.ModuleType("mini_vllm.attention.paged_attention_ref")
    mod.AttentionBackendRef = AttentionBackendRef
    monkeypatch.setitem(sys.modules, "mini_vllm.attention.paged_attention_ref", mod)
    cfg = _cfg()
    for name in ("reference", "ref"):
        be = AttentionBackend.create(cfg, backend=name)
        assert isinstance(be, AttentionBackendRef) and be.config is cfg


@pytest.mark.parametrize("hd", [32, 96, 256])
def test_unsupported_head_dim_raises(hd):
    with pytest.raises(RuntimeError, match="head_dim"):
        AttentionBackendGPU(_cfg(head_dim=hd))


def test_unsupported_group_ratio_raises():
    with pytest.raises(RuntimeError, match="query heads"):
        AttentionBackendGPU(_cfg(num_heads=34, num_kv_heads=2))


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU error")
def test_no_gpu_raises_instead_of_falling_back():
    with pytest.raises(RuntimeError, match="requires a ROCm GPU"):
        AttentionBackend.create(_cfg(), backend="hip")
    with pytest.raises(RuntimeError, match="requires a ROCm GPU"):
        AttentionBackend.create(_cfg(), backend="triton")


def test_cpu_tensors_are_rejected():
    kc = torch.zeros(4, 2, 4, 64, dtype=torch.float16)
    k = torch.zeros(1, 2, 64, dtype=torch.float16)
    with pytest.raises(AssertionError, match="cuda"):
        hip_cache_write(k, k, kc, kc.clone(), torch.tensor([0]), 4)
    with pytest.raises(AssertionError):
        hip_decode_attention(torch.zeros(1, 4, 64, dtype=torch.float16), kc, kc.clone(),
                             torch.tensor([[0]]), torch.tensor([1]), 4)


def test_decode_asserts_match_reference_preconditions():
    q = torch.zeros(1, 4, 96, dtype=torch.float16)
    kc = torch.zeros(4, 2, 16, 96, dtype=torch.float16)
    with pytest.raises(AssertionError, match="head_dim"):
        hip_decode_attention(q, kc, kc, torch.tensor([[0]]), torch.tensor([1]), 16)
    q = torch.zeros(1, 4, 64, dtype=torch.float16)
    kc = torch.zeros(4, 3, 16, 64, dtype=torch.float16)
    with pytest.raises(AssertionError, match="divisible"):
        hip_decode_attention(q, kc, kc, torch.tensor([[0]]), torch.tensor([1]), 16)
    kc = torch.zeros(4, 2, 12, 64, dtype=torch.float16)
    with pytest.raises(AssertionError, match="power of 2"):
        hip_decode_attention(q, kc, kc, torch.tensor([[0]]), torch.tensor([1]), 12)


# ----------------------------------------------------------------- pool --


def test_pool_shapes_and_accessors():
    pool = KVCachePool.allocate(2, 8, 4, 4, 128, dtype=torch.float16, device=torch.device("cpu"))
    assert (pool.num_layers, pool.num_blocks, pool.block_size, pool.num_kv_heads,
            pool.head_dim) == (2, 8, 4, 4, 128)
    for layer in range(2):
        assert pool.key_caches[layer].shape == (8, 4, 4, 128)
        assert pool.get_key_cache(layer) is pool.key_caches[layer]
        assert pool.get_value_cache(layer) is pool.value_caches[layer]
        assert pool.key_caches[layer].is_contiguous()


@pytest.mark.parametrize("args,name", [
    ((1, 0, 4, 2, 64), "num_blocks"), ((0, 8, 4, 2, 64), "num_layers"),
    ((1, 8, 0, 2, 64), "block_size"), ((1, 8, 4, 0, 64), "num_kv_heads"),
    ((1, 8, 4, 2, 0), "head_dim"),
])
def test_pool_rejects_non_positive_sizes(args, name):
    with pytest.raises(ValueError, match=name):
        KVCachePool.allocate(*args, device=torch.device("cpu"))


def test_pool_reset_and_bytes():
    pool = KVCachePool.allocate(3, 16, 4, 4, 128, dtype=torch.float16, device=torch.device("cpu"))
    for t in pool.key_caches + pool.value_caches:
        t.fill_(1.5)
    pool.reset()
    assert all((t == 0).all() for t in pool.key_caches + pool.value_caches)
    assert pool.total_slots == 64
    assert pool.bytes_per_block_per_layer == 2 * 4 * 4 * 128 * 2
    assert pool.bytes_per_block_total == 3 * pool.bytes_per_block_per_layer
    assert pool.total_bytes == 16 * pool.bytes_per_block_total
    bf = KVCachePool.allocate(1, 8, 4, 2, 64, dtype=torch.bfloat16, device=torch.device("cpu"))
    f32 = KVCachePool.allocate(1, 8, 4, 2, 64, dtype=torch.float32, device=torch.device("cpu"))
    assert f32.bytes_per_block_per_layer == 2 * bf.bytes_per_block_per_layer


def test_num_blocks_budget_rules():
    assert compute_num_gpu_blocks(32, 8, 128, 16, num_gpu_blocks_override=256) == 256
    with pytest.raises(RuntimeError, match="num_gpu_blocks_override"):
        compute_num_gpu_blocks(32, 8, 128, 16, num_gpu_blocks_override=MIN_BLOCKS - 1)
    assert compute_num_gpu_blocks(32, 8, 128, 16, device=torch.device("cpu")) == MIN_BLOCKS
    for util in (0.0, 1.5, -0.1):
        with pytest.raises(ValueError, match="gpu_memory_utilization"):
            compute_num_gpu_blocks(1, 1, 64, 4, gpu_memory_utilization=util)


def test_metadata_types_keep_reference_fields():
    g = AttentionGroup([0, 1], "decode_gpu", torch.tensor([3, 4]), torch.ones(2, dtype=torch.long),
                       torch.tensor([4, 5]))
    m = AttentionMetadata(groups=[g], decode_block_tables=torch.tensor([[0], [1]]), block_size=16)
    assert m.decode_group() is g
    assert m.prefill_slot_mapping.dtype == torch.long and m.prefill_slot_mapping.numel() == 0
    assert AttentionMetadata().decode_group() is None


def test_cached_checks_follow_versions_and_can_be_invalidated():
    """The per-step check cache matches the same tensor objects at the same
    in-place version. An in-place torch write bumps the version (a new
    check); a write through a numpy view does not, and
    invalidate_cached_metadata() drops the entry so the next call checks
    again."""
    from mini_vllm.attention import paged_attention_gpu as pg

    pg.invalidate_cached_metadata()
    bt = torch.zeros(2, 4, dtype=torch.int32)
    kv = torch.ones(2, dtype=torch.int32)
    pg._cache_put("plan", (bt, kv), ("x",), "plan-1")
    assert pg._cache_get("plan", (bt, kv), ("x",)) == "plan-1"
    assert pg._cache_get("plan", (bt.clone(), kv), ("x",)) is None  # another tensor
    kv.numpy()[0] = 9  # invisible to torch: same version, the entry still matches
    assert pg._cache_get("plan", (bt, kv), ("x",)) == "plan-1"
    pg.invalidate_cached_metadata()
    assert pg._cache_get("plan", (bt, kv), ("x",)) is None
    pg._cache_put("plan", (bt, kv), ("x",), "plan-2")
    kv.add_(0)  # an in-place torch op bumps the version
    assert pg._cache_get("plan", (bt, kv), ("x",)) is None
