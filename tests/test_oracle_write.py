"""Pins the oracle's KV write (oracle.paged_ref.write_to_paged_cache).

Every case is a known answer taken from the reference's own write tests
(tests/test_cache_write.py, cited per test) — explicit slot -> (block,
offset) positions, last-writer-wins, -1 skip, range and validation errors —
plus agreement with the independent numpy token loop (oracle.brute.write).
"""

import numpy as np
import pytest
import torch

from oracle import brute
from oracle.paged_ref import write_to_paged_cache


@pytest.fixture
def pool():
    """4 blocks x 2 kv heads x block 4 x head_dim 8, fp16 (test_cache_write.py:19-24)."""
    return torch.empty(4, 2, 4, 8, dtype=torch.float16), torch.empty(4, 2, 4, 8, dtype=torch.float16)


def _kv(n, seed=0, heads=2, dim=8, dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n, heads, dim, generator=g).to(dtype),
            torch.randn(n, heads, dim, generator=g).to(dtype))


def test_single_slot_position(pool):
    # test_cache_write.py:32-46: slot 5 at block_size 4 -> block 1, offset 1
    kc, vc = pool
    k, v = _kv(1)
    write_to_paged_cache(k, v, kc, vc, torch.tensor([5]), 4)
    assert torch.equal(kc[1, :, 1, :], k[0]) and torch.equal(vc[1, :, 1, :], v[0])


def test_prefill_slots_0_to_7(pool):
    # test_cache_write.py:54-70
    kc, vc = pool
    k, v = _kv(8, 1)
    write_to_paged_cache(k, v, kc, vc, torch.arange(8), 4)
    for t in range(8):
        assert torch.equal(kc[t // 4, :, t % 4, :], k[t])
        assert torch.equal(vc[t // 4, :, t % 4, :], v[t])


def test_block_boundaries(pool):
    # test_cache_write.py:137-161: slots 3, 4, 7, 8
    kc, vc = pool
    k, v = _kv(4, 2)
    write_to_paged_cache(k, v, kc, vc, torch.tensor([3, 4, 7, 8]), 4)
    for t, (b, o) in enumerate([(0, 3), (1, 0), (1, 3), (2, 0)]):
        assert torch.equal(kc[b, :, o, :], k[t]) and torch.equal(vc[b, :, o, :], v[t])


def test_non_contiguous_blocks():
    # test_cache_write.py:169-190: slots 20, 69, 14 -> blocks 5, 17, 3 / offsets 0, 1, 2
    kc = torch.empty(32, 2, 4, 8, dtype=torch.float16)
    vc = torch.empty(32, 2, 4, 8, dtype=torch.float16)
    k, v = _kv(3, 3)
    write_to_paged_cache(k, v, kc, vc, torch.tensor([20, 69, 14]), 4)
    for t, (b, o) in enumerate([(5, 0), (17, 1), (3, 2)]):
        assert torch.equal(kc[b, :, o, :], k[t]) and torch.equal(vc[b, :, o, :], v[t])


def test_last_writer_wins(pool):
    # test_cache_write.py:197-212
    kc, vc = pool
    k, v = _kv(2, 4)
    write_to_paged_cache(k, v, kc, vc, torch.tensor([5, 5]), 4)
    assert torch.equal(kc[1, :, 1, :], k[1]) and torch.equal(vc[1, :, 1, :], v[1])


def test_unwritten_slots_unchanged(pool):
    # test_cache_write.py:247-282
    kc, vc = pool
    kc.copy_(torch.randn_like(kc, dtype=torch.float32).half())
    vc.copy_(torch.randn_like(vc, dtype=torch.float32).half())
    k0, v0 = kc.clone(), vc.clone()
    k, v = _kv(2, 5)
    write_to_paged_cache(k, v, kc, vc, torch.tensor([2, 10]), 4)
    changed = torch.zeros(4, 4, dtype=torch.bool)
    changed[0, 2] = changed[2, 2] = True
    for b in range(4):
        for o in range(4):
            if not changed[b, o]:
                assert torch.equal(kc[b, :, o, :], k0[b, :, o, :])
                assert torch.equal(vc[b, :, o, :], v0[b, :, o, :])


def test_minus_one_skips(pool):
    # test_cache_write.py:310-336
    kc, vc = pool
    kc.zero_(); vc.zero_()
    k = torch.full((4, 2, 8), 42.0, dtype=torch.float16)
    write_to_paged_cache(k, k.clone(), kc, vc, torch.tensor([-1, 5, -1, 8]), 4)
    assert (kc[1, :, 1, :] == 42).all() and (kc[2, :, 0, :] == 42).all()
    assert (kc[0, :, 0, :] == 0).all() and int((kc == 42).sum()) == 2 * 2 * 8


@pytest.mark.parametrize("slot", [16, -2])
def test_out_of_range_raises(pool, slot):
    # test_cache_write.py:343-373
    kc, vc = pool
    k, v = _kv(1)
    with pytest.raises(IndexError, match="out of range"):
        write_to_paged_cache(k, v, kc, vc, torch.tensor([slot]), 4)


@pytest.mark.parametrize(
    "case, match",
    [
        ("value_dim", "key shape.*!=.*value shape"),
        ("slot_len", "slot_mapping length"),
        ("heads", "num_kv_heads"),
        ("head_dim", "head_dim"),
        ("block_size", "block_size"),
        ("dtype", "dtype"),
        ("block_size_zero", "block_size must be > 0"),
        ("cache_shape", "cache shape"),
    ],
)
def test_validation_messages(pool, case, match):
    # test_cache_write.py:380-465
    kc, vc = pool
    k, v = _kv(1)
    slots, bs = torch.tensor([0]), 4
    if case == "value_dim":
        v = torch.randn(1, 2, 9).half()
    elif case == "slot_len":
        k, v = _kv(2)
    elif case == "heads":
        k, v = _kv(1, heads=4)
    elif case == "head_dim":
        k, v = _kv(1, dim=16)
    elif case == "block_size":
        bs = 8
    elif case == "dtype":
        k, v = _kv(1, dtype=torch.float32)
    elif case == "block_size_zero":
        bs = 0
    elif case == "cache_shape":
        vc = torch.empty(2, 2, 4, 8, dtype=torch.float16)
    with pytest.raises(ValueError, match=match):
        write_to_paged_cache(k, v, kc, vc, slots, bs)


def test_in_place(pool):
    # test_cache_write.py:472-484
    kc, vc = pool
    ptr = kc.data_ptr()
    k, v = _kv(1)
    write_to_paged_cache(k, v, kc, vc, torch.tensor([5]), 4)
    assert kc.data_ptr() == ptr


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_matches_numpy_token_loop(dtype):
    g = torch.Generator().manual_seed(7)
    kc = torch.randn(16, 3, 8, 32, generator=g).to(dtype)
    vc = torch.randn(16, 3, 8, 32, generator=g).to(dtype)
    k = torch.randn(40, 3, 32, generator=g).to(dtype)
    v = torch.randn(40, 3, 32, generator=g).to(dtype)
    slots = torch.randperm(16 * 8, generator=g)[:40]
    slots[::7] = -1
    ek, ev = brute.write(k.float().numpy(), v.float().numpy(), kc.float().numpy(),
                         vc.float().numpy(), slots.numpy(), 8)
    write_to_paged_cache(k, v, kc, vc, slots, 8)
    np.testing.assert_array_equal(kc.float().numpy(), ek)
    np.testing.assert_array_equal(vc.float().numpy(), ev)
