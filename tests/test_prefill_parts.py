"""The prefill key split's plan (prefill_key_parts): which units are cut,
where, and into how many parts (host logic; the GPU tests check the
results)."""
import pytest

from mini_vllm.attention.paged_attention_gpu import (PREFILL_MAX_PARTS, PREFILL_PART_KEYS,
                                                     prefill_key_parts)


@pytest.mark.parametrize("key_ends,cus", [
    ([3600 + 16 * i for i in range(64)], 256),    # one long chunk: 64 units
    ([1552 + 16 * i for i in range(128)], 256),   # two sequences
    ([300, 5000, 513, 1024, 1, 256, 257], 256),   # ragged, tiny
    ([100000] * 3, 256),                           # a very long prefix
    ([4096] * 300, 256),                           # more units than CUs
    ([], 256),
])
def test_parts_tile_each_unit(key_ends, cus):
    parts = prefill_key_parts(key_ends, cus)
    assert len(parts) == len(key_ends)
    n = len(key_ends)
    cap = min(PREFILL_MAX_PARTS, cus // n) if 0 < n < cus else 1
    for ke, pr in zip(key_ends, parts):
        assert 1 <= len(pr) <= max(1, cap)
        assert pr[0][0] == 0 and pr[-1][1] == ke
        for (a, b), (c, _) in zip(pr, pr[1:]):
            assert b == c  # contiguous
        for a, b in pr:
            assert a % PREFILL_PART_KEYS == 0 and a < b
        if len(pr) > 1:  # every cut part holds at least two blocks of keys, but the last
            assert all(b - a >= 2 * PREFILL_PART_KEYS for a, b in pr[:-1])
            assert pr[-1][1] - pr[-1][0] > PREFILL_PART_KEYS


def test_split_only_when_units_leave_cus_idle():
    assert [len(p) for p in prefill_key_parts([4096] * 256, 256)] == [1] * 256
    assert [len(p) for p in prefill_key_parts([4096] * 128, 256)] == [2] * 128
    assert [len(p) for p in prefill_key_parts([4096] * 64, 256)] == [4] * 64
    assert [len(p) for p in prefill_key_parts([4096] * 2, 256)] == [PREFILL_MAX_PARTS] * 2
    # short units stay whole: a part needs two blocks of keys
    assert [len(p) for p in prefill_key_parts([511, 512, 1024], 256)] == [1, 1, 2]
    assert prefill_key_parts([4096] * 64, 256, max_parts=1) == [[(0, 4096)]] * 64


def test_parts_are_balanced():
    for ke in (4096, 3600, 2049, 100000):
        pr = prefill_key_parts([ke], 256)[0]
        sizes = [b - a for a, b in pr]
        assert max(sizes) - min(sizes) <= 2 * PREFILL_PART_KEYS
