"""The oracle's chunked prefill (reference paged_attention_ref.py:167-244)
against closed forms and a float64 brute force with explicit causal
positions (oracle/brute.py)."""

import numpy as np
import torch

from oracle import brute, paged_ref


def _pool(seed, nb=12, hkv=2, bs=4, d=8):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(nb, hkv, bs, d, generator=g, dtype=torch.float64),
            torch.randn(nb, hkv, bs, d, generator=g, dtype=torch.float64), g)


def test_first_token_of_fresh_sequence_returns_its_own_value_row():
    kc, vc, g = _pool(0)
    bt = torch.tensor([[5, 2, -1]])
    q = torch.randn(3, 4, 8, generator=g, dtype=torch.float64)  # Hq 4, Hkv 2
    out = paged_ref.prefill_attention(q, kc, vc, bt, [0], [0], [3], 4)
    # token 0 attends only position 0 (block 5, offset 0); head h reads kv head h // 2
    for h in range(4):
        assert torch.allclose(out[0, h], vc[5, h // 2, 0], atol=1e-12)


def test_single_token_chunk_equals_decode():
    kc, vc, g = _pool(1)
    bt = torch.tensor([[3, 7, 1, -1]])
    q = torch.randn(1, 4, 8, generator=g, dtype=torch.float64)
    pre = paged_ref.prefill_attention(q, kc, vc, bt, [0], [9], [1], 4)
    dec = paged_ref.decode_attention(q, kc, vc, bt, [0], torch.tensor([9]), 4)
    assert torch.allclose(pre, dec, atol=1e-12)


def test_random_chunks_match_fp64_brute_force():
    kc, vc, g = _pool(2, nb=24)
    bt = torch.tensor([[0, 5, 9, 13, -1, -1], [2, 3, 17, 20, 21, -1], [11, -1, -1, -1, -1, -1]])
    seqs, cached, qlen = [2, 0, 1], [1, 6, 9], [2, 7, 8]
    q = torch.randn(sum(qlen), 4, 8, generator=g, dtype=torch.float64)
    out = paged_ref.prefill_attention(q, kc, vc, bt, seqs, cached, qlen, 4)
    ref = brute.prefill(q.numpy(), kc.numpy(), vc.numpy(), bt.numpy(), seqs, cached, qlen, 4)
    assert np.abs(out.numpy() - ref).max() < 1e-12


def test_causal_mask_excludes_future_positions():
    """Changing V at a position after the query's own leaves that row alone."""
    kc, vc, g = _pool(3)
    bt = torch.tensor([[4, 8, -1]])
    q = torch.randn(5, 2, 8, generator=g, dtype=torch.float64)  # Hq 2 (n_rep 1)
    a = paged_ref.prefill_attention(q, kc, vc, bt, [0], [2], [5], 4)
    vc2 = vc.clone()
    vc2[8, :, 2] += 100.0  # position 6 = last query token's own position
    b = paged_ref.prefill_attention(q, kc, vc2, bt, [0], [2], [5], 4)
    assert torch.equal(a[:4], b[:4])
    assert not torch.allclose(a[4], b[4])


def test_chunk_argument_form_equals_pool_form_after_write():
    """The GPU backend's form (prefix from the pool, chunk K/V from the
    arguments) equals the pool-only form once the chunk has been written
    to its slots -- the runner's write-first order."""
    kc, vc, g = _pool(5, nb=30)
    bs = 4
    bt = torch.tensor([[7, 1, 22, 4, 9, -1], [3, 28, 15, 11, 0, 2], [5, 6, -1, -1, -1, -1]])
    seqs, cached, qlen = [1, 0, 2], [6, 0, 3], [13, 10, 4]
    q = torch.randn(sum(qlen), 4, 8, generator=g, dtype=torch.float64)
    k = torch.randn(sum(qlen), 2, 8, generator=g, dtype=torch.float64)
    v = torch.randn(sum(qlen), 2, 8, generator=g, dtype=torch.float64)
    got = paged_ref.prefill_attention_chunk_args(q, k, v, kc, vc, bt, seqs, cached, qlen, bs)
    kc2, vc2 = kc.clone(), vc.clone()
    slots, off = [], 0
    for s, c, ql in zip(seqs, cached, qlen):
        for t in range(ql):
            p = c + t
            slots.append(int(bt[s, p // bs]) * bs + p % bs)
    paged_ref.write_to_paged_cache(k, v, kc2, vc2, torch.tensor(slots), bs)
    want = paged_ref.prefill_attention(q, kc2, vc2, bt, seqs, cached, qlen, bs)
    assert torch.allclose(got, want, atol=1e-12)
    ref = brute.prefill(q.numpy(), kc2.numpy(), vc2.numpy(), bt.numpy(), seqs, cached, qlen, bs)
    assert np.abs(got.numpy() - ref).max() < 1e-10
