"""Pins the decode oracle (oracle.paged_ref) and the fp64 brute force.

Closed forms that a plausible slip (wrong GQA index, wrong scale, an
off-by-one in the block/offset walk, reading past kv_len) would break are
checked against BOTH implementations; random and reference-style cases
then check the two against each other.
"""

import math

import numpy as np
import pytest
import torch

from oracle import brute, paged_ref


def _run_both(q, kc, vc, bt, kv_len, bs):
    ref = paged_ref.decode_from_tables(q, kc, vc, bt, torch.as_tensor(kv_len), bs)
    bf = brute.decode(q.double().numpy(), kc.double().numpy(), vc.double().numpy(),
                      bt.numpy(), np.asarray(kv_len), bs)
    return ref.double().numpy(), bf


def _nan_pool(nb, hkv, bs, d):
    return (torch.full((nb, hkv, bs, d), float("nan")),
            torch.full((nb, hkv, bs, d), float("nan")))


def test_kv_len_one_returns_v_row_of_grouped_kv_head():
    """kv_len 1: softmax over one token is 1, out = that token's V row of
    kv head h // n_rep (repeat_interleave grouping, paged_attention_ref.py:146-147)."""
    hq, hkv, d, bs = 8, 2, 16, 4
    kc, vc = _nan_pool(6, hkv, bs, d)
    g = torch.Generator().manual_seed(1)
    kc[3, :, 0] = torch.randn(hkv, d, generator=g)
    vc[3, :, 0] = torch.arange(hkv * d, dtype=torch.float32).view(hkv, d)
    q = torch.randn(1, hq, d, generator=g)
    bt = torch.tensor([[3, -1]])
    ref, bf = _run_both(q, kc, vc, bt, [1], bs)
    want = np.stack([vc[3, h // (hq // hkv), 0].numpy() for h in range(hq)])
    np.testing.assert_array_equal(ref[0], want)
    np.testing.assert_allclose(bf[0], want, rtol=0, atol=1e-12)
    # a modulo mapping (h % hkv) would give a different answer here
    wrong = np.stack([vc[3, h % hkv, 0].numpy() for h in range(hq)])
    assert not np.allclose(want, wrong)


def test_equal_keys_give_mean_of_attended_values():
    """All keys equal -> uniform weights -> out = mean of the first kv_len
    V rows; rows past kv_len are NaN, so reading them would show."""
    hq, hkv, d, bs, kv_len = 4, 1, 8, 4, 10
    kc, vc = _nan_pool(8, hkv, bs, d)
    table = [5, 2, 7]
    g = torch.Generator().manual_seed(2)
    key_row = torch.randn(d, generator=g)
    rows = []
    for j in range(kv_len):
        b, o = table[j // bs], j % bs
        kc[b, 0, o] = key_row
        vc[b, 0, o] = torch.randn(d, generator=g)
        rows.append(vc[b, 0, o].clone())
    q = torch.randn(1, hq, d, generator=g)
    ref, bf = _run_both(q, kc, vc, torch.tensor([table + [-1]]), [kv_len], bs)
    want = torch.stack(rows).double().mean(0).numpy()
    for h in range(hq):
        np.testing.assert_allclose(ref[0, h], want, atol=1e-6)
        np.testing.assert_allclose(bf[0, h], want, atol=1e-12)


def test_two_token_closed_form_pins_scale():
    """q = e0, k1 = 2 e0, k2 = 0, head_dim 4 -> logits (1, 0) under scale
    4 ** -0.5, weight of token 1 = sigmoid(1) = 0.7310585786300049
    (scale 1 would give sigmoid(2) = 0.8807970779778823)."""
    d, bs = 4, 2
    kc, vc = _nan_pool(2, 1, bs, d)
    kc[1, 0, 0] = torch.tensor([2.0, 0, 0, 0])
    kc[1, 0, 1] = torch.zeros(4)
    vc[1, 0, 0] = torch.tensor([1.0, 0, 0, 0])
    vc[1, 0, 1] = torch.tensor([0.0, 1, 0, 0])
    q = torch.tensor([[[1.0, 0, 0, 0]]])
    ref, bf = _run_both(q, kc, vc, torch.tensor([[1]]), [2], bs)
    w = 0.7310585786300049
    want = np.array([w, 1 - w, 0, 0])
    np.testing.assert_allclose(ref[0, 0], want, atol=1e-7)
    np.testing.assert_allclose(bf[0, 0], want, atol=1e-15)


def test_dominant_logit_selects_its_value_row():
    """One key aligned with q at large norm -> output equals its V row."""
    hq, hkv, d, bs, n = 2, 1, 32, 16, 37
    g = torch.Generator().manual_seed(3)
    kc = torch.randn(4, hkv, bs, d, generator=g)
    vc = torch.randn(4, hkv, bs, d, generator=g)
    q = torch.randn(1, hq, d, generator=g)
    q[0, 1] = q[0, 0]
    table = [2, 0, 3]
    # token 21 -> logical block 1 -> physical block 0, offset 5
    kc[0, 0, 5] = q[0, 0] * 50.0
    ref, bf = _run_both(q, kc, vc, torch.tensor([table]), [n], bs)
    for h in range(hq):
        np.testing.assert_allclose(ref[0, h], vc[0, 0, 5].double().numpy(), atol=1e-6)
        np.testing.assert_allclose(bf[0, h], vc[0, 0, 5].double().numpy(), atol=1e-9)


def test_gather_follows_table_order():
    """Non-contiguous table [7, 3, 15] (test_paged_attention_ref.py:193-199):
    gathered token j is K[table[j // bs], :, j % bs]."""
    bs = 4
    kc = torch.arange(16 * 2 * bs * 3, dtype=torch.float32).view(16, 2, bs, 3)
    vc = -kc
    k, v = paged_ref.gather_paged_kv(kc, vc, [7, 3, 15], 10, bs)
    for j in range(10):
        assert torch.equal(k[j], kc[[7, 3, 15][j // bs], :, j % bs])
        assert torch.equal(v[j], vc[[7, 3, 15][j // bs], :, j % bs])
    with pytest.raises(IndexError, match="insufficient"):
        paged_ref.gather_paged_kv(kc, vc, [0], 8, bs)
    e, _ = paged_ref.gather_paged_kv(kc, vc, [], 0, bs)
    assert e.shape == (0, 2, 3)


def test_minus_one_padding_is_dropped():
    """Row [b0, b1, -1, -1]: the -1 entries never reach the gather
    (paged_attention_ref.py:137-138)."""
    g = torch.Generator().manual_seed(4)
    kc, vc = torch.randn(8, 2, 4, 8, generator=g), torch.randn(8, 2, 4, 8, generator=g)
    q = torch.randn(1, 4, 8, generator=g)
    a, _ = _run_both(q, kc, vc, torch.tensor([[6, 1, -1, -1]]), [7], 4)
    b, _ = _run_both(q, kc, vc, torch.tensor([[6, 1]]), [7], 4)
    np.testing.assert_array_equal(a, b)


def _ramp(shape, base):
    """Deterministic ramp of the reference GPU tests (test_paged_attention_gpu.py:118-124)."""
    n = int(np.prod(shape))
    return (base + torch.arange(n, dtype=torch.float32)).view(*shape)


def test_reference_gpu_style_ramp_batch():
    """Ragged batch [5, 17, 32, 50] with ramp values (huge logits, one-hot
    softmax) — the reference GPU suite's inputs (:520-539)."""
    bs, hq, hkv, d = 16, 4, 2, 64
    kc, vc = _nan_pool(256, hkv, bs, d)
    rows = []
    for i, n in enumerate([5, 17, 32, 50]):
        blocks = list(range(i * 32, i * 32 + -(-n // bs)))
        k = _ramp((n, hkv, d), 10.0 + i * 100)
        v = _ramp((n, hkv, d), 1010.0 + i * 100)
        paged_ref.write_to_paged_cache(k, v, kc, vc, torch.tensor(
            [blocks[j // bs] * bs + j % bs for j in range(n)]), bs)
        rows.append(blocks + [-1] * (4 - len(blocks)))
    q = _ramp((4, hq, d), 50.0)
    ref, bf = _run_both(q, kc, vc, torch.tensor(rows), [5, 17, 32, 50], bs)
    np.testing.assert_allclose(ref, bf, rtol=1e-5, atol=1e-3)  # values ~1e5: fp32 ulp ~1e-2


@pytest.mark.parametrize("hq,hkv,d,bs", [(14, 2, 64, 16), (28, 4, 128, 16), (8, 8, 64, 8),
                                         (16, 1, 64, 32), (4, 2, 128, 1)])
def test_random_oracle_matches_fp64(hq, hkv, d, bs):
    g = torch.Generator().manual_seed(hq * 1000 + d + bs)
    lens = [1, bs, bs + 1, 3 * bs + 5, 2 * bs - 1]
    nb = sum(-(-n // bs) for n in lens) + 3
    kc = torch.randn(nb, hkv, bs, d, generator=g)
    vc = torch.randn(nb, hkv, bs, d, generator=g)
    perm = torch.randperm(nb, generator=g).tolist()
    rows, it, mx = [], iter(perm), max(-(-n // bs) for n in lens)
    for n in lens:
        r = [next(it) for _ in range(-(-n // bs))]
        rows.append(r + [-1] * (mx - len(r)))
    q = torch.randn(len(lens), hq, d, generator=g)
    ref, bf = _run_both(q, kc, vc, torch.tensor(rows), lens, bs)
    assert np.abs(ref - bf).max() < 1e-5


def test_golden_c1_fixture():
    """The committed c1 fixture (tests/golden/make_golden.py): the oracle
    reproduces it and the fp64 brute force agrees within 1e-5."""
    import os

    path = os.path.join(os.path.dirname(__file__), "golden", "c1_decode.npz")
    z = np.load(path)
    kc, vc = torch.from_numpy(z["key_cache"]), torch.from_numpy(z["value_cache"])
    q, bt, kv = torch.from_numpy(z["query"]), torch.from_numpy(z["block_table"]), torch.from_numpy(z["kv_len"])
    # the fixture's pool is the state after the KV write of the new tokens
    out = paged_ref.decode_from_tables(q, kc, vc, bt, kv, int(z["block_size"]))
    np.testing.assert_allclose(out.numpy(), z["out"], rtol=0, atol=1e-6)
    bf = brute.decode(z["query"], z["key_cache"], z["value_cache"], z["block_table"], z["kv_len"],
                      int(z["block_size"]))
    assert np.abs(bf - z["out"]).max() < 1e-5
    assert not np.isnan(z["out"]).any()
