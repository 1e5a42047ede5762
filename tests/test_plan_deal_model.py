"""The closed forms decode_plan_wave_kernel builds its work list with,
checked on the CPU against brute force (no GPU, no library).

A sequence of T tiles cut into np = ceil(T / L) pieces gives piece j the
tiles [floor(j T / np), floor((j + 1) T / np)): r = T mod np pieces of
q + 1 tiles and np - r of q tiles (q = T div np). The kernel uses
* bb(j) = floor(j r / np) larger pieces before piece j, and piece j is a
  larger one iff (j r mod np) + r >= np;
* the i-th larger piece is j = ceil((i + 1) np / r) - 1 and the i-th
  smaller one j = floor(i np / (np - r)) (the inverse, slot -> piece);
* a group's deal position = its size bucket's start + the groups of the
  bucket in earlier sequences + its index among its sequence's groups of
  the bucket, then snake order over the CUs; the inverse walks back from a
  slot to (sequence, piece, kv head).
Each must be a bijection onto the slots, with sizes non-increasing by
position; a wrong floor/ceil or an off-by-one breaks one of the asserts.
"""

import random

import pytest


def _pieces(T, L):
    np_ = -(-T // L)
    return [((j * T) // np_, ((j + 1) * T) // np_) for j in range(np_)]


@pytest.mark.parametrize("seed", range(2))
def test_piece_counts_and_their_inverse(seed):
    rnd = random.Random(seed)
    for _ in range(3000):
        T, L = rnd.randint(1, 5000), rnd.randint(1, 600)
        pieces = _pieces(T, L)
        np_ = len(pieces)
        q, r = T // np_, T % np_
        big_idx, small_idx = [], []
        for j, (t0, t1) in enumerate(pieces):
            bb = (j * r) // np_
            big = (j * r) % np_ + r >= np_
            assert t0 == j * q + bb
            assert t1 - t0 == q + (1 if big else 0)
            assert bb == sum(1 for k in range(j) if pieces[k][1] - pieces[k][0] == q + 1)
            (big_idx if big else small_idx).append(j)
        assert len(big_idx) == r
        for i, j in enumerate(big_idx):
            assert -(-(i + 1) * np_ // r) - 1 == j
        for i, j in enumerate(small_idx):
            assert (i * np_) // (np_ - r) == j


def _deal(kvs, L, hkv, cus):
    """Forward positions and slots as the kernel computes them, and the inverse."""
    tiles = [-(-k // 16) for k in kvs]
    nps = [-(-t // L) for t in tiles]
    shift = 0
    while ((L - 1) >> shift) >= 64:
        shift += 1
    rows = []
    for t, n in zip(tiles, nps):
        q, r = (t // n, t % n) if n else (0, 0)
        kb = (L - q) >> shift if n else 0
        ka = (L - q - 1) >> shift if r else kb
        na, nb = (n * hkv, 0) if ka == kb else (r * hkv, (n - r) * hkv)
        rows.append(dict(n=n, q=q, r=r, ka=ka, kb=kb, na=na, nb=nb))
    cnt = [0] * 64
    for w in rows:
        cnt[w["ka"]] += w["na"]
        cnt[w["kb"]] += w["nb"]
    start = [sum(cnt[:k]) for k in range(64)]
    run = [0] * 64
    for w in rows:  # sequences in order within each bucket
        w["pa"] = start[w["ka"]] + run[w["ka"]]
        run[w["ka"]] += w["na"]
        w["pb"] = start[w["kb"]] + run[w["kb"]]
        run[w["kb"]] += w["nb"]
    G = sum(nps) * hkv
    rounds = -(-G // cus)

    def snake(pos):
        rd, c = divmod(pos, cus)
        return rd * cus + (c if ((rounds - 1 - rd) & 1) == 0 else cus - 1 - c)

    fwd = {}
    for b, w in enumerate(rows):
        for j in range(w["n"]):
            bb = (j * w["r"]) // w["n"]
            big = (j * w["r"]) % w["n"] + w["r"] >= w["n"]
            for h in range(hkv):
                pos = (w["pa"] + j * hkv + h if w["ka"] == w["kb"]
                       else w["pa"] + bb * hkv + h if big else w["pb"] + (j - bb) * hkv + h)
                fwd[snake(pos)] = (b, j, h, pos)

    def inverse(slot):
        pos = snake(slot)  # the snake order is its own inverse within a round
        k = next(k for k in range(64) if start[k] <= pos < start[k] + cnt[k])
        b, in_a = next((b, w["ka"] == k and w["pa"] <= pos < w["pa"] + w["na"])
                       for b, w in enumerate(rows)
                       if (w["ka"] == k and w["pa"] <= pos < w["pa"] + w["na"])
                       or (w["kb"] == k and w["pb"] <= pos < w["pb"] + w["nb"]))
        w = rows[b]
        idx = pos - (w["pa"] if in_a else w["pb"])
        i, h = divmod(idx, hkv)
        if w["ka"] == w["kb"]:
            j = i
        elif in_a:
            j = -(-(i + 1) * w["n"] // w["r"]) - 1
        else:
            j = (i * w["n"]) // (w["n"] - w["r"])
        return b, j, h

    return G, fwd, inverse, tiles, nps, shift


@pytest.mark.parametrize("seed", range(2))
def test_deal_is_a_sorted_bijection_with_an_inverse(seed):
    rnd = random.Random(100 + seed)
    for _ in range(150):
        B = rnd.randint(1, 64)
        hkv = rnd.choice([1, 2, 4, 8])
        top = rnd.choice([100, 2048, 32768])
        kvs = [rnd.randint(1, top) for _ in range(B)]
        L = rnd.randint(4, 200)
        cus = rnd.choice([256, 100, 7])
        G, fwd, inverse, tiles, nps, shift = _deal(kvs, L, hkv, cus)
        assert sorted(fwd) == list(range(G))
        by_pos = sorted(fwd.values(), key=lambda v: v[3])
        sizes = [_pieces(tiles[b], L)[j] for b, j, _, _ in by_pos]
        buckets = [(L - (t1 - t0)) >> shift for t0, t1 in sizes]
        assert buckets == sorted(buckets)
        for slot, (b, j, h, _) in fwd.items():
            assert inverse(slot) == (b, j, h)
