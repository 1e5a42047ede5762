"""Seeded synthetic decode-step workloads at the benchmark shapes.

A workload is one decode step of one layer: every sequence has
``kv_len - 1`` cached tokens in a paged pool and writes its new token's K/V
at position ``kv_len - 1`` (slot ``bt[b, (kv_len-1) // bs] * bs +
(kv_len-1) % bs``), then attends over ``kv_len`` tokens.

Configurations (Qwen2-0.5B attention: 14 query heads, 2 kv heads,
head_dim 64; block_size 16 throughout):

  c1  fp32, batch 4, kv_len {17, 64, 130, 255}, pool 256 blocks, tables
      drawn without replacement from the pool (the CPU-runnable case)
  c2  bf16, batch 64, kv_len ~ U{128..2048}, pool = needed blocks + 10 %,
      randomly permuted tables (headline benchmark)
  c3  bf16, batch 16, kv_len ~ U{8192..32768} (long context, many partitions)
  c4  bf16, batch 256, kv_len = clip(round(lognormal(ln 300, 1.0)), 1, 8192);
      groups of 8 sequences share their first min(4, (kv_len-1)//16)
      physical blocks (prefix sharing), so every written slot is private
  c5  bf16, 28 query / 4 kv heads, head_dim 128, batch 128,
      kv_len ~ U{512..4096}, 1 % of K entries scaled x8

Values are N(0, 1) from ``torch.Generator().manual_seed(seed)`` (CPU) in
the order: table permutation, K pool, V pool, query, new K, new V. With
``nan_fill`` every pool slot no sequence reads (and every slot about to be
written) holds NaN, so a read outside the attended range or a missing write
poisons the result.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np
import torch


@dataclass(frozen=True)
class WorkloadSpec:
    name: str
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    dtype: torch.dtype
    batch: int
    ctx: tuple                   # ("fixed", [..]) | ("uniform", lo, hi) | ("lognormal", median, sigma, lo, hi)
    pool_blocks: Optional[int] = None   # fixed pool size, else needed * pool_slack
    pool_slack: float = 1.10
    share_group: int = 0         # sequences per prefix-sharing group (0 = none)
    share_blocks: int = 0        # shared leading blocks per group
    k_outlier_frac: float = 0.0  # fraction of K entries scaled by k_outlier_scale
    k_outlier_scale: float = 1.0


SPECS: Dict[str, WorkloadSpec] = {
    "c1": WorkloadSpec("c1", 14, 2, 64, 16, torch.float32, 4, ("fixed", [17, 64, 130, 255]),
                       pool_blocks=256),
    "c2": WorkloadSpec("c2", 14, 2, 64, 16, torch.bfloat16, 64, ("uniform", 128, 2048)),
    "c3": WorkloadSpec("c3", 14, 2, 64, 16, torch.bfloat16, 16, ("uniform", 8192, 32768)),
    "c4": WorkloadSpec("c4", 14, 2, 64, 16, torch.bfloat16, 256, ("lognormal", 300, 1.0, 1, 8192),
                       share_group=8, share_blocks=4),
    "c5": WorkloadSpec("c5", 28, 4, 128, 16, torch.bfloat16, 128, ("uniform", 512, 4096),
                       k_outlier_frac=0.01, k_outlier_scale=8.0),
}

HEADLINE = "c2"


def context_lengths(spec: WorkloadSpec, seed: int) -> List[int]:
    kind = spec.ctx[0]
    if kind == "fixed":
        return list(spec.ctx[1])
    rs = np.random.RandomState(seed)
    if kind == "uniform":
        return [int(x) for x in rs.randint(spec.ctx[1], spec.ctx[2] + 1, size=spec.batch)]
    if kind == "lognormal":
        median, sigma, lo, hi = spec.ctx[1:]
        x = np.round(rs.lognormal(math.log(median), sigma, size=spec.batch))
        return [int(v) for v in np.clip(x, lo, hi)]
    raise ValueError(kind)


@dataclass
class Layout:
    """Block tables and pool size of a workload (no tensor data)."""

    spec: WorkloadSpec
    kv_lens: List[int]
    rows: List[List[int]]
    num_blocks: int
    shared_blocks: int = 0   # physical blocks referenced by more than one row

    @property
    def max_blocks(self) -> int:
        return max(len(r) for r in self.rows)

    def block_table(self) -> torch.Tensor:
        bt = torch.full((len(self.rows), self.max_blocks), -1, dtype=torch.int64)
        for i, r in enumerate(self.rows):
            bt[i, : len(r)] = torch.tensor(r, dtype=torch.int64)
        return bt

    def new_token_slots(self) -> torch.Tensor:
        bs = self.spec.block_size
        return torch.tensor(
            [r[(n - 1) // bs] * bs + (n - 1) % bs for r, n in zip(self.rows, self.kv_lens)],
            dtype=torch.int64,
        )


def make_layout(spec: WorkloadSpec, seed: int = 0, generator: Optional[torch.Generator] = None) -> Layout:
    bs = spec.block_size
    lens = context_lengths(spec, seed)
    need = [-(-n // bs) for n in lens]
    g = generator if generator is not None else torch.Generator().manual_seed(seed)
    if spec.share_group:
        # per group: `share_blocks` shared ids, then private ids per sequence
        shared_use = [min(spec.share_blocks, (n - 1) // bs) for n in lens]
        groups = [list(range(i, min(i + spec.share_group, len(lens))))
                  for i in range(0, len(lens), spec.share_group)]
        total = sum(spec.share_blocks for _ in groups) + sum(
            k - s for k, s in zip(need, shared_use))
    else:
        total = sum(need)
    num_blocks = spec.pool_blocks or int(math.ceil(total * spec.pool_slack))
    perm = torch.randperm(num_blocks, generator=g).tolist()
    it = iter(perm)
    rows: List[List[int]] = []
    shared_count = 0
    if spec.share_group:
        rows = [[] for _ in lens]
        for grp in groups:
            shared = [next(it) for _ in range(spec.share_blocks)]
            shared_count += spec.share_blocks
            for i in grp:
                rows[i] = shared[: shared_use[i]] + [next(it) for _ in range(need[i] - shared_use[i])]
    else:
        rows = [[next(it) for _ in range(k)] for k in need]
    return Layout(spec, lens, rows, num_blocks, shared_count)


@dataclass
class DecodeCase:
    """Tensors of one decode step (on ``device``)."""

    layout: Layout
    query: torch.Tensor          # [B, Hq, D]
    key_cache: torch.Tensor      # [NB, Hkv, BS, D] (before the write)
    value_cache: torch.Tensor
    new_key: torch.Tensor        # [B, Hkv, D]
    new_value: torch.Tensor
    slot_mapping: torch.Tensor   # [B] int64
    block_table: torch.Tensor    # [B, max_blocks] int64
    kv_len: torch.Tensor         # [B] int64 (kv_len_after)
    extra: dict = field(default_factory=dict)


def live_slot_mask(layout: Layout) -> torch.Tensor:
    """[num_blocks, block_size] bool: slots some sequence reads before the write."""
    bs = layout.spec.block_size
    live = torch.zeros(layout.num_blocks * bs, dtype=torch.bool)
    for r, n in zip(layout.rows, layout.kv_lens):
        if n <= 1:
            continue
        ids = torch.tensor(r, dtype=torch.int64)
        j = torch.arange(n - 1)
        live[ids[j // bs] * bs + j % bs] = True
    return live.view(layout.num_blocks, bs)


def make_case(
    spec: WorkloadSpec | str,
    seed: int = 0,
    device: torch.device | str = "cpu",
    dtype: Optional[torch.dtype] = None,
    nan_fill: bool = False,
) -> DecodeCase:
    """Materialise a workload; values are generated in fp32 on the CPU, then
    rounded to ``dtype`` (default: the spec's)."""
    if isinstance(spec, str):
        spec = SPECS[spec]
    dtype = dtype or spec.dtype
    g = torch.Generator().manual_seed(seed)
    layout = make_layout(spec, seed, g)
    nb, hkv, bs, d, hq, b = (layout.num_blocks, spec.num_kv_heads, spec.block_size,
                             spec.head_dim, spec.num_q_heads, len(layout.kv_lens))
    kc = torch.randn(nb, hkv, bs, d, generator=g)
    vc = torch.randn(nb, hkv, bs, d, generator=g)
    q = torch.randn(b, hq, d, generator=g)
    nk = torch.randn(b, hkv, d, generator=g)
    nv = torch.randn(b, hkv, d, generator=g)
    if spec.k_outlier_frac > 0:
        mask = torch.rand(kc.shape, generator=g) < spec.k_outlier_frac
        kc = torch.where(mask, kc * spec.k_outlier_scale, kc)
        nmask = torch.rand(nk.shape, generator=g) < spec.k_outlier_frac
        nk = torch.where(nmask, nk * spec.k_outlier_scale, nk)
    if nan_fill:
        dead = ~live_slot_mask(layout)                      # [nb, bs]
        dead = dead.view(nb, 1, bs, 1).expand(nb, hkv, bs, d)
        kc = kc.masked_fill(dead, float("nan"))
        vc = vc.masked_fill(dead, float("nan"))
    dev = torch.device(device)
    return DecodeCase(
        layout=layout,
        query=q.to(dtype).to(dev),
        key_cache=kc.to(dtype).to(dev),
        value_cache=vc.to(dtype).to(dev),
        new_key=nk.to(dtype).to(dev),
        new_value=nv.to(dtype).to(dev),
        slot_mapping=layout.new_token_slots().to(dev),
        block_table=layout.block_table().to(dev),
        kv_len=torch.tensor(layout.kv_lens, dtype=torch.int64).to(dev),
    )


def decode_bytes(layout: Layout, dtype: torch.dtype, unique: bool = False) -> int:
    """Algorithmic HBM bytes of the decode: K+V of attended tokens, Q in,
    O out, table entries read (8 bytes each) and the lengths (4 bytes each).
    ``unique`` counts each physical (block, kv head) token once (shared
    prefixes are read once from HBM in the ideal)."""
    s = layout.spec
    e = torch.empty((), dtype=dtype).element_size()
    bs = s.block_size
    if unique:
        per_block = {}
        for r, n in zip(layout.rows, layout.kv_lens):
            for j in range(-(-n // bs)):
                cnt = min(bs, n - j * bs)
                per_block[r[j]] = max(per_block.get(r[j], 0), cnt)
        toks = sum(per_block.values())
    else:
        toks = sum(layout.kv_lens)
    kv = toks * s.num_kv_heads * s.head_dim * 2 * e
    b = len(layout.kv_lens)
    qo = b * s.num_q_heads * s.head_dim * 2 * e
    tables = sum(-(-n // bs) for n in layout.kv_lens) * 8
    return kv + qo + tables + 4 * b


def write_bytes(layout: Layout, dtype: torch.dtype) -> int:
    """Algorithmic bytes of the KV write: new K+V read and written, 8-byte slots."""
    s = layout.spec
    e = torch.empty((), dtype=dtype).element_size()
    t = len(layout.kv_lens)
    return 2 * (2 * t * s.num_kv_heads * s.head_dim * e) + 8 * t
