"""Restatement of the reference's PyTorch paged-attention path (the oracle).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg; never by the product.

Each function cites the reference lines it restates. Loop structure is kept
(per token for the write, per sequence for the decode) because this module
is also the CPU baseline that bench.py times.
"""

from __future__ import annotations

from typing import List, Sequence, Tuple

import torch
import torch.nn.functional as F


# ---------------------------------------------------------------------------
# KV write — mini_vllm/cache/cache_write.py:25-140
# ---------------------------------------------------------------------------


def _validate_write(key, value, key_cache, value_cache, slot_mapping, block_size) -> None:
    """Input checks of ``_validate_inputs`` (cache_write.py:82-140), same order."""
    if key.shape != value.shape:
        raise ValueError(f"key shape {tuple(key.shape)} != value shape {tuple(value.shape)}")
    if key_cache.shape != value_cache.shape:
        raise ValueError(
            f"key_cache shape {tuple(key_cache.shape)} != value_cache shape "
            f"{tuple(value_cache.shape)}"
        )
    if block_size <= 0:
        raise ValueError(f"block_size must be > 0, got {block_size}")
    n_tok, n_kv, hd = key.shape
    _, n_kv_c, bs_c, hd_c = key_cache.shape
    if len(slot_mapping) != n_tok:
        raise ValueError(f"slot_mapping length {len(slot_mapping)} != num_tokens {n_tok}")
    if n_kv != n_kv_c:
        raise ValueError(f"key num_kv_heads {n_kv} != key_cache num_kv_heads {n_kv_c}")
    if hd != hd_c:
        raise ValueError(f"key head_dim {hd} != key_cache head_dim {hd_c}")
    if block_size != bs_c:
        raise ValueError(f"block_size argument {block_size} != key_cache block_size dim {bs_c}")
    if key.dtype != key_cache.dtype:
        raise ValueError(f"key dtype {key.dtype} != key_cache dtype {key_cache.dtype}")
    if value.dtype != value_cache.dtype:
        raise ValueError(f"value dtype {value.dtype} != value_cache dtype {value_cache.dtype}")
    if key.device != key_cache.device:
        raise ValueError(f"key device {key.device} != key_cache device {key_cache.device}")
    if value.device != value_cache.device:
        raise ValueError(f"value device {value.device} != value_cache device {value_cache.device}")


def write_to_paged_cache(
    key: torch.Tensor,
    value: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    block_size: int,
) -> None:
    """Per-token scatter (cache_write.py:25-74).

    slot -1 skips; a slot outside [0, num_blocks*block_size) raises
    IndexError at that token (earlier tokens stay written); duplicate slots
    resolve to the last writer.
    """
    _validate_write(key, value, key_cache, value_cache, slot_mapping, block_size)
    total_slots = key_cache.shape[0] * block_size
    for t in range(key.shape[0]):
        slot = int(slot_mapping[t].item())
        if slot == -1:
            continue
        if slot < -1 or slot >= total_slots:
            raise IndexError(
                f"slot_mapping[{t}] = {slot} out of range [0, {total_slots}) "
                f"(block_size={block_size}, num_blocks={key_cache.shape[0]})"
            )
        blk, off = divmod(slot, block_size)
        key_cache[blk, :, off, :] = key[t]
        value_cache[blk, :, off, :] = value[t]


# ---------------------------------------------------------------------------
# Gather — mini_vllm/cache/cache_read.py:19-84
# ---------------------------------------------------------------------------


def gather_paged_kv(
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: List[int],
    num_tokens: int,
    block_size: int,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Logical block i -> physical block_table[i], min(block_size, remaining)
    tokens per block, ``[Hkv, T, D] -> [T, Hkv, D]``; IndexError with
    "insufficient" when the table is too short."""
    _, n_kv, _, hd = key_cache.shape
    if num_tokens == 0:
        e = torch.empty(0, n_kv, hd, dtype=key_cache.dtype, device=key_cache.device)
        return e, e.clone()
    ks, vs = [], []
    remaining, i = num_tokens, 0
    while remaining > 0:
        if i >= len(block_table):
            raise IndexError(
                f"block_table length {len(block_table)} insufficient to cover {num_tokens} "
                f"tokens (logical_idx={i}, block_size={block_size})"
            )
        n = min(block_size, remaining)
        ks.append(key_cache[block_table[i], :, :n, :].permute(1, 0, 2))
        vs.append(value_cache[block_table[i], :, :n, :].permute(1, 0, 2))
        remaining -= n
        i += 1
    return torch.cat(ks, dim=0), torch.cat(vs, dim=0)


# ---------------------------------------------------------------------------
# Decode — mini_vllm/attention/paged_attention_ref.py:102-161
# ---------------------------------------------------------------------------


def decode_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_indices: Sequence[int],
    cached_len_before: torch.Tensor,
    block_size: int,
) -> torch.Tensor:
    """``AttentionBackendRef.decode_attention`` for one layer.

    For decode row i: kv_len = cached_len_before[i] + 1; the table row is
    ``block_tables[seq_indices[i]]`` with its -1 entries dropped; K/V are
    gathered, expanded to the query heads with ``repeat_interleave`` (query
    head h reads kv head h // n_rep) and fed to SDPA with scale
    head_dim ** -0.5 and no mask. Returns ``[B, Hq, D]`` in query's dtype.
    """
    num_decode, num_heads, head_dim = query.shape
    if num_decode == 0:
        return query
    n_rep = num_heads // key_cache.shape[1]
    scale = head_dim ** -0.5
    outs = []
    for i in range(num_decode):
        kv_len = int(cached_len_before[i].item()) + 1
        row = block_tables[seq_indices[i]]
        ids = [int(b.item()) for b in row if b.item() != -1]
        k, v = gather_paged_kv(key_cache, value_cache, ids, kv_len, block_size)
        k = k.repeat_interleave(n_rep, dim=1)
        v = v.repeat_interleave(n_rep, dim=1)
        o = F.scaled_dot_product_attention(
            query[i].unsqueeze(0).unsqueeze(2),
            k.permute(1, 0, 2).unsqueeze(0),
            v.permute(1, 0, 2).unsqueeze(0),
            scale=scale,
            is_causal=False,
        )
        outs.append(o.squeeze(2))
    return torch.cat(outs, dim=0)


def decode_from_tables(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    kv_len_after: torch.Tensor,
    block_size: int,
) -> torch.Tensor:
    """Decode with the GPU entry point's arguments (row i <-> sequence i,
    ``kv_len_after = cached_len_before + 1``), as the reference GPU tests'
    ``_decode_ref`` does (tests/test_paged_attention_gpu.py:127-151)."""
    b = query.shape[0]
    cached = kv_len_after.to(torch.int64) - 1
    return decode_attention(query, key_cache, value_cache, block_table, list(range(b)), cached,
                            block_size)


def prefill_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_indices: Sequence[int],
    cached_len_before: Sequence[int],
    query_len: Sequence[int],
    block_size: int,
) -> torch.Tensor:
    """``AttentionBackendRef.prefill_attention`` (paged_attention_ref.py:167-244):
    gather cached + chunk tokens from the pool, causal mask
    ``key_pos <= query_pos`` with query positions offset by the cached
    length, SDPA per sequence."""
    num_heads, head_dim = query.shape[1], query.shape[2]
    n_rep = num_heads // key_cache.shape[1]
    scale = head_dim ** -0.5
    outs, off = [], 0
    for i, s in enumerate(seq_indices):
        c, ql = int(cached_len_before[i]), int(query_len[i])
        kv_len = c + ql
        ids = [int(b) for b in block_tables[int(s)].tolist() if b != -1]
        k, v = gather_paged_kv(key_cache, value_cache, ids, kv_len, block_size)
        k = k.repeat_interleave(n_rep, dim=1)
        v = v.repeat_interleave(n_rep, dim=1)
        mask = torch.arange(kv_len).unsqueeze(0) <= torch.arange(c, c + ql).unsqueeze(1)
        o = F.scaled_dot_product_attention(
            query[off:off + ql].permute(1, 0, 2).unsqueeze(0),
            k.permute(1, 0, 2).unsqueeze(0),
            v.permute(1, 0, 2).unsqueeze(0),
            attn_mask=mask,
            is_causal=False,
            scale=scale,
        )
        outs.append(o.squeeze(0).permute(1, 0, 2))
        off += ql
    return torch.cat(outs, dim=0)


def prefill_attention_chunk_args(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_indices: Sequence[int],
    cached_len_before: Sequence[int],
    query_len: Sequence[int],
    block_size: int,
) -> torch.Tensor:
    """``AttentionBackendGPU.prefill_attention`` (paged_attention_gpu.py:
    577-661): the cached prefix from the pool (gather of ``cached`` tokens),
    the chunk's keys / values from ``key`` / ``value`` (rows in sequence
    order), ``cat``, ``repeat_interleave`` to the query heads, SDPA with the
    offset causal mask ``key_pos <= cached + t``."""
    num_heads, head_dim = query.shape[1], query.shape[2]
    n_rep = num_heads // key_cache.shape[1]
    scale = head_dim ** -0.5
    outs, off = [], 0
    for i, s in enumerate(seq_indices):
        c, ql = int(cached_len_before[i]), int(query_len[i])
        if c > 0:
            ids = [int(b) for b in block_tables[int(s)].tolist() if b != -1]
            pk, pv = gather_paged_kv(key_cache, value_cache, ids, c, block_size)
        else:
            pk = key_cache.new_empty(0, key_cache.shape[1], head_dim)
            pv = pk.clone()
        k = torch.cat([pk, key[off:off + ql]], dim=0).repeat_interleave(n_rep, dim=1)
        v = torch.cat([pv, value[off:off + ql]], dim=0).repeat_interleave(n_rep, dim=1)
        mask = torch.arange(c + ql).unsqueeze(0) <= torch.arange(c, c + ql).unsqueeze(1)
        o = F.scaled_dot_product_attention(
            query[off:off + ql].permute(1, 0, 2).unsqueeze(0),
            k.permute(1, 0, 2).unsqueeze(0),
            v.permute(1, 0, 2).unsqueeze(0),
            attn_mask=mask,
            is_causal=False,
            scale=scale,
        )
        outs.append(o.squeeze(0).permute(1, 0, 2))
        off += ql
    return torch.cat(outs, dim=0)
