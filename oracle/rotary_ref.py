"""Restatement of the reference's rotary embedding (the oracle for the
fused RoPE + KV write).

TEST INFRASTRUCTURE ONLY: imported by tests/ (and smoke()), never by the
product.

``RotaryTables`` follows ``RotaryEmbedding.__init__``
(mini_vllm/model/rotary.py:16-35): ``inv_freq = 1 / theta**(arange(0, D, 2)
/ D)``, angles ``t * inv_freq`` for ``t < max_seq_len``, duplicated to
``[.., D]``, ``cos`` / ``sin`` cast to the model dtype. ``rotary`` follows
``__call__`` + ``_rotate_half`` (:44-82): ``x * cos[pos] +
cat(-x2, x1) * sin[pos]`` as eager torch ops in the tensors' dtype (each op
rounds). ``rope_then_write`` is the runner's sequence (qwen_runner.py:
164-170): rotate q, rotate k, write k and v with the oracle's KV write.
"""

from __future__ import annotations

import torch

from .paged_ref import write_to_paged_cache


class RotaryTables:
    """cos / sin tables of ``RotaryEmbedding`` (rotary.py:16-35)."""

    def __init__(self, head_dim: int, theta: float = 1000000.0, max_seq_len: int = 32768,
                 dtype: torch.dtype = torch.float32) -> None:
        self.head_dim = head_dim
        inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
        t = torch.arange(max_seq_len, dtype=torch.float32)
        freqs = torch.outer(t, inv_freq)
        emb = torch.cat((freqs, freqs), dim=-1)
        self.cos = emb.cos().to(dtype)
        self.sin = emb.sin().to(dtype)


def rotary(x: torch.Tensor, positions: torch.Tensor, tables: RotaryTables) -> torch.Tensor:
    """``RotaryEmbedding.__call__`` (rotary.py:44-82) on ``x`` ``[T, H, D]``."""
    cos = tables.cos[positions].unsqueeze(-2)
    sin = tables.sin[positions].unsqueeze(-2)
    half = x.shape[-1] // 2
    rotated = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return x * cos + rotated * sin


def rope_then_write(q, k, v, positions, tables, key_cache, value_cache, slot_mapping, block_size):
    """The runner's three calls (qwen_runner.py:164-170) on CPU tensors:
    returns (q_rot, k_rot) and writes k_rot / v into the caches in place."""
    q_rot = rotary(q, positions, tables)
    k_rot = rotary(k, positions, tables)
    write_to_paged_cache(k_rot, v, key_cache, value_cache, slot_mapping, block_size)
    return q_rot, k_rot
