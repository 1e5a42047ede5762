"""Float64 numpy brute force of the decode step (pins oracle.paged_ref).

TEST INFRASTRUCTURE ONLY. Independent of paged_ref: explicit slot
arithmetic instead of the gather/cat/permute chain, explicit
max-subtracted softmax in float64 instead of torch SDPA, and an explicit
kv-head index instead of ``repeat_interleave``. The maths it states is the
definition the reference's decode implements
(mini_vllm/attention/paged_attention_ref.py:102-161):

    out[b, h] = sum_j softmax_j(scale * q[b, h] . k_j) v_j,
    k_j = K[bt[b, j // bs], h // n_rep, j % bs],   j < kv_len[b],
    scale = head_dim ** -0.5.
"""

from __future__ import annotations

import numpy as np


def write(key, value, key_cache, value_cache, slots, block_size):
    """Token loop of the KV write on numpy arrays (returns new caches)."""
    kc = np.array(key_cache, copy=True)
    vc = np.array(value_cache, copy=True)
    n_slots = kc.shape[0] * block_size
    for t, s in enumerate(np.asarray(slots).tolist()):
        if s == -1:
            continue
        if not 0 <= s < n_slots:
            raise IndexError(f"slot {s} out of range")
        kc[s // block_size, :, s % block_size, :] = key[t]
        vc[s // block_size, :, s % block_size, :] = value[t]
    return kc, vc


def token_rows(block_table_row, kv_len, block_size):
    """(block, offset) of tokens 0..kv_len-1 of one sequence."""
    row = np.asarray(block_table_row)
    j = np.arange(kv_len)
    return row[j // block_size], j % block_size


def decode(q, key_cache, value_cache, block_table, kv_len, block_size, scale=None):
    """float64 decode; inputs are array-likes convertible to float64."""
    q = np.asarray(q, dtype=np.float64)
    kc = np.asarray(key_cache, dtype=np.float64)
    vc = np.asarray(value_cache, dtype=np.float64)
    bt = np.asarray(block_table)
    lens = np.asarray(kv_len).tolist()
    b_n, hq, d = q.shape
    hkv = kc.shape[1]
    n_rep = hq // hkv
    if scale is None:
        scale = d ** -0.5
    out = np.zeros((b_n, hq, d), dtype=np.float64)
    for b in range(b_n):
        blk, off = token_rows(bt[b], int(lens[b]), block_size)
        for h in range(hq):
            kvh = h // n_rep
            k = kc[blk, kvh, off, :]  # [L, D]
            v = vc[blk, kvh, off, :]
            logits = (k @ q[b, h]) * scale
            m = logits.max()
            p = np.exp(logits - m)
            out[b, h] = (p[:, None] * v).sum(axis=0) / p.sum()
    return out


def prefill(q, key_cache, value_cache, block_tables, seq_indices, cached_len_before, query_len,
            block_size, scale=None):
    """float64 chunked prefill: query token t of sequence i sits at position
    cached_len_before[i] + t and attends key positions 0 .. that position
    (mini_vllm/attention/paged_attention_ref.py:167-244). ``q`` is the
    concatenation [sum(query_len), Hq, D] in sequence order."""
    q = np.asarray(q, dtype=np.float64)
    kc = np.asarray(key_cache, dtype=np.float64)
    vc = np.asarray(value_cache, dtype=np.float64)
    bt = np.asarray(block_tables)
    hq, d = q.shape[1], q.shape[2]
    n_rep = hq // kc.shape[1]
    if scale is None:
        scale = d ** -0.5
    out = np.zeros_like(q)
    off = 0
    for i, s in enumerate(seq_indices):
        c, ql = int(cached_len_before[i]), int(query_len[i])
        blk, pos = token_rows(bt[int(s)], c + ql, block_size)
        for t in range(ql):
            n = c + t + 1  # causal: positions 0 .. c + t
            for h in range(hq):
                k = kc[blk[:n], h // n_rep, pos[:n], :]
                v = vc[blk[:n], h // n_rep, pos[:n], :]
                logits = (k @ q[off + t, h]) * scale
                p = np.exp(logits - logits.max())
                out[off + t, h] = (p[:, None] * v).sum(axis=0) / p.sum()
        off += ql
    return out


def rotary_complex(x, positions, head_dim, theta):
    """RoPE as the complex product of RoFormer: pair (x_i, x_{i+D/2}) is the
    complex number z_i, rotated by angle pos * theta**(-2i/D) (float64
    angles, no tables), i.e. the map the reference's rotate_half form
    (mini_vllm/model/rotary.py:44-82) implements. x: [T, H, D]."""
    x = np.asarray(x, dtype=np.float64)
    half = head_dim // 2
    inv = theta ** (-np.arange(half, dtype=np.float64) * 2.0 / head_dim)
    ang = np.asarray(positions, dtype=np.float64)[:, None] * inv[None, :]  # [T, half]
    rot = np.exp(1j * ang)[:, None, :]                                      # [T, 1, half]
    z = (x[..., :half] + 1j * x[..., half:]) * rot
    return np.concatenate([z.real, z.imag], axis=-1)
