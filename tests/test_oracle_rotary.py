"""Pins the rotary-embedding oracle (oracle/rotary_ref.py), CPU only.

* Against HuggingFace's Qwen2RotaryEmbedding + apply_rotary_pos_emb (the
  check of the reference's own tests/test_rotary.py:test_rope_vs_hf), with
  the same theta / table length, at fp32.
* Against an independent float64 complex-rotation brute force
  (oracle/brute.py:rotary_complex), which uses angles instead of tables.
* Properties the maths fixes: position 0 is the identity; pair norms are
  preserved; q.k after rotation depends only on the position difference.
* bf16: the oracle's output is the per-op rounding of the exact rotation
  (within two bf16 rounding steps of the float64 value).
"""

import numpy as np
import pytest
import torch

from oracle import brute
from oracle.rotary_ref import RotaryTables, rotary


def _x(t, h, d, seed=0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(t, h, d, generator=g).to(dtype)


def test_matches_hf_qwen2_rotary():
    tr = pytest.importorskip("transformers")
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RotaryEmbedding, apply_rotary_pos_emb

    d, theta, max_seq = 64, 10000.0, 128
    cfg = tr.Qwen2Config(hidden_size=512, num_attention_heads=8, num_key_value_heads=2,
                         head_dim=d, rope_theta=theta, max_position_embeddings=max_seq)
    hf = Qwen2RotaryEmbedding(cfg)
    tables = RotaryTables(d, theta, max_seq, torch.float32)
    x = _x(5, 8, d)
    pos = torch.tensor([0, 5, 10, 15, 127])
    ours = rotary(x, pos, tables)
    xb = x.permute(1, 0, 2).unsqueeze(0)  # [1, H, T, D]
    cos, sin = hf(xb, pos.unsqueeze(0))
    ref, _ = apply_rotary_pos_emb(xb, xb, cos, sin)
    ref = ref.squeeze(0).permute(1, 0, 2)
    assert (ours - ref).abs().max().item() < 1e-5


@pytest.mark.parametrize("d,theta", [(64, 1000000.0), (128, 10000.0)])
def test_matches_complex_rotation_fp64(d, theta):
    tables = RotaryTables(d, theta, 4096, torch.float32)
    x = _x(40, 3, d, seed=1)
    pos = torch.randint(0, 4096, (40,), generator=torch.Generator().manual_seed(2))
    ours = rotary(x, pos, tables).double().numpy()
    ref = brute.rotary_complex(x.numpy(), pos.numpy(), d, theta)
    # fp32 angles t * inv_freq at t < 4096 are off by < 4096 * 2**-24 rad
    assert np.abs(ours - ref).max() < 2e-3 * np.abs(x.numpy()).max()


def test_position_zero_is_identity():
    tables = RotaryTables(64, 10000.0, 16, torch.float32)
    x = _x(3, 4, 64)
    assert torch.equal(rotary(x, torch.zeros(3, dtype=torch.long), tables), x)


def test_pair_norms_preserved():
    d = 128
    tables = RotaryTables(d, 1000000.0, 2048, torch.float32)
    x = _x(16, 2, d, seed=3)
    y = rotary(x, torch.arange(0, 2048, 128), tables)
    h = d // 2
    nx = x[..., :h] ** 2 + x[..., h:] ** 2
    ny = y[..., :h] ** 2 + y[..., h:] ** 2
    assert torch.allclose(nx, ny, rtol=1e-5, atol=1e-5)


def test_dot_product_depends_on_position_difference():
    d = 64
    tables = RotaryTables(d, 10000.0, 512, torch.float32)
    q, k = _x(1, 1, d, seed=4), _x(1, 1, d, seed=5)
    def dot(m, n):
        return (rotary(q, torch.tensor([m]), tables) * rotary(k, torch.tensor([n]), tables)).sum().item()
    base = dot(7, 3)
    for shift in (1, 50, 300):
        assert abs(dot(7 + shift, 3 + shift) - base) < 1e-4


def test_bf16_is_rounded_rotation():
    d = 64
    t16 = RotaryTables(d, 1000000.0, 1024, torch.bfloat16)
    x = _x(32, 2, d, seed=6, dtype=torch.bfloat16)
    pos = torch.randint(0, 1024, (32,), generator=torch.Generator().manual_seed(7))
    ours = rotary(x, pos, t16).double()
    # exact rotation with the bf16 tables' values
    c = t16.cos[pos].double().unsqueeze(1)
    s = t16.sin[pos].double().unsqueeze(1)
    xd = x.double()
    h = d // 2
    ref = torch.cat([xd[..., :h] * c[..., :h] - xd[..., h:] * s[..., :h],
                     xd[..., h:] * c[..., h:] + xd[..., :h] * s[..., h:]], dim=-1)
    # two products and a sum, each rounded to bf16 (relative 2**-8 each)
    bound = 3 * 2.0 ** -8 * (xd.abs().amax(-1, keepdim=True)) * 2
    assert ((ours - ref).abs() <= bound).all()
