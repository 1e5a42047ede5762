"""Seeded random sweep against the oracle, beyond the hand-picked cases.

Each seed draws a head shape (n_rep 1..16, head_dim 64 / 128), a block
size (1..256), a dtype and a batch of lengths that mixes edge values (1,
one below / at / above a 16-token tile, one block, one block + 1) with
random ones, for
* the decode: the fused layer call (write + decode in one launch) and the
  two separate calls; pools must come out bit-identical to each other and
  the output within the dtype's tolerance of the fp32 oracle, NaN-filled
  free slots included;
* the prefill: random cached prefixes and chunk lengths per sequence.
"""

import random

import pytest
import torch

from benchmarks.paged_decode_workloads import WorkloadSpec, make_case
from gpu_util import DEV, TOL, bits, oracle_step, say, to_device
from mini_vllm.attention.paged_attention_gpu import hip_cache_write, hip_decode_attention
from test_gpu_prefill import _case, _ref, _run

pytestmark = pytest.mark.gpu

SHAPES = [(14, 2, 64), (28, 4, 128), (8, 8, 64), (16, 1, 128), (12, 3, 64), (32, 2, 128),
          (6, 6, 128), (10, 5, 64), (16, 1, 64), (9, 3, 128)]
BLOCKS = [1, 2, 4, 8, 16, 32, 64, 128, 256]
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _decode_spec(seed):
    r = random.Random(1000 + seed)
    hq, hkv, d = r.choice(SHAPES)
    bs = r.choice(BLOCKS)
    dt = r.choice(DTYPES)
    batch = r.randint(1, 24)
    edge = [1, 15, 16, 17, bs, bs + 1]
    lens = [r.choice(edge) if r.random() < 0.4 else r.randint(1, 3000) for _ in range(batch)]
    return WorkloadSpec(f"sweep{seed}", hq, hkv, d, bs, dt, batch, ("fixed", lens))


@pytest.mark.parametrize("seed", range(32))
def test_decode_sweep(seed):
    spec = _decode_spec(seed)
    say("decode sweep", seed, spec.num_q_heads, spec.num_kv_heads, spec.head_dim, spec.block_size,
        spec.dtype, spec.ctx[1])
    case = make_case(spec, seed=seed, nan_fill=True)
    d = to_device(case)
    bs = spec.block_size
    kc1, vc1 = d.key_cache.clone(), d.value_cache.clone()
    hip_cache_write(d.new_key, d.new_value, kc1, vc1, d.slot_mapping, bs)
    out1 = hip_decode_attention(d.query, kc1, vc1, d.block_table, d.kv_len, bs)
    kc2, vc2 = d.key_cache.clone(), d.value_cache.clone()
    out2 = hip_decode_attention(d.query, kc2, vc2, d.block_table, d.kv_len, bs,
                                new_key=d.new_key, new_value=d.new_value, slot_mapping=d.slot_mapping)
    torch.cuda.synchronize()
    for x, y in ((out1, out2), (kc1, kc2), (vc1, vc2)):
        assert torch.equal(bits(x.cpu()), bits(y.cpu()))
    want, _, _ = oracle_step(case)
    out = out2.float().cpu()
    assert not torch.isnan(out).any()
    err = (out - want).abs().max().item()
    assert err <= TOL[spec.dtype], err


def _prefill_args(seed):
    r = random.Random(2000 + seed)
    hq, hkv, d = r.choice(SHAPES)
    bs = r.choice(BLOCKS)
    dt = r.choice(DTYPES)
    n = r.randint(1, 5)
    cached = [r.choice([0, 1, bs, r.randint(0, 700)]) for _ in range(n)]
    qlen = [r.choice([1, 15, 16, 17, r.randint(1, 300)]) for _ in range(n)]
    return hq, hkv, d, bs, dt, cached, qlen


@pytest.mark.parametrize("seed", range(16))
def test_prefill_sweep(seed):
    hq, hkv, d, bs, dt, cached, qlen = _prefill_args(seed)
    say("prefill sweep", seed, hq, hkv, d, bs, dt, cached, qlen)
    c = _case(hq, hkv, d, bs, dt, cached, qlen, seed=seed, fused=seed % 3 == 0)
    out = _run(c)
    assert not torch.isnan(out).any()
    err = (out - _ref(c)).abs().max().item()
    assert err <= TOL[dt], err
