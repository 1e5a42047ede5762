"""Paged prefill attention (mv_paged_prefill) against the oracle.

The oracle restates the reference GPU backend's prefill
(oracle/paged_ref.py:prefill_attention_chunk_args): prefix from the pool,
chunk K/V from the arguments, offset causal mask, in fp32 on the same
(rounded) inputs. Pool rows the kernel must not read (free blocks and the
chunk's own slots) hold NaN, so a stray read fails the comparison.
"""

import pytest
import torch

from gpu_util import DEV, TOL, say
from mini_vllm.attention import AttentionBackend, _hip
from mini_vllm.attention import paged_attention_gpu as pag
from mini_vllm.attention.paged_attention_gpu import hip_prefill_attention
from mini_vllm.model_runner.base import AttentionGroup, AttentionMetadata, ModelConfig
from oracle import paged_ref

pytestmark = pytest.mark.gpu


def _case(hq, hkv, d, bs, dtype, cached, qlen, seed=0, fused=False, extra_blocks=16):
    g = torch.Generator().manual_seed(seed)
    n = len(cached)
    need = [-(-c // bs) for c in cached]
    nb = sum(need) + extra_blocks
    width = max(need + [1]) + 2
    perm = torch.randperm(nb, generator=g)
    bt = torch.full((n + 1, width), -1, dtype=torch.int64)  # row 0 unused: rows are seq_indices
    pos = 0
    for i, m in enumerate(need):
        bt[i + 1, :m] = perm[pos:pos + m]
        pos += m
    kc = torch.full((nb, hkv, bs, d), float("nan"))
    vc = torch.full((nb, hkv, bs, d), float("nan"))
    for i, c in enumerate(cached):  # real values only in the prefix slots
        for p in range(c):
            b = int(bt[i + 1, p // bs])
            kc[b, :, p % bs] = torch.randn(hkv, d, generator=g)
            vc[b, :, p % bs] = torch.randn(hkv, d, generator=g)
    t = sum(qlen)
    if fused:
        qkv = torch.randn(t, (hq + 2 * hkv) * d, generator=g)
        q = qkv[:, : hq * d].reshape(t, hq, d)
        k = qkv[:, hq * d:(hq + hkv) * d].reshape(t, hkv, d)
        v = qkv[:, (hq + hkv) * d:].reshape(t, hkv, d)
    else:
        q = torch.randn(t, hq, d, generator=g)
        k = torch.randn(t, hkv, d, generator=g)
        v = torch.randn(t, hkv, d, generator=g)
    r = lambda x: x.to(dtype).float()  # noqa: E731  values the kernel sees
    return dict(q=r(q), k=r(k), v=r(v), kc=r(kc), vc=r(vc), bt=bt, rows=list(range(1, n + 1)),
                cached=cached, qlen=qlen, bs=bs, dtype=dtype, fused=fused, hq=hq, hkv=hkv, d=d)


def _run(c):
    dt = c["dtype"]
    if c["fused"]:
        t = c["q"].shape[0]
        qkv = torch.cat([c["q"].reshape(t, -1), c["k"].reshape(t, -1), c["v"].reshape(t, -1)], 1)
        qkv = qkv.to(dt).to(DEV)
        hq, hkv, d = c["hq"], c["hkv"], c["d"]
        q = qkv[:, : hq * d].view(t, hq, d)
        k = qkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
        v = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
    else:
        q, k, v = (c[n].to(dt).to(DEV) for n in ("q", "k", "v"))
    out = hip_prefill_attention(q, k, v, c["kc"].to(dt).to(DEV), c["vc"].to(dt).to(DEV),
                                c["bt"].to(DEV), c["rows"], c["cached"], c["qlen"], c["bs"])
    torch.cuda.synchronize()
    return out.float().cpu()


def _ref(c):
    return paged_ref.prefill_attention_chunk_args(c["q"], c["k"], c["v"], c["kc"], c["vc"], c["bt"],
                                                  c["rows"], c["cached"], c["qlen"], c["bs"])


CACHED = [0, 100, 5, 300, 2047, 64]
QLEN = [37, 64, 1, 129, 3, 200]

SHAPES = [  # (hq, hkv, d, bs, dtype)
    (14, 2, 64, 16, torch.bfloat16),
    (14, 2, 64, 16, torch.float32),
    (28, 4, 128, 16, torch.bfloat16),
    (8, 8, 64, 32, torch.float16),     # n_rep 1
    (16, 1, 128, 16, torch.bfloat16),  # n_rep 16
    (16, 1, 64, 64, torch.bfloat16),   # n_rep 16, block 64
    (10, 2, 64, 16, torch.bfloat16),   # n_rep 5: 6 tokens per row wave, 2 padding rows
    (12, 2, 64, 16, torch.float16),    # n_rep 6: 5 tokens per row wave (20 per work group)
    (8, 2, 128, 16, torch.float16),    # head_dim 128 in fp16
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}-{s[1]}-{s[2]}-bs{s[3]}-{s[4]}")
def test_prefill_matches_oracle(shape):
    hq, hkv, d, bs, dt = shape
    say("prefill", shape)
    c = _case(hq, hkv, d, bs, dt, CACHED, QLEN, seed=1)
    out = _run(c)
    ref = _ref(c)
    assert not torch.isnan(out).any()
    err = (out - ref).abs().max().item()
    assert err <= TOL[dt], err


def test_bench_step_shape():
    """The bench's own prefill step: 4 sequences x (1536 cached + 512 chunk)
    at the Qwen2-0.5B shape in bf16 (256 whole work groups, every stage of
    the lazy softmax reference), in a fused QKV buffer as the runner has it."""
    say("prefill: bench step 4 x (1536 + 512)")
    c = _case(14, 2, 64, 16, torch.bfloat16, [1536] * 4, [512] * 4, seed=9, fused=True)
    out = _run(c)
    assert not torch.isnan(out).any()
    err = (out - _ref(c)).abs().max().item()
    assert err <= TOL[torch.bfloat16], err


def test_fused_qkv_views():
    say("prefill fused qkv")
    c = _case(14, 2, 64, 16, torch.bfloat16, [40, 0, 333], [77, 16, 50], seed=2, fused=True)
    err = (_run(c) - _ref(c)).abs().max().item()
    assert err <= TOL[torch.bfloat16], err


def test_prefix_spanning_two_id_windows():
    """block_size 1: a 3000-token prefix needs 3000 block ids, two windows of 2048."""
    say("prefill two windows")
    c = _case(14, 2, 64, 1, torch.bfloat16, [3000, 10], [40, 20], seed=3, extra_blocks=64)
    err = (_run(c) - _ref(c)).abs().max().item()
    assert err <= TOL[torch.bfloat16], err


def test_more_than_16_query_heads_per_kv_head_is_unsupported():
    """As the decode path (and the backend's constructor): at most 16 query
    heads per kv head -- one MFMA row tile per wave."""
    c = _case(32, 1, 64, 16, torch.bfloat16, [10], [4], seed=6)
    with pytest.raises(RuntimeError, match="not supported"):
        _run(c)


def test_insufficient_table_raises():
    say("prefill insufficient table")
    c = _case(14, 2, 64, 16, torch.bfloat16, [50], [8], seed=4)
    c["bt"][1, 2] = 10_000  # not a pool block
    with pytest.raises(IndexError, match="insufficient"):
        _run(c)
    c["bt"] = c["bt"][:, :2]  # too short for 50 tokens
    with pytest.raises(IndexError, match="insufficient"):
        _run(c)


def test_backend_prefill_groups():
    """AttentionBackendGPU.prefill_attention over two prefill groups."""
    say("backend prefill")
    c = _case(14, 2, 64, 16, torch.bfloat16, [0, 90, 17], [33, 21, 8], seed=5)
    cfg = ModelConfig(num_layers=1, hidden_size=896, num_heads=14, num_kv_heads=2, head_dim=64,
                      dtype=torch.bfloat16)
    be = AttentionBackend.create(cfg, backend="hip")
    nb = c["kc"].shape[0]
    pool = be.allocate_pool(1, nb, 16, 2, 64, torch.bfloat16, DEV)
    pool.key_caches[0].copy_(c["kc"].to(torch.bfloat16))
    pool.value_caches[0].copy_(c["vc"].to(torch.bfloat16))
    lt = lambda x: torch.tensor(x, dtype=torch.long)  # noqa: E731
    groups = [
        AttentionGroup([1, 2], "prefill_gpu", lt(c["cached"][:2]), lt(c["qlen"][:2]),
                       lt([a + b for a, b in zip(c["cached"][:2], c["qlen"][:2])])),
        AttentionGroup([3], "prefill_gpu", lt(c["cached"][2:]), lt(c["qlen"][2:]),
                       lt([c["cached"][2] + c["qlen"][2]])),
    ]
    meta = AttentionMetadata(groups=groups, prefill_block_tables=c["bt"].to(DEV), block_size=16,
                             num_kv_heads=2, head_dim=64)
    out = be.prefill_attention(0, c["q"].to(torch.bfloat16).to(DEV), c["k"].to(torch.bfloat16).to(DEV),
                               c["v"].to(torch.bfloat16).to(DEV), meta, pool)
    torch.cuda.synchronize()
    err = (out.float().cpu() - _ref(c)).abs().max().item()
    assert err <= TOL[torch.bfloat16], err


# ---- key split (mv_paged_prefill_parts): launches with fewer units than CUs

def _max_parts(c):
    """The most parts the plan cuts a unit of this case into."""
    lib = _hip.load()
    tpg = lib.mv_prefill_tokens_per_group(c["hq"], c["hkv"], c["d"], _hip.MV_DTYPE[c["dtype"]])
    keys = [cc + t0 + min(tpg, q - t0) for cc, q in zip(c["cached"], c["qlen"])
            for t0 in range(0, q, tpg) for _ in range(c["hkv"])]
    cus = torch.cuda.get_device_properties(DEV).multi_processor_count
    return max(len(p) for p in pag.prefill_key_parts(keys, cus))


SPLIT_SHAPES = [  # (hq, hkv, d, bs, dtype): units of one 512-token chunk, parts
    (14, 2, 64, 16, torch.bfloat16),   # 64 units, 4 parts
    (14, 2, 64, 16, torch.float32),    # 64 units, 4 parts
    (28, 4, 128, 16, torch.bfloat16),  # 128 units, 2 parts
    (8, 8, 64, 32, torch.float16),     # n_rep 1: 32 units, 8 parts
    (16, 1, 128, 16, torch.bfloat16),  # n_rep 16: 64 units, 4 parts
]


@pytest.mark.parametrize("shape", SPLIT_SHAPES, ids=lambda s: f"{s[0]}-{s[1]}-{s[2]}-bs{s[3]}-{s[4]}")
def test_key_split_long_prefix(shape):
    """One sequence's 512-token chunk over a 3584-token prefix: too few
    units for the CUs, so each unit's keys are cut into parts and merged by
    the last part to finish."""
    hq, hkv, d, bs, dt = shape
    say("prefill key split", shape)
    c = _case(hq, hkv, d, bs, dt, [3584], [512], seed=7)
    assert _max_parts(c) > 1
    out = _run(c)
    assert not torch.isnan(out).any()
    err = (out - _ref(c)).abs().max().item()
    assert err <= TOL[dt], err


def test_key_split_mixed_units():
    """Cut and whole units in one launch: a long prefix, and a chunk-only
    sequence whose parts read their keys from the key / value rows."""
    say("prefill key split, mixed")
    # n_rep 1: 128 tokens per work group, 8 kv heads: 112 units, 2 parts at most
    c = _case(8, 8, 64, 32, torch.float16, [2000, 0, 7], [100, 1500, 30], seed=8)
    assert _max_parts(c) == 2
    err = (_run(c) - _ref(c)).abs().max().item()
    assert err <= TOL[torch.float16], err


def test_key_split_is_deterministic_and_matches_whole_units(monkeypatch):
    """The parts are folded in part order: repeated calls give the same
    bits; and the result is that of the uncut launch within fp32 rounding."""
    say("prefill key split, repeats")
    c = _case(14, 2, 64, 16, torch.float32, [3000], [256], seed=9)
    assert _max_parts(c) > 1
    first = _run(c)
    for _ in range(3):
        assert torch.equal(_run(c), first)
    monkeypatch.setenv("MVATTN_PREFILL_PARTS", "1")
    whole = _run(c)  # a new table tensor: a new plan, uncut
    assert (first - whole).abs().max().item() <= 1e-5
    assert (whole - _ref(c)).abs().max().item() <= TOL[torch.float32]


# ---- the softmax reference: stages kept as computed, or redone exactly

def _scaled(c, q_mul=1.0, k_mul=1.0, k_keys=None):
    """The case with Q (and K: all keys, or prefix positions k_keys of every
    sequence) multiplied, rounded again to the case's type."""
    dt = c["dtype"]
    out = dict(c)
    out["q"] = (c["q"] * q_mul).to(dt).float()
    k, kc = c["k"], c["kc"].clone()
    if k_keys is None:
        k = (k * k_mul).to(dt).float()
        kc = (kc * k_mul).to(dt).float()
    else:
        bs = c["bs"]
        for row, cached in zip(c["rows"], c["cached"]):
            for p in k_keys:
                if p < cached:
                    b = int(c["bt"][row, p // bs])
                    kc[b, :, p % bs] = (kc[b, :, p % bs] * k_mul).to(dt).float()
    out["k"], out["kc"] = k, kc
    return out


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("d", [64, 128])
def test_sharp_scores(dt, d):
    """Q x 4: scores of a few tens in the exponent's units, so stage sums
    leave [2^-12, 2^12] and those stages are computed exactly (reference
    moved, O rescaled); head_dim 64 (two wave sets) and 128 (one)."""
    say("prefill sharp scores", dt, d)
    c = _scaled(_case(14, 2, d, 16, dt, [1536, 300, 0], [512, 40, 100], seed=11), q_mul=4.0)
    out = _run(c)
    assert not torch.isnan(out).any()
    err = (out - _ref(c)).abs().max().item()
    say("max abs err", err)
    assert err <= TOL[dt], err


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=str)
def test_late_key_with_a_far_higher_score(dt):
    """16 prefix keys (positions 1200-1215) with K x 12: their stage's sums
    overflow the range, the reference moves up by tens of units, and the
    stages after it are kept as computed again (sums far below 1, l above)."""
    say("prefill late high key", dt)
    c = _scaled(_case(14, 2, 64, 16, dt, [1536, 1300], [512, 64], seed=12), k_mul=12.0,
                k_keys=range(1200, 1216))
    out = _run(c)
    assert not torch.isnan(out).any()
    err = (out - _ref(c)).abs().max().item()
    say("max abs err", err)
    assert err <= TOL[dt], err


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=str)
def test_scores_far_below_zero(dt):
    """Every score near -60 in the exponent's units: the first stage's sums
    fall below 2^-12 and are computed exactly, which moves the reference
    down to the row maximum."""
    say("prefill negative scores", dt)
    c = _case(14, 2, 64, 16, dt, [700, 0], [300, 33], seed=13)
    c["q"] = (c["q"].abs() * 2 + 1).to(dt).float()
    c["k"] = (-(c["k"].abs() * 2 + 1)).to(dt).float()
    kc = c["kc"]
    c["kc"] = torch.where(torch.isnan(kc), kc, -(kc.abs() * 2 + 1)).to(dt).float()
    out = _run(c)
    assert not torch.isnan(out).any()
    err = (out - _ref(c)).abs().max().item()
    say("max abs err", err)
    assert err <= TOL[dt], err
