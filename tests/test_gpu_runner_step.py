"""The model runner's mixed step (chunked prefill + decode) through the backend.

QwenModelRunner.execute_model (reference qwen_runner.py:150-197) runs, per
layer, on one step's token rows [prefill tokens | decode tokens]:
  1. q, k = rope(q), rope(k); write_kv_cache(layer, k, v, slot_mapping) over
     ALL rows (prefill and decode slots, input_builder.py:69-96);
  2. prefill_attention(layer, q[:P], k[:P], v[:P], attn_meta, pool);
  3. decode_attention(layer, q[P:], decode_meta, pool) with the metadata
     _build_decode_meta rebases to 0-based decode rows (:213-251);
  4. attn_out[:P], attn_out[P:] = the two results.
Here three layers of one pool run that sequence in four forms:
  * "write": write_kv_cache of all rows (q, k already rotated), as listed;
  * "rope": rope_write_kv_cache (fused RoPE of q and k + the write);
  * "fused": write_kv_cache of the prefill rows, then
    decode_attention_with_write of the decode rows (the decode write inside
    the decode launch);
  * "sublayer": rope_write_kv_cache of the prefill rows, then
    decode_attention_with_rope_write of the decode rows (RoPE, write and
    decode of the decode rows in one launch).
Every layer's attention output is checked against the oracle (the
reference's CPU backend restated: write, then prefill from the pool, then
decode) within the dtype tolerance, and its pool bit for bit. Pool rows no
one may read (free blocks, the slots written this step) hold NaN before the
step. The V rows are a strided column view of one fused QKV buffer, as the
runner's qkv_proj produces. The step also runs captured in a HIP graph and
replays with the step's data copied into its static tensors.
"""

from __future__ import annotations

import math

import pytest
import torch

from gpu_util import DEV, TOL, bits, say
from mini_vllm.attention import AttentionBackend
from mini_vllm.attention import paged_attention_gpu as pg
from mini_vllm.model_runner.base import AttentionGroup, AttentionMetadata, ModelConfig
from oracle import paged_ref, rotary_ref

pytestmark = pytest.mark.gpu

HQ, HKV, D, BS, LAYERS = 14, 2, 64, 16, 3
THETA, MAX_POS = 1000000.0, 4096


NB, MAX_BLOCKS = 9000, 136  # fixed pool and table width: replays keep their shapes


def _layout(seed: int, n_dec: int, pre_cached=(176, 0), pre_q=(83, 50)):
    """A step: two chunked-prefill sequences (by default one with a cached
    prefix and one fresh) and n_dec decode sequences with kv_len_after ~
    U{128..2048}; physical blocks dealt from a random permutation as a block
    manager would, every sequence's blocks its own."""
    g = torch.Generator().manual_seed(seed)
    pre_cached, pre_q = list(pre_cached), list(pre_q)
    dec_kv = torch.randint(128, 2049, (n_dec,), generator=g).tolist()
    need_pre = [math.ceil((c + q) / BS) for c, q in zip(pre_cached, pre_q)]
    need_dec = [math.ceil(k / BS) for k in dec_kv]
    nb = NB
    assert sum(need_pre) + sum(need_dec) <= nb
    perm = torch.randperm(nb, generator=g).tolist()
    max_blocks = MAX_BLOCKS
    assert max(need_pre + need_dec) <= max_blocks
    pos = 0

    def table(needs):
        nonlocal pos
        t = torch.full((len(needs), max_blocks), -1, dtype=torch.int64)
        for i, m in enumerate(needs):
            t[i, :m] = torch.tensor(perm[pos:pos + m])
            pos += m
        return t

    pre_bt, dec_bt = table(need_pre), table(need_dec)
    positions, slots = [], []
    for i, (c, q) in enumerate(zip(pre_cached, pre_q)):
        for p in range(c, c + q):
            positions.append(p)
            slots.append(int(pre_bt[i, p // BS]) * BS + p % BS)
    for i, k in enumerate(dec_kv):
        p = k - 1
        positions.append(p)
        slots.append(int(dec_bt[i, p // BS]) * BS + p % BS)
    return dict(nb=nb, pre_cached=pre_cached, pre_q=pre_q, dec_kv=dec_kv, pre_bt=pre_bt,
                dec_bt=dec_bt, positions=torch.tensor(positions), slots=torch.tensor(slots))


def _layer_data(lay, dtype, seed):
    """Per layer: the pool before the step (real values in the cached
    prefixes, NaN elsewhere) and the step's fused QKV rows (pre-rotation)."""
    g = torch.Generator().manual_seed(seed)
    t = lay["positions"].numel()
    layers = []
    for _ in range(LAYERS):
        kc = torch.full((lay["nb"], HKV, BS, D), float("nan"))
        vc = torch.full((lay["nb"], HKV, BS, D), float("nan"))
        rows = [(lay["pre_bt"][i], c) for i, c in enumerate(lay["pre_cached"])]
        rows += [(lay["dec_bt"][i], k - 1) for i, k in enumerate(lay["dec_kv"])]
        for bt_row, cached in rows:
            for blk in range(math.ceil(cached / BS)):
                n = min(BS, cached - blk * BS)
                b = int(bt_row[blk])
                kc[b, :, :n] = torch.randn(HKV, n, D, generator=g)
                vc[b, :, :n] = torch.randn(HKV, n, D, generator=g)
        qkv = torch.randn(t, (HQ + 2 * HKV) * D, generator=g)
        layers.append(dict(kc=kc.to(dtype), vc=vc.to(dtype), qkv=qkv.to(dtype)))
    return layers


def _split(qkv):
    t = qkv.shape[0]
    q = qkv[:, : HQ * D].view(t, HQ, D)
    k = qkv[:, HQ * D:(HQ + HKV) * D].view(t, HKV, D)
    v = qkv[:, (HQ + HKV) * D:].view(t, HKV, D)  # strided view, as qkv_proj's
    return q, k, v


def _metadata(lay, device):
    """AttentionMetadata as ModelInputBuilder.build makes it (groups with
    global decode seq_indices), and the runner's rebased decode metadata."""
    n_pre, n_dec = len(lay["pre_q"]), len(lay["dec_kv"])
    pre_c = torch.tensor(lay["pre_cached"], dtype=torch.int64, device=device)
    pre_q = torch.tensor(lay["pre_q"], dtype=torch.int64, device=device)
    dec_c = torch.tensor(lay["dec_kv"], dtype=torch.int64, device=device) - 1
    dec_q = torch.ones(n_dec, dtype=torch.int64, device=device)
    p = sum(lay["pre_q"])
    slots = lay["slots"].to(device)
    meta = AttentionMetadata(
        groups=[AttentionGroup(list(range(n_pre)), "prefill_gpu", pre_c, pre_q, pre_c + pre_q),
                AttentionGroup(list(range(n_pre, n_pre + n_dec)), "decode_gpu", dec_c, dec_q,
                               dec_c + dec_q)],
        prefill_slot_mapping=slots[:p], prefill_block_tables=lay["pre_bt"].to(device),
        prefill_positions=lay["positions"][:p].to(device),
        decode_block_tables=lay["dec_bt"].to(device), decode_slot_mapping=slots[p:],
        decode_positions=lay["positions"][p:].to(device), block_size=BS, num_kv_heads=HKV,
        head_dim=D)
    dg = meta.groups[1]
    # the runner's rebased group: the same length tensors, rows 0..B-1
    decode_meta = AttentionMetadata(
        groups=[AttentionGroup(list(range(n_dec)), "decode_gpu", dg.cached_len_before,
                               dg.query_len, dg.kv_len_after)],
        decode_block_tables=meta.decode_block_tables, decode_slot_mapping=meta.decode_slot_mapping,
        decode_positions=meta.decode_positions, block_size=BS, num_kv_heads=HKV, head_dim=D)
    return meta, decode_meta, slots


def _oracle(lay, layers, tables, form):
    """The reference's CPU backend on the same rounded values, per layer:
    (rope,) write of all rows, prefill from the pool, decode."""
    p = sum(lay["pre_q"])
    res = []
    for L in layers:
        kc, vc = L["kc"].float().clone(), L["vc"].float().clone()
        q, k, v = (x.float() for x in _split(L["qkv"]))
        if form in ("rope", "sublayer"):
            dt = L["qkv"].dtype
            # the reference rounds after every op in the model dtype
            tab = rotary_ref.RotaryTables(D, THETA, MAX_POS, dtype=dt)
            q = rotary_ref.rotary(q.to(dt), lay["positions"], tab).float()
            k = rotary_ref.rotary(k.to(dt), lay["positions"], tab).float()
        paged_ref.write_to_paged_cache(k, v, kc, vc, lay["slots"], BS)
        n_pre = len(lay["pre_q"])
        pre = paged_ref.prefill_attention(q[:p], kc, vc, lay["pre_bt"], list(range(n_pre)),
                                          lay["pre_cached"], lay["pre_q"], BS)
        dec = paged_ref.decode_from_tables(q[p:], kc, vc, lay["dec_bt"],
                                           torch.tensor(lay["dec_kv"]), BS)
        res.append((torch.cat([pre, dec]), kc, vc))
    return res


class _Step:
    """One step's device tensors (static, so a graph can keep them) and the
    runner's per-layer calls in one of the three forms."""

    def __init__(self, lay, layers, dtype, form):
        self.form, self.p = form, sum(lay["pre_q"])
        cfg = ModelConfig(num_layers=LAYERS, num_heads=HQ, num_kv_heads=HKV, head_dim=D,
                          dtype=dtype)
        self.be = AttentionBackend.create(cfg, backend="hip")
        self.pool = self.be.allocate_pool(LAYERS, lay["nb"], BS, HKV, D, dtype, DEV)
        self.qkv = [torch.empty_like(L["qkv"], device=DEV) for L in layers]
        self.meta, self.decode_meta, self.slots = _metadata(lay, DEV)
        self.positions = lay["positions"].to(DEV)
        self.rope = rotary_ref.RotaryTables(D, THETA, MAX_POS, dtype=dtype)
        self.rope.cos, self.rope.sin = self.rope.cos.to(DEV), self.rope.sin.to(DEV)

    def load(self, layers, lay=None):
        for i, L in enumerate(layers):
            self.pool.key_caches[i].copy_(L["kc"])
            self.pool.value_caches[i].copy_(L["vc"])
            self.qkv[i].copy_(L["qkv"])
        if lay is not None:  # a new step's metadata, into the same tensors
            meta, _, slots = _metadata(lay, "cpu")
            for dst, src in zip(self.meta.groups, meta.groups):
                dst.cached_len_before.copy_(src.cached_len_before)
                dst.query_len.copy_(src.query_len)
                dst.kv_len_after.copy_(src.kv_len_after)
            for name in ("prefill_block_tables", "decode_block_tables", "prefill_positions",
                         "decode_positions"):
                getattr(self.meta, name).copy_(getattr(meta, name))
            self.slots.copy_(slots)
            self.positions.copy_(lay["positions"])

    def run(self):
        p, be, pool = self.p, self.be, self.pool
        outs = []
        for layer in range(LAYERS):
            q, k, v = _split(self.qkv[layer])
            if self.form == "sublayer":
                q_pre, k_pre = be.rope_write_kv_cache(
                    layer, q[:p], k[:p], v[:p], self.positions[:p], self.rope, self.slots[:p],
                    return_key=True)
                attn_out = torch.zeros_like(q)
                attn_out[:p] = be.prefill_attention(layer, q_pre, k_pre, v[:p], self.meta, pool)
                attn_out[p:] = be.decode_attention_with_rope_write(
                    layer, q[p:], k[p:], v[p:], self.positions[p:], self.rope, self.slots[p:],
                    self.decode_meta, pool)
                outs.append(attn_out)
                continue
            if self.form == "rope":
                q, k = be.rope_write_kv_cache(layer, q, k, v, self.positions, self.rope,
                                              self.slots, return_key=True)
            elif self.form == "write":
                be.write_kv_cache(layer, k, v, self.slots)
            else:  # "fused": the prefill rows here, the decode rows inside the decode
                be.write_kv_cache(layer, k[:p], v[:p], self.slots[:p])
            attn_out = torch.zeros_like(q)
            attn_out[:p] = be.prefill_attention(layer, q[:p], k[:p], v[:p], self.meta, pool)
            if self.form == "fused":
                attn_out[p:] = be.decode_attention_with_write(
                    layer, q[p:], k[p:], v[p:], self.slots[p:], self.decode_meta, pool)
            else:
                attn_out[p:] = be.decode_attention(layer, q[p:], self.decode_meta, pool)
            outs.append(attn_out)
        return outs

    def check(self, outs, ref, tol, tag):
        for layer, (out, (o_ref, kc_ref, vc_ref)) in enumerate(zip(outs, ref)):
            err = (out.float().cpu() - o_ref).abs().max().item()
            assert err <= tol, (tag, layer, err)
            assert torch.equal(bits(self.pool.key_caches[layer].cpu().float()), bits(kc_ref)), (tag, layer)
            assert torch.equal(bits(self.pool.value_caches[layer].cpu().float()), bits(vc_ref)), (tag, layer)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("form", ["write", "rope", "fused", "sublayer"])
def test_mixed_step_eager(dtype, form):
    say("runner mixed step eager", form, dtype)
    lay = _layout(7, 64)
    layers = _layer_data(lay, dtype, 8)
    ref = _oracle(lay, layers, None, form)
    st = _Step(lay, layers, dtype, form)
    st.load(layers)
    outs = st.run()
    torch.cuda.synchronize()
    st.check(outs, ref, TOL[dtype], f"eager {form}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("form", ["write", "rope", "fused", "sublayer"])
def test_mixed_step_captured(dtype, form):
    """The whole 3-layer mixed step captured in one HIP graph (prefill
    planned on the device, decode plan of fixed size, checks deferred), then
    replayed with the captured step's data and with another step's (new
    decode lengths, slots and tables, new prefill prefixes, the same row
    counts), each replay checked against the oracle; a replay whose prefill
    table cannot cover its prefix is reported by check_deferred()."""
    say("runner mixed step captured", form, dtype)
    lay_a = _layout(7, 64)
    lay_b = _layout(9, 64, pre_cached=(40, 300))
    layers_a, layers_b = _layer_data(lay_a, dtype, 8), _layer_data(lay_b, dtype, 10)
    st = _Step(lay_a, layers_a, dtype, form)
    st.load(layers_a)
    pg.clear_deferred()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # eager warm-up: library, workspace, split
        st.run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = st.run()
    gid = pg.last_capture_id()
    for tag, lay, layers in (("A", lay_a, layers_a), ("B", lay_b, layers_b),
                             ("A again", lay_a, layers_a)):
        say("runner mixed step captured: replay", tag)
        st.load(layers, lay)
        graph.replay()
        torch.cuda.synchronize()
        pg.check_deferred(gid)
        st.check(outs, _oracle(lay, layers, None, form), TOL[dtype], f"captured {form} {tag}")
    say("runner mixed step captured: replay with a short prefill table row")
    st.load(layers_b, lay_b)
    st.meta.prefill_block_tables[1, 0] = -1  # sequence 1's prefix needs it
    graph.replay()
    torch.cuda.synchronize()
    with pytest.raises(IndexError, match="insufficient"):
        pg.check_deferred(gid)
    del graph
    pg.clear_deferred()
