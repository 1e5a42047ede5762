"""A decode step captured into a HIP graph and replayed with new metadata.

The step is three layers of (KV write, paged decode) on static tensors. The
capture runs the plan without reading it back (a launch of fixed size,
unused slots marked); each replay plans again from whatever the static
block table / kv_len / slot tensors hold. Every replay is checked against
the oracle, with eager work (the metadata copies) between replays, and the
checks captured with the step report bad metadata through check_deferred().
"""

import pytest
import torch

from benchmarks.paged_decode_workloads import WorkloadSpec, make_case
from gpu_util import DEV, TOL, bits, say
from mini_vllm.attention import paged_attention_gpu as pg
from oracle import paged_ref

pytestmark = pytest.mark.gpu

NB, BS, MB, B, HQ, HKV, D, LAYERS = 2048, 16, 64, 24, 14, 2, 64, 3
DT = torch.bfloat16


def _case(seed, lo, hi):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (B,), generator=g)
    need = [(int(n) + BS - 1) // BS for n in lens]
    perm = torch.randperm(NB, generator=g)
    bt = torch.full((B, MB), -1, dtype=torch.int64)
    pos = 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[pos:pos + n]
        pos += n
    last = lens - 1
    slots = bt[torch.arange(B), last // BS] * BS + last % BS
    layers = []
    for _ in range(LAYERS):
        layers.append(dict(
            q=torch.randn(B, HQ, D, generator=g).to(DT),
            nk=torch.randn(B, HKV, D, generator=g).to(DT),
            nv=torch.randn(B, HKV, D, generator=g).to(DT),
            kc=torch.randn(NB, HKV, BS, D, generator=g).to(DT),
            vc=torch.randn(NB, HKV, BS, D, generator=g).to(DT),
        ))
    return dict(bt=bt, kv=lens.to(torch.int64), slots=slots, layers=layers)


def _oracle(case):
    res = []
    for L in case["layers"]:
        kc, vc = L["kc"].clone(), L["vc"].clone()
        paged_ref.write_to_paged_cache(L["nk"], L["nv"], kc, vc, case["slots"], BS)
        out = paged_ref.decode_from_tables(L["q"].float(), kc.float(), vc.float(), case["bt"],
                                           case["kv"], BS)
        res.append((out, kc, vc))
    return res


class _Static:
    """Device tensors whose addresses the graph keeps; cases are copied in."""

    def __init__(self):
        self.bt = torch.empty(B, MB, dtype=torch.int64, device=DEV)
        self.kv = torch.empty(B, dtype=torch.int64, device=DEV)
        self.slots = torch.empty(B, dtype=torch.int64, device=DEV)
        self.layers = [dict(q=torch.empty(B, HQ, D, dtype=DT, device=DEV),
                            nk=torch.empty(B, HKV, D, dtype=DT, device=DEV),
                            nv=torch.empty(B, HKV, D, dtype=DT, device=DEV),
                            kc=torch.empty(NB, HKV, BS, D, dtype=DT, device=DEV),
                            vc=torch.empty(NB, HKV, BS, D, dtype=DT, device=DEV))
                       for _ in range(LAYERS)]

    def load(self, case):
        self.bt.copy_(case["bt"])
        self.kv.copy_(case["kv"])
        self.slots.copy_(case["slots"])
        for dst, src in zip(self.layers, case["layers"]):
            for k in dst:
                dst[k].copy_(src[k])

    def step(self):
        outs = []
        for L in self.layers:
            pg.hip_cache_write(L["nk"], L["nv"], L["kc"], L["vc"], self.slots, BS)
            outs.append(pg.hip_decode_attention(L["q"], L["kc"], L["vc"], self.bt, self.kv, BS))
        return outs


def _check(st, outs, ref, tag):
    for layer, (L, out, (o_ref, kc_ref, vc_ref)) in enumerate(zip(st.layers, outs, ref)):
        err = (out.float().cpu() - o_ref).abs().max().item()
        assert err <= TOL[DT], (tag, layer, err)
        assert torch.equal(bits(L["kc"].cpu()), bits(kc_ref)), (tag, layer)
        assert torch.equal(bits(L["vc"].cpu()), bits(vc_ref)), (tag, layer)


def test_captured_step_replays_new_metadata():
    say("graph: capture")
    pg.clear_deferred()
    case_a, case_b = _case(1, 1, MB * BS), _case(2, 300, 700)
    ref_a, ref_b = _oracle(case_a), _oracle(case_b)
    st = _Static()
    st.load(case_a)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # eager warm-up: library, workspace, split
        st.step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = st.step()
    for tag, case, ref in (("A", case_a, ref_a), ("B", case_b, ref_b), ("A again", case_a, ref_a)):
        say("graph: replay", tag)
        st.load(case)
        graph.replay()
        torch.cuda.synchronize()
        pg.check_deferred()
        _check(st, outs, ref, tag)

    say("graph: replay with a zero kv_len")
    bad = dict(case_b)
    bad["kv"] = case_b["kv"].clone()
    bad["kv"][3] = 0
    st.load(bad)
    graph.replay()
    torch.cuda.synchronize()
    with pytest.raises(ValueError, match="kv_len"):
        pg.check_deferred()

    say("graph: replay with a table entry outside the pool")
    bad = dict(case_b)
    bad["bt"] = case_b["bt"].clone()
    bad["bt"][5, 0] = NB + 7
    st.load(bad)
    graph.replay()
    torch.cuda.synchronize()
    with pytest.raises(IndexError, match="not pool blocks"):
        pg.check_deferred()

    say("graph: replay B after the bad ones")
    st.load(case_b)
    graph.replay()
    torch.cuda.synchronize()
    pg.check_deferred()
    _check(st, outs, ref_b, "B last")
    del graph
    pg.clear_deferred()


def test_eager_calls_after_capture_still_validate():
    say("graph: eager after capture")
    case = _case(3, 50, 400)
    st = _Static()
    st.load(case)
    ref = _oracle(case)
    outs = st.step()
    torch.cuda.synchronize()
    _check(st, outs, ref, "eager")
    st.kv[0] = 0  # in-place edit: the next call plans (and checks) again
    with pytest.raises(ValueError, match="kv_len"):
        st.step()


def test_captured_long_pieces_fetch_the_rest_of_their_ids():
    """A launch of fixed size stores each work group's block ids at the
    widest piece's stride, and the kernel copies only the first 64 before
    it knows its piece. Here 520 (sequence, kv head) units of 1100-1300
    tokens make pieces of about 80 table entries: every work group fetches
    the rest of its list once its work item is known. Replayed twice, the
    second time with shorter kv_len in place."""
    lens = [1100 + (37 * i) % 200 for i in range(260)]
    spec = WorkloadSpec("long-pieces", 14, 2, 64, 16, DT, len(lens), ("fixed", lens))
    case = make_case(spec, seed=5, nan_fill=True)
    q, kc, vc = case.query.to(DEV), case.key_cache.to(DEV), case.value_cache.to(DEV)
    bt, kv = case.block_table.to(DEV), case.kv_len.to(DEV)
    # the step's new tokens (their slots are NaN until written)
    pg.hip_cache_write(case.new_key.to(DEV), case.new_value.to(DEV), kc, vc,
                       case.slot_mapping.to(DEV), 16)
    kc_ref, vc_ref = case.key_cache.float(), case.value_cache.float()
    paged_ref.write_to_paged_cache(case.new_key.float(), case.new_value.float(), kc_ref, vc_ref,
                                   case.slot_mapping, 16)
    pg.clear_deferred()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # eager warm-up
        pg.hip_decode_attention(q, kc, vc, bt, kv, 16)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = pg.hip_decode_attention(q, kc, vc, bt, kv, 16)
    shorter = case.kv_len - torch.arange(len(lens)) % 300
    for tag, lengths in (("full", case.kv_len), ("shorter", shorter)):
        say("graph: long pieces", tag)
        kv.copy_(lengths)
        graph.replay()
        torch.cuda.synchronize()
        pg.check_deferred()
        ref = paged_ref.decode_from_tables(case.query.float(), kc_ref, vc_ref, case.block_table,
                                           lengths, 16)
        err = (out.float().cpu() - ref).abs().max().item()
        assert err <= TOL[DT], (tag, err)
    del graph
    pg.clear_deferred()


def _current_workspace():
    return next(iter(pg._WORKSPACES.values()), None)


def test_workspace_growth_after_capture_keeps_the_graphs_buffer():
    """A graph captured with a small merge workspace, then an eager decode
    big enough to need a larger one: the library keeps the buffer the graph
    was captured with (the merge keeps state in it between calls), so
    tensors allocated afterwards cannot land in it. Replays stay exact and
    the new tensors keep their contents."""
    say("graph: workspace growth after capture")
    pg.clear_deferred()
    for dev in list(pg._WORKSPACES):  # start from a small workspace, as a fresh process
        pg._RETIRED_WORKSPACES.append(pg._WORKSPACES.pop(dev))
    case = _case(11, 300, MB * BS)
    ref = _oracle(case)
    st = _Static()
    st.load(case)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        st.step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = st.step()
    small = _current_workspace()
    assert small is not None
    # an eager decode whose partials need more workspace (32 query heads of
    # head_dim 128, 16 sequences of 2048 tokens cut into ~8 pieces each)
    spec = WorkloadSpec("ws-grow", 32, 2, 128, 16, DT, 16, ("fixed", [2048] * 16))
    big = make_case(spec, seed=0, nan_fill=False)
    q, kc, vc = big.query.to(DEV), big.key_cache.to(DEV), big.value_cache.to(DEV)
    pg.hip_decode_attention(q, kc, vc, big.block_table.to(DEV), big.kv_len.to(DEV), 16)
    torch.cuda.synchronize()
    assert _current_workspace().numel() > small.numel(), "the eager call did not grow the workspace"
    fillers = [torch.full((1 << 20,), 7, dtype=torch.int32, device=DEV) for _ in range(32)]
    for rep in range(3):
        st.load(case)
        graph.replay()
        torch.cuda.synchronize()
        pg.check_deferred()
        _check(st, outs, ref, f"replay {rep}")
    for f in fillers:
        assert int((f != 7).sum()) == 0
    del graph
    pg.clear_deferred()


def test_second_capture_over_the_same_metadata_plans_on_its_own():
    """Two graphs captured over the same static (unmodified) metadata
    tensors: the second records its own plan and check kernels (caches are
    keyed by capture id), so replaying only the second one with new lengths
    is exact; each graph's deferred checks are read by its id only."""
    say("graph: second capture over the same metadata")
    pg.clear_deferred()
    case_a, case_b = _case(21, 1, MB * BS), _case(22, 200, 900)
    st = _Static()
    st.load(case_a)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        st.step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g1 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g1):
        outs1 = st.step()
    id1 = pg.last_capture_id()
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2):
        outs2 = st.step()
    id2 = pg.last_capture_id()
    assert id1 and id2 and id1 != id2
    st.load(case_b)
    g2.replay()
    torch.cuda.synchronize()
    pg.check_deferred(id2)
    _check(st, outs2, _oracle(case_b), "second graph, new lengths")
    # a bad replay of the first graph is reported for it, not for the second
    bad = dict(case_b)
    bad["kv"] = case_b["kv"].clone()
    bad["kv"][0] = 0
    st.load(bad)
    g1.replay()
    torch.cuda.synchronize()
    with pytest.raises(ValueError, match="kv_len"):
        pg.check_deferred(id1)
    pg.check_deferred(id2)
    del outs1, g1, g2
    pg.clear_deferred()
