"""Decode-step benchmark: paged decode + KV write at the Qwen2-0.5B shape on one MI355X.

One *step* is one decode-layer call of the attention backend on the
headline workload (c2: 14 query / 2 kv heads, head_dim 64, block 16, bf16,
batch 64, kv_len ~ U{128..2048}): the KV write of the step's 64 new tokens
and the paged decode over every sequence's blocks, as one launch (the write
fused into the decode kernel; pool and output bit-identical to the two
separate calls, which are timed beside it). Successive steps use successive
layers of a pool that holds >= 1 GiB in total (the same step metadata, a
different layer's K/V, as in a real engine step). One rotation runs through
the warm-up and every timed loop, so each launch reads a layer that at least
1 GiB of other reads has passed since it was last read: the 256 MB Infinity
Cache cannot serve it, and the measured bandwidth is HBM bandwidth. All
inputs are resident in HBM before timing starts.

Printed (one JSON line): ``value`` = algorithmic bytes of the layer call
(decode + write) / µs per layer call, in GB/s; ``roofline`` for that one
kernel (KV write and cross-partition merge fused) against 8 TB/s;
``workloads`` = the same layer call on the other configurations (c3-c5),
timed the same way; and ``cpu_baseline`` = the oracle's PyTorch CPU path
(the reference's per-token write and per-sequence gather + SDPA loops)
timed on this host's cores in fp32, write and decode apart, on c1 in full
and on c2's shape.

    python bench.py [--steps K] [--warmup W] [--workload c2] [--no-cpu-baseline]
                    [--no-workloads]
    python bench.py --copy-calibration   # plain 256 MiB copies, for PMC byte scaling

``roofline.traffic`` (HBM bytes per layer-call launch) comes from the
rocprofv3 FETCH_SIZE / WRITE_SIZE summary committed under profiles/ for the
workload (``traffic_source`` names it). It is reported only when that
summary was taken on the current decode kernel source (its
``source_sha256`` line matches the hash of the kernel's source files with
comments and layout removed); otherwise it is null and ``traffic_note``
says why.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "mini-vllm-continuous-batching-lab_amd")
sys.path[:0] = [ROOT, PKG]

import torch  # noqa: E402

from benchmarks.paged_decode_workloads import (  # noqa: E402
    HEADLINE, SPECS, WorkloadSpec, decode_bytes, make_layout, write_bytes)

METRIC = "paged decode µs/layer-call + achieved HBM GB/s (% peak), Qwen2-0.5B bs64"
PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0
MIN_WORKING_SET = 1 << 30
OTHER_WORKLOADS = ("c3", "c4", "c5")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_layers(spec, layout, n_layers, device, seed):
    """Per-layer pools (K, V), queries and new-token K/V, N(0,1) in the
    workload's dtype, made on the GPU."""
    g = torch.Generator(device=device).manual_seed(seed)
    nb, hkv, bs, d = layout.num_blocks, spec.num_kv_heads, spec.block_size, spec.head_dim
    b = len(layout.kv_lens)
    layers = []
    for _ in range(n_layers):
        layers.append(dict(
            k=torch.randn(nb, hkv, bs, d, generator=g, device=device).to(spec.dtype),
            v=torch.randn(nb, hkv, bs, d, generator=g, device=device).to(spec.dtype),
            q=torch.randn(b, spec.num_q_heads, d, generator=g, device=device).to(spec.dtype),
            nk=torch.randn(b, hkv, d, generator=g, device=device).to(spec.dtype),
            nv=torch.randn(b, hkv, d, generator=g, device=device).to(spec.dtype),
        ))
    return layers


def layers_for_working_set(spec, layout):
    pool_bytes = 2 * layout.num_blocks * spec.num_kv_heads * spec.block_size * spec.head_dim * \
        torch.tensor([], dtype=spec.dtype).element_size()
    return max(2, math.ceil(MIN_WORKING_SET / pool_bytes)), pool_bytes


class Rotation:
    """The layer each launch reads, in one sequence over the whole run
    (warm-up and every timed loop): the layer read next is always the one
    read longest ago."""

    def __init__(self, layers):
        self.layers = layers
        self.n = 0

    def take(self):
        L = self.layers[self.n % len(self.layers)]
        self.n += 1
        return L


_SLEEP_CYCLES_PER_MS = None


def _hold_gpu(stream, ms):
    """Keep the GPU busy for about ``ms`` so the host can enqueue the timed
    launches ahead of it (torch's bounded clock-spin kernel)."""
    global _SLEEP_CYCLES_PER_MS
    if _SLEEP_CYCLES_PER_MS is None:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        torch.cuda._sleep(1_000_000)
        b.record(stream)
        b.synchronize()
        _SLEEP_CYCLES_PER_MS = 1_000_000 / max(a.elapsed_time(b), 1e-3)
    torch.cuda._sleep(int(_SLEEP_CYCLES_PER_MS * ms))


def time_loop(fn, n, stream, host_us=60.0):
    """GPU time per iteration: the launches run back to back on the GPU
    (host overhead, up to ``host_us`` per iteration, hidden behind a held
    GPU), bracketed by HIP events recorded on the launch stream."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    _hold_gpu(stream, 5 + host_us * 1e-3 * n)
    start.record(stream)
    for i in range(n):
        fn(i)
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) * 1e3 / n  # µs per iteration


def wall_loop(fn, n):
    """Host-inclusive time per iteration (Python wrapper + launch + GPU)."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(n):
        fn(i)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e6 / n


def same_bytes_copy_us(nbytes, device, steps, stream):
    """One plain device copy (torch's copy kernel) moving ``nbytes`` of HBM
    traffic, half read and half written, rotated over >= 1 GiB of buffers
    so the 256 MB MALL cannot serve it: what one launch of that much
    traffic costs on this GPU at this size, launch and ramp included."""
    elems = max(1, nbytes // 4)  # bf16 elements per side: nbytes / 2 bytes each way
    n_buf = max(2, math.ceil(MIN_WORKING_SET / (4 * elems)))
    src = [torch.empty(elems, dtype=torch.bfloat16, device=device).fill_(1) for _ in range(n_buf)]
    dst = [torch.empty_like(x) for x in src]
    for i in range(n_buf):
        dst[i].copy_(src[i])
    return time_loop(lambda i: dst[i % n_buf].copy_(src[i % n_buf]), steps, stream)


def rope_tables(head_dim, theta, max_pos, dtype, device):
    """cos / sin tables of the model's rotary embedding (RotaryEmbedding,
    mini_vllm/model/rotary.py:16-35), built on the device."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim))
    emb = torch.outer(torch.arange(max_pos, dtype=torch.float32, device=device), inv)
    emb = torch.cat((emb, emb), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def torch_rope(x, pos, cos, sin):
    """The reference's eager rotary (rotary.py:44-82): the unfused sequence
    the fused kernel replaces, timed beside it."""
    c, s = cos[pos].unsqueeze(-2), sin[pos].unsqueeze(-2)
    h = x.shape[-1] // 2
    return x * c + torch.cat((-x[..., h:], x[..., :h]), dim=-1) * s


def prefill_measure(dev, steps, warmup):
    """Chunked prefill at the Qwen2-0.5B shape (14 q / 2 kv heads, head_dim
    64, block 16, bf16): 4 sequences with 1536 cached tokens and a 512-token
    chunk each. The HIP kernel against the reference's algorithm
    (paged_attention_gpu.py:577-661: prefix gather, cat, repeat_interleave,
    masked SDPA per sequence; SDPA in fp32, the safe path for batched
    products on this platform)."""
    import torch.nn.functional as F
    from mini_vllm.attention.paged_attention_gpu import gather_prefix_kv, hip_prefill_attention

    hq, hkv, d, bs, dt = 14, 2, 64, 16, torch.bfloat16
    cached, qlen = [1536] * 4, [512] * 4
    n = len(cached)
    need = [-(-(c + q) // bs) for c, q in zip(cached, qlen)]
    nb = sum(need) + 64
    g = torch.Generator(device=dev).manual_seed(0)
    perm = torch.randperm(nb, device=dev, generator=g)
    bt = torch.full((n, max(need)), -1, dtype=torch.int64, device=dev)
    pos = 0
    for i, m in enumerate(need):
        bt[i, :m] = perm[pos:pos + m]
        pos += m
    kc = torch.randn(nb, hkv, bs, d, device=dev, generator=g).to(dt)
    vc = torch.randn(nb, hkv, bs, d, device=dev, generator=g).to(dt)
    t = sum(qlen)
    q = torch.randn(t, hq, d, device=dev, generator=g).to(dt)
    k = torch.randn(t, hkv, d, device=dev, generator=g).to(dt)
    v = torch.randn(t, hkv, d, device=dev, generator=g).to(dt)
    rows = list(range(n))
    stream = torch.cuda.current_stream(dev)

    def hip(i):
        hip_prefill_attention(q, k, v, kc, vc, bt, rows, cached, qlen, bs)

    def reference(i):
        pk, pv = gather_prefix_kv(kc, vc, bt, cached, rows, bs)
        off = poff = 0
        for c, ql in zip(cached, qlen):
            fk = torch.cat([pk[poff:poff + c], k[off:off + ql]]).repeat_interleave(hq // hkv, dim=1)
            fv = torch.cat([pv[poff:poff + c], v[off:off + ql]]).repeat_interleave(hq // hkv, dim=1)
            mask = (torch.arange(c + ql, device=dev).unsqueeze(0)
                    <= torch.arange(c, c + ql, device=dev).unsqueeze(1))
            F.scaled_dot_product_attention(
                q[off:off + ql].permute(1, 0, 2).unsqueeze(0).float().contiguous(),
                fk.permute(1, 0, 2).unsqueeze(0).float().contiguous(),
                fv.permute(1, 0, 2).unsqueeze(0).float().contiguous(),
                attn_mask=mask, scale=d ** -0.5)
            off += ql
            poff += c

    for i in range(warmup):
        hip(i)
        reference(i)
    n_steps = max(5, steps // 10)
    us = time_loop(hip, n_steps, stream, host_us=300.0)
    us_ref = time_loop(reference, n_steps, stream, host_us=2000.0)
    # causal MACs: token t of a chunk attends cached + t + 1 keys, QK^T and PV
    flops = sum(4 * hq * d * (ql * c + ql * (ql + 1) // 2) for c, ql in zip(cached, qlen))
    tflops = flops / us / 1e6
    return {
        "workload": "Qwen2-0.5B chunked prefill: 14 q / 2 kv heads, head_dim 64, block 16, bf16, "
                    "4 sequences x (1536 cached + 512 chunk)",
        "us": round(us, 2),
        "tflops": round(tflops, 2),
        "frac_of_bf16_peak": round(tflops / PEAK_BF16_TFLOPS, 4),
        "reference_algorithm_us": round(us_ref, 1),
    }


def plan_step_us(bt, kv, bs, num_blocks, dev, spec, plan_decode, reps=20):
    """Host time of one step's decode plan in steady state (median): the
    plan kernel plus the read-back of its status. Fresh copies of the
    metadata defeat the per-step plan cache, as a new engine step would."""
    times = []
    for _ in range(reps):
        b2, k2 = bt.clone(), kv.clone()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        plan_decode(b2, k2, bs, num_blocks, dev, spec.head_dim, spec.dtype, spec.num_kv_heads)
        times.append((time.perf_counter() - t0) * 1e6)
    return statistics.median(times)


def checks_measure(dev, stream, bt, kv, slots, num_blocks, bs, steps):
    """GPU time (events) of the per-step metadata checks, called through the
    C ABI so that no per-step cache skips them: the slot check at the
    step's token count and at a 32k-token prefill step (the grid path over
    a workspace hash table), and the fused-write check (both launches)."""
    import ctypes

    from mini_vllm.attention import _hip

    lib = _hip.load()
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    s = ctypes.c_void_p(stream.cuda_stream)
    status = torch.empty(2, dtype=torch.int32, device=dev)
    out = {}
    big = torch.randperm(max(2 * 32768, num_blocks * bs), device=dev)[:32768].to(torch.int64)
    for name, sl in (("slots_check_us", slots), ("slots_check_32k_us", big)):
        n = sl.numel()
        nbytes = lib.mv_kv_slots_check_workspace_bytes(n)
        ws = torch.empty(max(nbytes, 8), dtype=torch.uint8, device=dev)
        total = max(num_blocks * bs, 2 * 32768)
        call = lambda i: lib.mv_kv_slots_check(ptr(sl), n, total, ptr(status), ptr(ws),  # noqa: E731
                                               nbytes, s)
        for i in range(5):
            call(i)
        out[name] = round(time_loop(call, steps, stream), 3)
    n = kv.shape[0]
    nbytes = lib.mv_decode_write_check_workspace_bytes(n)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    call = lambda i: lib.mv_decode_write_check(  # noqa: E731
        ptr(slots), ptr(bt), 1, bt.stride(0), ptr(kv), 1, n, bt.shape[1], bs, ptr(status),
        ptr(ws), nbytes, s)
    for i in range(5):
        call(i)
    out["fused_write_check_us"] = round(time_loop(call, steps, stream), 3)
    return out


def measure_workload(name, steps, warmup, dev, stream, seed):
    """The fused layer call (KV write + decode, one launch) and decode alone
    on another configuration, timed as the headline: >= 1 GiB of per-layer
    pools in one rotation, event-timed back-to-back launches."""
    from mini_vllm.attention.paged_attention_gpu import hip_decode_attention, plan_decode

    spec = SPECS[name]
    layout = make_layout(spec, seed)
    n_layers, _ = layers_for_working_set(spec, layout)
    layers = build_layers(spec, layout, n_layers, dev, seed)
    bt = layout.block_table().to(dev)
    kv = torch.tensor(layout.kv_lens, dtype=torch.int64, device=dev)
    slots = layout.new_token_slots().to(dev)
    bs = spec.block_size
    plan = plan_decode(bt, kv, bs, layout.num_blocks, dev, spec.head_dim, spec.dtype,
                       spec.num_kv_heads)
    rot = Rotation(layers)

    def layer_call(i):
        L = rot.take()
        hip_decode_attention(L["q"], L["k"], L["v"], bt, kv, bs, new_key=L["nk"],
                             new_value=L["nv"], slot_mapping=slots)

    def decode_only(i):
        L = rot.take()
        hip_decode_attention(L["q"], L["k"], L["v"], bt, kv, bs)

    for i in range(max(warmup, n_layers)):
        layer_call(i)
    us = time_loop(layer_call, steps, stream)
    us_dec = time_loop(decode_only, steps, stream)
    dec_bytes = decode_bytes(layout, spec.dtype)
    wr_bytes = write_bytes(layout, spec.dtype)
    res = {
        "shape": f"{spec.num_q_heads} q / {spec.num_kv_heads} kv heads, head_dim {spec.head_dim}, "
                 f"block {bs}, batch {len(layout.kv_lens)}, kv_len {spec.ctx}",
        "mean_kv_len": round(sum(layout.kv_lens) / len(layout.kv_lens), 1),
        "us_per_layer_call": round(us, 3),
        "decode_us": round(us_dec, 3),
        "algorithmic_bytes": dec_bytes + wr_bytes,
        "gbs": round((dec_bytes + wr_bytes) / us / 1e3, 1),
        "frac": round((dec_bytes + wr_bytes) / us / 1e3 / PEAK_HBM_GBS, 4),
        "work_groups": plan.num_groups,
        "partition_tokens": plan.partition_tokens,
        "layers_rotated": n_layers,
    }
    if layout.shared_blocks:
        uniq = decode_bytes(layout, spec.dtype, unique=True) + wr_bytes
        res["unique_bytes"] = uniq
        res["frac_unique"] = round(uniq / us / 1e3 / PEAK_HBM_GBS, 4)
    del layers, rot
    torch.cuda.empty_cache()
    return res


def reference_shapes(dev, stream, steps):
    """The reference's own micro-benchmark shapes (Qwen2-0.5B heads: 14 q /
    2 kv, head_dim 64, block 16, fp16; batch 1 and 4 at context 16, 128 and
    512; benchmarks/benchmark_paged_attention.py:273-503): decode alone, by
    events over back-to-back launches and host-inclusive (the wrapper's
    Python, as the reference's timing includes). Context for the published
    Triton rows only: those come from another GPU."""
    from mini_vllm.attention.paged_attention_gpu import hip_decode_attention

    published = {(1, 16): 101.84, (1, 128): 121.11, (1, 512): 287.16,
                 (4, 16): 78.95, (4, 128): 121.67, (4, 512): 300.03}
    rows = []
    for (b, ctx), ref_us in published.items():
        spec = WorkloadSpec(f"ref-b{b}-c{ctx}", 14, 2, 64, 16, torch.float16, b,
                            ("fixed", [ctx] * b), pool_blocks=max(512, b * (-(-ctx // 16)) * 2))
        layout = make_layout(spec, 0)
        L = build_layers(spec, layout, 1, dev, 1)[0]
        bt = layout.block_table().to(dev)
        kv = torch.tensor(layout.kv_lens, dtype=torch.int64, device=dev)

        def call(i):
            hip_decode_attention(L["q"], L["k"], L["v"], bt, kv, 16)

        for i in range(10):
            call(i)
        us = time_loop(call, steps, stream)
        us_wall = wall_loop(call, steps)
        rows.append({"batch": b, "ctx": ctx, "us": round(us, 2),
                     "host_inclusive_us": round(us_wall, 2),
                     "reference_triton_us_rtx3060": ref_us})
    return rows


def _cpu_median(fn, budget_s, max_n=7):
    fn()  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < max_n and (len(times) < 2 or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times) * 1e6, len(times)


def cpu_baseline(spec, layout, layer, budget_s=8.0):
    """The oracle's CPU path (the reference's loops, fp32) on all host cores,
    write and decode timed apart: c2's shape (the headline's layer, full
    batch) on a bounded sample, and c1 in full."""
    from benchmarks.paged_decode_workloads import make_case
    from oracle import paged_ref

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)

    def timings(kc, vc, q, nk, nv, bt, kv, slots, bs, budget):
        def write():
            paged_ref.write_to_paged_cache(nk, nv, kc, vc, slots, bs)

        def decode():
            return paged_ref.decode_from_tables(q, kc, vc, bt, kv, bs)

        w_us, w_n = _cpu_median(write, budget / 4)
        d_us, d_n = _cpu_median(decode, budget)
        return w_us, d_us, min(w_n, d_n)

    # c2's shape: the bench's own layer, in fp32 on the CPU
    w_us, d_us, n = timings(layer["k"].float().cpu(), layer["v"].float().cpu(),
                            layer["q"].float().cpu(), layer["nk"].float().cpu(),
                            layer["nv"].float().cpu(), layout.block_table(),
                            torch.tensor(layout.kv_lens, dtype=torch.int64),
                            layout.new_token_slots(), spec.block_size, budget_s)
    nbytes = decode_bytes(layout, spec.dtype) + write_bytes(layout, spec.dtype)
    us = w_us + d_us
    c1 = make_case("c1", seed=0)
    c1_w, c1_d, c1_n = timings(c1.key_cache.clone(), c1.value_cache.clone(), c1.query,
                               c1.new_key, c1.new_value, c1.block_table, c1.kv_len,
                               c1.slot_mapping, 16, 2.0)
    return {
        "value": round(nbytes / us / 1e3, 4),
        "unit": "GB/s",
        "us_per_layer_call": round(us, 1),
        "write_us": round(w_us, 1),
        "decode_us": round(d_us, 1),
        "cores": cores,
        "kind": "port",
        "sample": (f"median of {n} write calls ({len(layout.kv_lens)} tokens) and {n} decode "
                   f"calls ({len(layout.kv_lens)} sequences) at {spec.name}'s shape in fp32 with "
                   f"torch.set_num_threads({cores}); GB/s on the bf16 workload's algorithmic "
                   f"bytes over write + decode"),
        "c1": {"write_us": round(c1_w, 1), "decode_us": round(c1_d, 1),
               "us_per_layer_call": round(c1_w + c1_d, 1),
               "sample": f"c1 in full (4 tokens written, 4 sequences decoded, fp32), "
                         f"median of {c1_n}"},
    }


TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "paged_decode_write_kernel_{workload}_traffic.md")
KERNEL_SOURCES = ("csrc/paged_decode.hip", "csrc/mv_tile.h", "csrc/mv_common.h",
                  "csrc/mv_coherent.h", "csrc/mv_rope.h", "csrc/mv_step_check.h")
COPY_BYTES = 256 << 20


def code_without_comments(text):
    """C/C++ source text with its comments removed and every run of blank
    space collapsed to one space: what the compiler sees, so an edit of a
    comment or of the layout leaves it unchanged. String and character
    literals are kept as written."""
    out, i, n = [], 0, len(text)
    while i < n:
        c = text[i]
        if c == "/" and text.startswith("//", i):
            j = text.find("\n", i)
            i = n if j < 0 else j
            out.append(" ")
        elif c == "/" and text.startswith("/*", i):
            j = text.find("*/", i + 2)
            i = n if j < 0 else j + 2
            out.append(" ")
        elif c in "\"'":
            j = i + 1
            while j < n and text[j] != c:
                j += 2 if text[j] == "\\" else 1
            out.append(text[i:j + 1])
            i = j + 1
        else:
            out.append(c)
            i += 1
    return " ".join("".join(out).split())


def kernel_source_sha256():
    """Hash of the decode kernel's sources (the files a PMC profile of it
    depends on) without comments or layout, as written into the traffic
    summaries."""
    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        with open(os.path.join(PKG, rel), encoding="utf-8") as f:
            h.update(code_without_comments(f.read()).encode())
        h.update(b"\0")
    return h.hexdigest()


def measured_traffic(workload):
    """HBM bytes per layer-call launch (the decode kernel with the KV write
    fused) from the committed PMC summary: (bytes, source, note). The bytes
    are None when there is no summary or it was taken on other kernel
    sources than the current ones."""
    path = TRAFFIC_SUMMARY.format(workload=workload)
    rel = os.path.relpath(path, ROOT)
    fields = {}
    try:
        with open(path) as f:
            for line in f:
                key, sep, val = line.strip().partition(":")
                if sep and key in ("traffic_bytes_per_launch", "source_sha256"):
                    fields[key] = val.strip()
    except OSError:
        return None, None, f"no PMC summary at {rel}"
    if "traffic_bytes_per_launch" not in fields:
        return None, rel, f"{rel} has no traffic_bytes_per_launch line"
    if fields.get("source_sha256") != kernel_source_sha256():
        return None, rel, f"{rel} was profiled on other decode kernel sources than these"
    return int(fields["traffic_bytes_per_launch"]), rel, (
        "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of this kernel source, scaled by a plain copy's "
        "counts (committed summary, not measured in this run)")


def copy_calibration(steps):
    """A plain device copy of COPY_BYTES (read COPY_BYTES, write COPY_BYTES)
    per launch: what FETCH_SIZE / WRITE_SIZE report for it scales the
    counters of the decode kernel to bytes."""
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_launch": COPY_BYTES, "launches": steps}), flush=True)
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default=HEADLINE, choices=sorted(SPECS))
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-workloads", action="store_true",
                    help="skip the other configurations' layer calls")
    ap.add_argument("--copy-calibration", action="store_true")
    args = ap.parse_args(argv)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: the decode hot path runs on a single MI355X "
              f"(requested --gpus {args.gpus}, WORLD_SIZE {world}); multi-GPU sharding is "
              f"design-only in this build.", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    if args.copy_calibration:
        return copy_calibration(args.steps if args.steps != 200 else 10)

    from mini_vllm.attention import _hip
    from mini_vllm.attention.paged_attention_gpu import (
        hip_cache_write, hip_decode_attention, hip_rope_kv_cache_write, plan_decode)

    _hip.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    spec = SPECS[args.workload]
    layout = make_layout(spec, args.seed)
    bs = spec.block_size
    n_layers, pool_bytes = layers_for_working_set(spec, layout)
    log(f"[bench] workload {spec.name}: B={len(layout.kv_lens)} blocks={layout.num_blocks} "
        f"layers={n_layers} ({n_layers * pool_bytes / 2**30:.2f} GiB of K/V)")
    layers = build_layers(spec, layout, n_layers, dev, args.seed)
    rot = Rotation(layers)
    bt = layout.block_table().to(dev)
    kv = torch.tensor(layout.kv_lens, dtype=torch.int64, device=dev)
    slots = layout.new_token_slots().to(dev)
    stream = torch.cuda.current_stream(dev)

    # per-step validation/planning (once per engine step, shared by all layers)
    plan = plan_decode(bt, kv, bs, layout.num_blocks, dev, spec.head_dim, spec.dtype,
                       spec.num_kv_heads)
    plan_us = plan_step_us(bt, kv, bs, layout.num_blocks, dev, spec, plan_decode)
    checks = checks_measure(dev, stream, bt, kv, slots, layout.num_blocks, bs, 50)
    log(f"[bench] checks (GPU us): {checks}")

    def layer_call(i):  # one launch: the step's KV write fused into the decode
        L = rot.take()
        hip_decode_attention(L["q"], L["k"], L["v"], bt, kv, bs, new_key=L["nk"],
                             new_value=L["nv"], slot_mapping=slots)

    def layer_call_two(i):  # the reference's two calls: write, then decode
        L = rot.take()
        hip_cache_write(L["nk"], L["nv"], L["k"], L["v"], slots, bs)
        hip_decode_attention(L["q"], L["k"], L["v"], bt, kv, bs)

    def decode_only(i):
        L = rot.take()
        hip_decode_attention(L["q"], L["k"], L["v"], bt, kv, bs)

    def write_only(i):
        L = rot.take()
        hip_cache_write(L["nk"], L["nv"], L["k"], L["v"], slots, bs)

    for i in range(max(args.warmup, n_layers)):
        layer_call_two(i)
        layer_call(i)
    torch.cuda.synchronize()
    log(f"[bench] warmup done ({args.warmup} steps); timing {args.steps} steps")
    us_step = time_loop(layer_call, args.steps, stream)
    us_two = time_loop(layer_call_two, args.steps, stream)
    us_decode = time_loop(decode_only, args.steps, stream)
    us_write = time_loop(write_only, args.steps, stream)
    us_wall = wall_loop(layer_call, args.steps)
    us_two_wall = wall_loop(layer_call_two, args.steps)
    log(f"[bench] layer call {us_step:.2f} us (write fused); write + decode calls {us_two:.2f} us "
        f"(decode {us_decode:.2f}, write {us_write:.2f})")

    # The decode attention sub-layer (qwen_runner.py:164-190 for the decode
    # rows): RoPE of q and the new k, the KV write and the decode, in one
    # launch, against the two launches of fused RoPE + write, then decode.
    cos, sin = rope_tables(spec.head_dim, 1000000.0, 32768, spec.dtype, dev)
    pos = kv - 1  # the new token's position in each sequence

    def sublayer(i):
        L = rot.take()
        hip_decode_attention(L["q"], L["k"], L["v"], bt, kv, bs, new_key=L["nk"],
                             new_value=L["nv"], slot_mapping=slots, positions=pos, cos=cos,
                             sin=sin)

    def sublayer_two(i):
        L = rot.take()
        q_rot, _ = hip_rope_kv_cache_write(L["q"], L["nk"], L["nv"], pos, cos, sin, L["k"], L["v"],
                                           slots, bs, return_key=False)
        hip_decode_attention(q_rot, L["k"], L["v"], bt, kv, bs)

    for i in range(args.warmup):
        sublayer(i)
        sublayer_two(i)
    us_sub = time_loop(sublayer, args.steps, stream)
    us_sub_two = time_loop(sublayer_two, args.steps, stream)
    log(f"[bench] attention sub-layer (RoPE + write + decode) {us_sub:.2f} us in one launch, "
        f"{us_sub_two:.2f} us as RoPE+write then decode")

    # A whole decode step captured into one HIP graph: the plan (replanned
    # from the static metadata at every replay), the RoPE rows, and
    # Qwen2-0.5B's 24 attention sub-layers; no host work per layer.
    from mini_vllm.attention.paged_attention_gpu import check_deferred, clear_deferred, last_capture_id
    graph_layers = 24
    graphs = {}
    for name, fn in (("sublayer", sublayer), ("write_decode", layer_call)):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(graph_layers):
                fn(i)
        gid = last_capture_id()
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        check_deferred(gid)
        g_steps = max(5, args.steps // graph_layers)
        us_graph = time_loop(lambda i: graph.replay(), g_steps, stream, host_us=100.0)
        us_graph_wall = wall_loop(lambda i: graph.replay(), g_steps)
        graphs[name] = (us_graph, us_graph_wall)
        del graph
        clear_deferred()
        log(f"[bench] captured step {name} ({graph_layers} layers + plan): {us_graph:.1f} us GPU, "
            f"{us_graph_wall:.1f} us host-inclusive")

    # The same step eager: new metadata tensors every step, as the
    # reference's input builder makes them (here device copies of the
    # step's tables, lengths, slots and positions), so the first layer
    # plans and checks and reads the results back once, and 24 sub-layer
    # calls follow; host-inclusive.
    def eager_step(i):
        b2, k2, s2, p2 = bt.clone(), kv.clone(), slots.clone(), pos.clone()
        for _ in range(graph_layers):
            L = rot.take()
            hip_decode_attention(L["q"], L["k"], L["v"], b2, k2, bs, new_key=L["nk"],
                                 new_value=L["nv"], slot_mapping=s2, positions=p2, cos=cos,
                                 sin=sin)

    for i in range(3):
        eager_step(i)
    us_eager_step = wall_loop(eager_step, max(5, args.steps // graph_layers))
    log(f"[bench] eager step ({graph_layers} sub-layers, plan and checks at the first): "
        f"{us_eager_step:.1f} us host-inclusive")

    # o_proj of the decode rows (qwen_runner.py:190-193): a [B, Hq*D] x
    # [Hq*D, hidden] GEMM (torch / hipBLASLt), for the fusion decision
    hidden = spec.num_q_heads * spec.head_dim
    w_o = torch.randn(hidden, hidden, device=dev).to(spec.dtype)
    a_o = torch.randn(len(layout.kv_lens), hidden, device=dev).to(spec.dtype)
    for _ in range(5):
        torch.matmul(a_o, w_o.t())
    us_oproj = time_loop(lambda i: torch.matmul(a_o, w_o.t()), args.steps, stream)
    log(f"[bench] o_proj GEMM [{len(layout.kv_lens)} x {hidden}] x [{hidden} x {hidden}]: "
        f"{us_oproj:.2f} us")

    prefill = prefill_measure(dev, args.steps, min(args.warmup, 5))
    log(f"[bench] prefill {prefill['us']:.1f} us ({prefill['tflops']:.1f} TFLOP/s), "
        f"reference algorithm {prefill['reference_algorithm_us']:.1f} us")

    # RoPE of the step's q and new k + KV write: fused kernel against the
    # reference's sequence (two eager rotaries, then the cache write)
    def rope_fused(i):
        L = rot.take()
        hip_rope_kv_cache_write(L["q"], L["nk"], L["nv"], pos, cos, sin, L["k"], L["v"], slots, bs,
                                return_key=False)

    def rope_unfused(i):
        L = rot.take()
        torch_rope(L["q"], pos, cos, sin)
        k = torch_rope(L["nk"], pos, cos, sin)
        hip_cache_write(k, L["nv"], L["k"], L["v"], slots, bs)

    for i in range(args.warmup):
        rope_fused(i)
        rope_unfused(i)
    us_rope = time_loop(rope_fused, args.steps, stream)
    us_rope_unfused = time_loop(rope_unfused, args.steps, stream, host_us=200.0)
    us_rope_wall = wall_loop(rope_fused, args.steps)
    us_rope_unfused_wall = wall_loop(rope_unfused, args.steps)
    log(f"[bench] rope+write fused {us_rope:.2f} us (host-incl {us_rope_wall:.1f}), "
        f"unfused {us_rope_unfused:.2f} us (host-incl {us_rope_unfused_wall:.1f})")

    dec_bytes = decode_bytes(layout, spec.dtype)
    wr_bytes = write_bytes(layout, spec.dtype)
    us_copy = same_bytes_copy_us(dec_bytes + wr_bytes, dev, args.steps, stream)
    log(f"[bench] plain copy of the same HBM bytes: {us_copy:.2f} us")
    ref_shapes = reference_shapes(dev, stream, max(20, args.steps // 4))
    log("[bench] reference shapes: " + ", ".join(
        f"b{r['batch']} ctx{r['ctx']} {r['us']:.1f} us" for r in ref_shapes))
    traffic, traffic_source, traffic_note = measured_traffic(spec.name)
    gbs = (dec_bytes + wr_bytes) / us_step / 1e3
    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_step / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if spec.dtype == torch.bfloat16 else str(spec.dtype).replace("torch.", ""),
        "data": "synthetic",
        "config": {
            "workload": (f"{spec.name}: paged decode layer call (KV write + decode), "
                         f"{spec.num_q_heads} q / {spec.num_kv_heads} kv heads, head_dim "
                         f"{spec.head_dim}, block {bs}, batch {len(layout.kv_lens)}, "
                         f"kv_len {spec.ctx}"),
            "batch": len(layout.kv_lens),
            "mean_kv_len": round(sum(layout.kv_lens) / len(layout.kv_lens), 1),
            "layers_rotated": n_layers,
            "parallelism": "single GPU",
        },
        "us_per_layer_call": round(us_step, 3),
        "layer_call": "one launch: decode with the step's KV write fused (hip_decode_attention "
                      "with new_key/new_value/slot_mapping); pool and output bit-identical to "
                      "the two calls",
        "two_call_us_per_layer_call": round(us_two, 3),
        "decode_us": round(us_decode, 3),
        "write_us": round(us_write, 3),
        "host_inclusive_us_per_layer_call": round(us_wall, 3),
        "two_call_host_inclusive_us": round(us_two_wall, 3),
        "pct_peak_hbm": round(100 * gbs / PEAK_HBM_GBS, 2),
        "plan_us_per_step": round(plan_us, 1),
        "checks": checks,
        "sublayer": {
            "what": "decode attention sub-layer (qwen_runner.py:164-190, decode rows): RoPE of q "
                    "and new k + KV write + decode",
            "one_launch_us": round(us_sub, 3),
            "rope_write_then_decode_us": round(us_sub_two, 3),
        },
        "graph_step": {
            "what": "one HIP graph: decode plan + RoPE rows + 24 attention sub-layers (RoPE + "
                    "KV write + decode, one launch each)",
            "layers": graph_layers,
            "us_per_step": round(graphs["sublayer"][0], 2),
            "us_per_layer": round(graphs["sublayer"][0] / graph_layers, 3),
            "host_inclusive_us_per_step": round(graphs["sublayer"][1], 2),
            "without_rope_us_per_step": round(graphs["write_decode"][0], 2),
            "eager_host_inclusive_us_per_step": round(us_eager_step, 2),
        },
        "o_proj_gemm_us": round(us_oproj, 3),
        "prefill": prefill,
        "rope_write": {
            "what": "RoPE of the step's q and new k + KV write (qwen_runner.py:164-170)",
            "fused_us": round(us_rope, 3),
            "unfused_us": round(us_rope_unfused, 3),
            "fused_host_inclusive_us": round(us_rope_wall, 2),
            "unfused_host_inclusive_us": round(us_rope_unfused_wall, 2),
        },
        "reference_shapes": ref_shapes,
        "partition_tokens": plan.partition_tokens,
        "work_groups": plan.num_groups,
        "roofline": {
            "bound": "hbm",
            "kernel": "paged_decode_kernel with the KV write fused (one launch per layer call, "
                      "partition merge fused)",
            "achieved": round(gbs, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(gbs / PEAK_HBM_GBS, 4),
            "algorithmic_bytes": dec_bytes + wr_bytes,
            "decode_only_frac": round(dec_bytes / us_decode / 1e3 / PEAK_HBM_GBS, 4),
            "same_bytes_copy_us": round(us_copy, 3),
            "same_bytes_copy_frac": round((dec_bytes + wr_bytes) / us_copy / 1e3 / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "traffic_note": traffic_note,
        },
        "workloads": {},
        "cpu_baseline": None,
    }
    if layout.shared_blocks:  # shared prefixes: the roofline on the bytes that must move
        uniq = decode_bytes(layout, spec.dtype, unique=True) + wr_bytes
        result["roofline"]["unique_bytes"] = uniq
        result["roofline"]["frac_unique"] = round(uniq / us_step / 1e3 / PEAK_HBM_GBS, 4)
    cpu_layer = layers[0]
    del layers, rot
    torch.cuda.empty_cache()
    if not args.no_workloads:
        for name in OTHER_WORKLOADS:
            if name == spec.name:
                continue
            w = measure_workload(name, max(50, args.steps // 2), args.warmup, dev, stream,
                                 args.seed)
            result["workloads"][name] = w
            log(f"[bench] {name}: layer call {w['us_per_layer_call']:.2f} us, frac {w['frac']}"
                + (f" (unique bytes {w['frac_unique']})" if "frac_unique" in w else ""))
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(spec, layout, cpu_layer)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
