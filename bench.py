"""Benchmark of the needle.js decode hot path on one MI355X.

Prints ONE JSON line.  `value` is the int8 matvec throughput (GB/s of
algorithmic bytes) on the isolated matvec workload: W int8 [4096][4096] with
fp32 scales per group of 32, x fp32 [4096], batch 1.  The inputs are resident
in HBM before timing starts; the timed launches rotate over enough weight
replicas (> 256 MB) that every launch streams its weights from HBM rather
than from the 256 MB Infinity Cache.  Launches are captured in one HIP graph;
at least `--steps` launches are timed, over at least 5 replays, each replay
bracketed by its own HIP events on the replay stream, and the median replay
gives the time per launch.  `steps` is the number of launches timed.

`parts` adds the other headline numbers: batch-8 matvec and single-query
int8-KV decode attention (8 heads x 64, contexts 512/2048/8192), each with
its HBM roofline fraction (peak 8 TB/s) and, for reference, the same kernel
on an Infinity-Cache-resident working set; the read-only streaming rate of a
1 GiB buffer and a device copy of each kernel's size (what one launch of
that size reaches); batch-64 constrained decode; the 2048-token prefill
(GEMM int8 TOPS and attention TFLOP/s each over its own kernel time, last
logits against the oracle's).

`parts.needle2_generate_b1` is Needle 2 at the shipped geometry, batch 1:
greedy generate of 64 tokens from a 128-token prompt (wall time of the whole
call, as NeedleModel.generate reports tokensPerSecond), plus decode-only and
prefill-only figures and the same call through the session methods.

`cpu_baseline` times the oracle (the C restatement of the reference CPU
path, one thread) on a bounded sample of the same matvec workload.  The
model legs' CPU baselines run their whole workloads on the oracle (threads
stated in each), never a sample scaled up.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT, ROOT / "needle.js_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20
ROTATE_BYTES = 640 << 20  # rotation set well above the Infinity Cache


def matvec_bytes(n, k, g, batch):
    """Algorithmic bytes of one int8 matvec launch: codes + scales + x + y."""
    return n * k + n * (k // g) * 4 + batch * k * 4 + batch * n * 4


def attention_bytes(length, heads):
    """K and V codes (64 B each per token-head), their f32 scales, q and out."""
    return heads * length * (64 + 64 + 4 + 4) + 2 * heads * 64 * 4


class GraphTimer:
    """Captures `launch(stream)` calls into one HIP graph and times replays."""

    def __init__(self, torch, launches):
        self.torch = torch
        self.graph = torch.cuda.CUDAGraph()
        self.stream = torch.cuda.Stream()
        self.n = len(launches)
        torch.cuda.synchronize()
        with torch.cuda.stream(self.stream):
            handle = self.stream.cuda_stream
            for f in launches:  # one eager pass before capture
                f(handle)
        self.stream.synchronize()
        with torch.cuda.graph(self.graph, stream=self.stream):
            handle = torch.cuda.current_stream().cuda_stream
            for f in launches:
                f(handle)
        torch.cuda.synchronize()

    def time(self, replays, warmup):
        """(median over the replays of the ms per launch, launches timed):
        at least 5 replays, each bracketed by its own pair of HIP events on
        the replay stream."""
        torch = self.torch
        replays = max(5, replays)
        for _ in range(warmup):
            self.graph.replay()
        torch.cuda.synchronize()
        events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(replays)]
        with torch.cuda.stream(self.stream):
            for start, stop in events:
                start.record(self.stream)
                self.graph.replay()
                stop.record(self.stream)
        torch.cuda.synchronize()
        per = sorted(start.elapsed_time(stop) / self.n for start, stop in events)
        return per[len(per) // 2], replays * self.n


def bench_matvec(torch, hip, n, k, g, batch, steps, warmup, rotate=True):
    import ctypes as C

    import numpy as np

    from needle_hip import lib as L
    from needle_hip import synth

    per = matvec_bytes(n, k, g, batch)
    replicas = max(1, math.ceil(ROTATE_BYTES / per)) if rotate else 1
    w, s = synth.int8_matrix(2026, f"bench-w{n}x{k}", n, k, g)
    mats = []
    for _ in range(replicas):
        h = C.c_void_p()
        hip._check(hip.lib.nd_mat_upload_i8(hip.ctx, L.ptr(w), L.ptr(s), n, k, g, C.byref(h)))
        mats.append(h)
    x = torch.from_numpy(synth.Stream(2026, "bench-x").normal((batch, k))).cuda()
    y = torch.empty((batch, n), dtype=torch.float32, device="cuda")

    def make(h):
        return lambda stream: hip._check(hip.lib.nd_matvec_d(
            hip.ctx, h, x.data_ptr(), batch, 0, n, y.data_ptr(), C.c_void_p(stream)))

    timer = GraphTimer(torch, [make(mats[i % replicas]) for i in range(max(replicas, 32))])
    ms, timed = timer.time(math.ceil(steps / timer.n), warmup)
    for h in mats:
        hip.lib.nd_mat_free(hip.ctx, h)
    gbs = per / (ms * 1e-3) / 1e9
    return {"bytes_per_launch": per, "replicas": replicas, "launches": timed,
            "ms_per_launch": ms, "GBps": gbs, "frac_hbm": gbs / HBM_PEAK_GBS}


def bench_matvec_span(torch, hip, n, k, g, steps, warmup):
    """The batch-1 matvec workload of bench_matvec (same rotated replicas,
    same graph timing) through nd_matvec_stamped_d: the same kernel body and
    grid with every workgroup's entry and exit read from the GPU's 100 MHz
    clock.  Per launch of the last replay: body span = latest exit - earliest
    entry; interval = earliest entry of the next launch - earliest entry of
    this one (the per-launch cadence the HIP events time).  Medians."""
    import ctypes as C

    import numpy as np

    from needle_hip import lib as L
    from needle_hip import synth

    per = matvec_bytes(n, k, g, 1)
    replicas = max(1, math.ceil(ROTATE_BYTES / per))
    w, s = synth.int8_matrix(2026, f"bench-w{n}x{k}", n, k, g)
    mats = []
    for _ in range(replicas):
        h = C.c_void_p()
        hip._check(hip.lib.nd_mat_upload_i8(hip.ctx, L.ptr(w), L.ptr(s), n, k, g, C.byref(h)))
        mats.append(h)
    x = torch.from_numpy(synth.Stream(2026, "bench-x").normal((1, k))).cuda()
    y = torch.empty((1, n), dtype=torch.float32, device="cuda")
    launches = max(replicas, 32)
    cap = 4096
    stamps = torch.zeros((launches, cap, 2), dtype=torch.int64, device="cuda")
    wgs = C.c_uint32(0)

    def make(i):
        h = mats[i % replicas]
        return lambda stream: hip._check(hip.lib.nd_matvec_stamped_d(
            hip.ctx, h, x.data_ptr(), 0, n, y.data_ptr(), stamps[i].data_ptr(), cap,
            C.byref(wgs), C.c_void_p(stream)))

    timer = GraphTimer(torch, [make(i) for i in range(launches)])
    ms, timed = timer.time(math.ceil(steps / timer.n), warmup)
    st = stamps[:, :wgs.value, :].cpu().numpy()
    for h in mats:
        hip.lib.nd_mat_free(hip.ctx, h)
    first = st[:, :, 0].min(axis=1)
    last_in = st[:, :, 0].max(axis=1)
    last = st[:, :, 1].max(axis=1)
    span_us = (last - first) * 0.01
    entry_spread_us = (last_in - first) * 0.01
    interval_us = np.diff(first) * 0.01
    return {"workgroups": wgs.value, "launches": int(launches), "events_ms_per_launch": ms,
            "body_span_us_median": float(np.median(span_us)),
            "body_span_us_mean": float(np.mean(span_us)),
            "entry_spread_us_median": float(np.median(entry_spread_us)),
            "launch_interval_us_median": float(np.median(interval_us)),
            "body_GBps": per / (float(np.median(span_us)) * 1e-6) / 1e9}


def cq_matvec_bytes(n, k, g, bits, batch):
    """Algorithmic bytes of one Cactus-Quant matvec call: packed codes,
    binary16 norms, x and y (the rotated copy of x is the call's own
    intermediate)."""
    kpad = -(-k // g) * g
    pb = 2 if bits == 5 else bits
    return n * kpad * pb // 8 + n * (kpad // g) * 2 + batch * k * 4 + batch * n * 4


def bench_cq_matvec(torch, hip, n, k, g, bits, batch, steps, warmup):
    """nd_matvec_d on a CQ matrix (rotation kernel + matvec kernel per call),
    weights rotated over enough HBM replicas to defeat the Infinity Cache."""
    import ctypes as C

    from needle_hip import lib as L
    from needle_hip import synth

    per = cq_matvec_bytes(n, k, g, bits, batch)
    replicas = max(1, math.ceil(ROTATE_BYTES / per))
    packed, norms = synth.cq_matrix(2026, f"bench-cq{n}x{k}g{g}b{bits}", n, k, g, bits)
    codebook = synth.cq_codebook()
    lo = {2: 0, 3: 4, 4: 12, 5: 0}[bits]
    book = codebook[lo:]
    mats = []
    for _ in range(replicas):
        h = C.c_void_p()
        hip._check(hip.lib.nd_mat_upload_cq(hip.ctx, L.ptr(packed), L.ptr(norms), L.ptr(book), n,
                                            k, g, bits, C.byref(h)))
        mats.append(h)
    x = torch.from_numpy(synth.Stream(2026, "bench-x").normal((batch, k))).cuda()
    y = torch.empty((batch, n), dtype=torch.float32, device="cuda")

    def make(h):
        return lambda stream: hip._check(hip.lib.nd_matvec_d(
            hip.ctx, h, x.data_ptr(), batch, 0, n, y.data_ptr(), C.c_void_p(stream)))

    timer = GraphTimer(torch, [make(mats[i % replicas]) for i in range(max(replicas, 32))])
    ms, timed = timer.time(math.ceil(steps / timer.n), warmup)
    for h in mats:
        hip.lib.nd_mat_free(hip.ctx, h)
    gbs = per / (ms * 1e-3) / 1e9
    return {"bits": bits, "group": g, "bytes_per_call": per, "replicas": replicas,
            "calls": timed, "ms_per_call": ms, "GBps": gbs,
            "frac_hbm": gbs / HBM_PEAK_GBS}


def bench_grammar_mask(torch, hip, reps, cpu_seconds):
    """Allowed-token masks of the tool-call grammar over an 8192-piece
    vocabulary, at every state along a complete two-call output of the demo
    tools (longest-piece tokenization): the device kernel alone (states
    resident in HBM, one launch per mask, HIP events), the host call with
    its undecided pieces settled and the allowed id list built, the same
    with the mask kept in a model's mask buffer for the selection (no id
    list), and the agent's own loop (a grammar clone fed per piece,
    tools/agent.ts:164-175) on the host as the CPU baseline."""
    import ctypes as C

    import numpy as np

    from needle_hip import synth
    from needle_hip.grammar import ToolCallGrammar, allowed_pieces
    from needle_hip.maskgen import GrammarMasker, state_words

    tools = synth.demo_tools()
    pieces, eligible = synth.tool_pieces(7, 8192, tools)
    masker = GrammarMasker(hip, tools, pieces, eligible)
    target = synth.DEMO_TOOL_OUTPUT.encode()
    g = ToolCallGrammar(tools, 4)
    states, points, undecided = [], [], []
    pos = 0
    while pos < len(target):
        allowed = masker.allowed(g, pos)
        undecided.append(masker.last_undecided)
        states.append(state_words(masker.program, g))
        points.append((g.clone(), pos))
        best = max((t for t in allowed if target.startswith(pieces[t], pos)),
                   key=lambda t: len(pieces[t]))
        g.feed(pieces[best])
        pos += len(pieces[best])
    width = max(s_.size for s_ in states)
    host = np.zeros((len(states), width), np.uint32)
    for i, s_ in enumerate(states):
        host[i, : s_.size] = s_
    dev_states = torch.from_numpy(host.view(np.int32)).cuda()
    words = (len(pieces) + 31) // 32
    allowed_d = torch.zeros(words, dtype=torch.int32, device="cuda")
    undecided_d = torch.zeros(words, dtype=torch.int32, device="cuda")
    # A stream of its own: torch's default stream has the null handle, which
    # the library reads as "the context's stream".
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()

    def run_all():
        for i in range(len(states)):
            hip._check(hip.lib.nd_grammar_mask_d(
                hip.ctx, masker._grammar, dev_states[i].data_ptr(), masker._pieces,
                65536 - points[i][1], allowed_d.data_ptr(), undecided_d.data_ptr(),
                C.c_void_p(stream.cuda_stream)))

    run_all()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(reps):
        run_all()
    stop.record(stream)
    torch.cuda.synchronize()
    kernel_ms = start.elapsed_time(stop) / (reps * len(states))
    t0 = time.perf_counter()
    for gg, p_ in points:
        masker.allowed(gg, p_)
    call_ms = (time.perf_counter() - t0) * 1e3 / len(points)
    # The resident loop's per-step host work: the mask into a model's mask
    # buffer (nd_needle_grammar_mask, a one-layer model of the same
    # vocabulary) and the undecided pieces settled; the selection then
    # reads the mask on the device.
    from needle_hip.needle2 import Needle2Geometry, Needle2Weights
    from needle_hip.runtime import Needle2Resident

    geo = Needle2Geometry(vocab=len(pieces), dim=128, heads=4, kv_heads=2, layers=1,
                          max_length=16, hadamard=256, engram_slots=64, sites=(0,),
                          kv_window=8)
    rt = Needle2Resident(hip, Needle2Weights(geo, 5))
    rt.reset(geo.max_length, 0)
    for gg, p_ in points[:4]:
        rt.grammar_mask(masker, masker.state(gg), 65536 - p_)
    t0 = time.perf_counter()
    for gg, p_ in points:
        _, und = rt.grammar_mask(masker, masker.state(gg), 65536 - p_)
        masker.settle(gg, und)
    resident_ms = (time.perf_counter() - t0) * 1e3 / len(points)
    rt.free()
    part = {"vocab": len(pieces), "states": len(states), "kernel_ms_per_mask": kernel_ms,
            "host_call_ms_per_mask": call_ms, "resident_call_ms_per_mask": resident_ms,
            "mean_undecided": float(np.mean(undecided)), "max_undecided": int(max(undecided))}
    cpu = None
    if cpu_seconds > 0:
        t0, n = time.perf_counter(), 0
        while n < len(points) and time.perf_counter() - t0 < cpu_seconds:
            gg, p_ = points[(n * 7) % len(points)]
            allowed_pieces(gg, pieces, eligible, p_)
            n += 1
        cpu_ms = (time.perf_counter() - t0) * 1e3 / max(1, n)
        cpu = {"value": cpu_ms, "unit": "ms/mask", "cores": 1, "kind": "port",
               "sample": f"{n} masks of the agent loop (grammar clone fed per piece) at states of "
                         f"the same output"}
        part["cpu_ms_per_mask"] = cpu_ms
        part["speedup_vs_cpu_loop"] = cpu_ms / call_ms
    masker.free()
    return part, cpu


def bench_attention(torch, hip, length, heads, steps, warmup, rotate=True):
    import ctypes as C

    from needle_hip import HipKvCache, synth

    per = attention_bytes(length, heads)
    replicas = max(1, math.ceil(ROTATE_BYTES / per)) if rotate else 1
    st = synth.Stream(7, f"bench-att{length}")
    K, V = st.normal((length, heads, 64)), st.normal((length, heads, 64))
    caches = []
    for _ in range(replicas):
        kv = HipKvCache(hip, 1, heads, max_length=length)
        kv.store(0, 0, K, V)
        caches.append(kv)
    q = torch.from_numpy(st.normal((heads * 64,))).cuda()
    out = torch.empty(heads * 64, dtype=torch.float32, device="cuda")

    def make(kv):
        return lambda stream: hip._check(hip.lib.nd_attention_d(
            hip.ctx, kv.handle, 0, length - 1, q.data_ptr(), heads, out.data_ptr(),
            C.c_void_p(stream)))

    timer = GraphTimer(torch, [make(caches[i % replicas]) for i in range(max(replicas, 32))])
    ms, timed = timer.time(math.ceil(steps / timer.n), warmup)
    for kv in caches:
        kv.free()
    gbs = per / (ms * 1e-3) / 1e9
    return {"bytes_per_call": per, "replicas": replicas, "calls": timed,
            "ms_per_call": ms, "GBps": gbs, "frac_hbm": gbs / HBM_PEAK_GBS}


def bench_attention_span(torch, hip, length, heads, steps, warmup):
    """The attention workload of bench_attention (same rotated replicas, same
    graph timing) through nd_attention_stamped_d: the same launch with each
    workgroup's thread 0 reading the 100 MHz clock at entry, after its
    wave's tiles, after the waves' combine, after publishing the chunk's
    partials, after counting in, and (the merging chunk) after the merge.
    Per launch of the last replay, relative to its earliest entry: medians
    over launches of the median and latest workgroup at each point, the
    latest arrival, the merge's end, and the interval to the next launch."""
    import ctypes as C

    import numpy as np

    from needle_hip import HipKvCache, synth

    per = attention_bytes(length, heads)
    replicas = max(1, math.ceil(ROTATE_BYTES / per))
    st = synth.Stream(7, f"bench-att{length}")
    K, V = st.normal((length, heads, 64)), st.normal((length, heads, 64))
    caches = []
    for _ in range(replicas):
        kv = HipKvCache(hip, 1, heads, max_length=length)
        kv.store(0, 0, K, V)
        caches.append(kv)
    q = torch.from_numpy(st.normal((heads * 64,))).cuda()
    out = torch.empty(heads * 64, dtype=torch.float32, device="cuda")
    launches = max(replicas, 32)
    cap = 4096
    stamps = torch.zeros((launches, cap, 8), dtype=torch.int64, device="cuda")
    wgs = C.c_uint32(0)

    def make(i):
        kv = caches[i % replicas]
        return lambda stream: hip._check(hip.lib.nd_attention_stamped_d(
            hip.ctx, kv.handle, 0, length - 1, q.data_ptr(), heads, out.data_ptr(),
            stamps[i].data_ptr(), cap, C.byref(wgs), C.c_void_p(stream)))

    timer = GraphTimer(torch, [make(i) for i in range(launches)])
    ms, _ = timer.time(math.ceil(steps / timer.n), warmup)
    a = stamps[:, :wgs.value, :].cpu().numpy()
    for kv in caches:
        kv.free()
    t0 = a[:, :, 0].min(axis=1)
    rel = (a[:, :, :6] - t0[:, None, None]) * 0.01  # microseconds after the launch's first entry
    merged = a[:, :, 6] == 1
    names = ["entry", "tiles_done", "combined", "published", "counted"]
    out_d = {"workgroups": wgs.value, "launches": int(launches), "events_ms_per_launch": ms}
    for i, nm in enumerate(names):
        out_d[f"{nm}_us_median_wg"] = float(np.median(np.median(rel[:, :, i], axis=1)))
        out_d[f"{nm}_us_last_wg"] = float(np.median(rel[:, :, i].max(axis=1)))
    merge_end = np.where(merged, rel[:, :, 5], 0).max(axis=1)
    out_d["merge_end_us"] = float(np.median(merge_end))
    out_d["merges_per_launch"] = float(np.median(merged.sum(axis=1)))
    # per merging chunk: its own arrival to its merge end
    gap = np.where(merged, rel[:, :, 5] - rel[:, :, 4], np.nan)
    out_d["merge_phase_us_median"] = float(np.nanmedian(gap))
    out_d["publish_phase_us_median"] = float(np.median(rel[:, :, 3] - rel[:, :, 2]))
    out_d["count_phase_us_median"] = float(np.median(rel[:, :, 4] - rel[:, :, 3]))
    out_d["combine_phase_us_median"] = float(np.median(rel[:, :, 2] - rel[:, :, 1]))
    out_d["tiles_phase_us_median"] = float(np.median(rel[:, :, 1] - rel[:, :, 0]))
    out_d["launch_interval_us_median"] = float(np.median(np.diff(t0) * 0.01))
    out_d["xcc_ok"] = bool(np.all(a[:, :, 7] == (np.arange(wgs.value) % 8)[None, :]))
    return out_d


def bench_needle2_span(torch, hip, steps, cq_bits=None):
    """Needle 2 at the shipped geometry (int8), batch 1, after a 128-token
    prompt: `steps` direct whole-step calls with the fused layer launches in
    their measurement form (nd_needle_test_stamps).  Per layer launch of the
    last step, microseconds after its first workgroup's entry: the Wo rows
    done, the mix's Wo wait over, the mix's signal to the projection, the
    projection done, the attention done, the launch's last exit; and the gap
    from that exit to the next launch's first entry; the projection and
    attention workgroups' phases (median and latest workgroup).  Medians
    over layers."""
    import numpy as np

    from needle_hip import NeedleModel, synth
    from needle_hip.needle2 import Needle2Geometry, Needle2Weights

    g = Needle2Geometry()
    model = NeedleModel(hip, Needle2Weights(g, 2026, cq_bits=cq_bits, cq_group=32)
                        if cq_bits else Needle2Weights(g, 2026))
    rt = model.create_resident_runtime()
    prompt = synth.Stream(2026, "needle2.prompt").integers(128, 0, g.vocab - 1)
    rt.reset(len(prompt) + steps + 1, 0)
    rt.prefill(prompt)
    cap = (g.layers + 1) * 64 * 16
    stamps = torch.zeros(cap, dtype=torch.int64, device="cuda")
    res = model.resident
    hip._check(hip.lib.nd_needle_test_stamps(hip.ctx, res.handle, stamps.data_ptr(), cap))
    tok = int(prompt[-1])
    for _ in range(steps):
        rt.step(tok, want_logits=False)
    torch.cuda.synchronize()
    a = stamps.view(g.layers + 1, 64, 16).cpu().numpy().astype(np.int64)
    hip._check(hip.lib.nd_needle_test_stamps(hip.ctx, res.handle, None, 0))
    model.dispose()
    # Wo workgroups: int8 16 rows each at d 512, Cactus-Quant 64 rows each
    W = g.dim // 64 if cq_bits else g.dim // (512 // (g.heads * 64 // 16))
    Q = 2 * (g.heads + g.kv_heads) + 1
    A = g.kv_heads
    rows = []
    for l in range(1, g.layers):
        e = a[l]
        act = e[: W + 1 + Q + A]
        t0 = act[:, 0].min()
        us = lambda v: float(v - t0) * 0.01
        mix = e[W]
        phases = {f"mix_{nm}": us(mix[i]) for i, nm in
                  ((4, "post_norms"), (5, "fwht1"), (6, "fwht2"), (7, "lanes"), (8, "pre_norm"),
                   (9, "phi"), (10, "engram"), (11, "input_norm"),
                   # int8 phi rows: split into LDS, MFMA done, wave partials
                   # met; Cactus-Quant: lanes in LDS, rotated, rows done
                   *(((12, "phi_staged"), (13, "phi_rotated"), (14, "phi_rows")) if cq_bits
                     else ((12, "phi_split"), (13, "phi_mfma"), (14, "phi_part"))))}
        rows.append({**phases, "wo_done": us(e[:W, 3].max()), "mix_entry": us(mix[0]),
                     "mix_wo_wait_done": us(mix[1]), "mix_signal": us(mix[2]),
                     "mix_exit": us(mix[3]), "qkv_done": us(e[W + 1: W + 1 + Q, 3].max()),
                     "att_done": us(e[W + 1 + Q: W + 1 + Q + A, 3].max()),
                     "launch_last_exit": us(act[:, 3].max()),
                     # the head projection workgroups (the routing one has no
                     # marks): wait over, input staged, rows computed, stores
                     # complete; the attention workgroups: wait over, q and
                     # gates issued, tile math done, waves combined, stored
                     **{f"qkv_{nm}_{fn.__name__}": us(fn(e[W + 1: W + Q, i])) for i, nm in
                        ((4, "wait_over"), (5, "staged"), (6, "rows"), (7, "stored"))
                        for fn in (np.median, np.max)},
                     # the Wo workgroups: int8 o in, weights in, stored;
                     # Cactus-Quant input staged, rows computed, stored
                     **{f"wo_{nm}_{fn.__name__}": us(fn(e[:W, i])) for i, nm in
                        ((0, "entry"), *(((4, "staged"), (5, "rows"), (6, "stored")) if cq_bits
                                         else ((4, "o_in"), (5, "w_in"), (6, "stored"))))
                        for fn in (np.median, np.max)},
                     **{f"att_{nm}_{fn.__name__}": us(fn(e[W + 1 + Q: W + 1 + Q + A, i]))
                        for i, nm in ((4, "wait_over"), (5, "issued"), (6, "tiles"), (7, "combined"),
                                      (8, "stored")) for fn in (np.median, np.max)},
                     "gap_to_next_us": float(a[l + 1][: W + 1 + Q + A, 0][
                         a[l + 1][: W + 1 + Q + A, 0] > 0].min() - act[:, 3].max()) * 0.01})
    out = {k: float(np.median([r[k] for r in rows])) for k in rows[0]}
    out["layers"] = len(rows)
    out["step_span_us"] = float(a[g.layers][:, 3].max() - a[0][a[0][:, 0] > 0][:, 0].min()) * 0.01
    return out


def decoder_weight_bytes(g):
    """int8 codes + f32 per-row scales read by one decode step (tied lm head)."""
    per_layer = [(g.heads + 2 * g.kv_heads) * 64 * g.dim, g.dim * g.heads * 64, g.ffn * g.dim,
                 g.dim * g.ffn]
    rows = [(g.heads + 2 * g.kv_heads) * 64, g.dim, g.ffn, g.dim]
    total = g.layers * (sum(per_layer) + 4 * sum(rows))
    return total + g.vocab * g.dim + 4 * g.vocab


def bench_constrained_decode(torch, hip, steps, warmup, check, threads, cpu_seconds):
    """Batched constrained greedy decode: 64 sequences, ragged contexts
    U{32..2048}, vocab 32768, ~2% allowed bitmask per sequence per step.
    Every step is one graph replay timed by its own pair of HIP events; the
    figure is the median step.  The CPU leg runs the whole workload (all 64
    sequences, every step) through the oracle on `threads` threads; it is
    also the greedy-identity check."""
    import numpy as np

    import oracle
    from needle_hip.models import (MASK_THRESHOLD24, PREFIX_SCALE, ConstrainedWorkload,
                                   DecoderGeometry, DecoderWeights, HipBatch, HipDecoder)

    steps = max(5, steps)
    g = DecoderGeometry()
    wl = ConstrainedWorkload(batch=64, steps=steps, min_context=32, max_context=2048,
                             vocab=g.vocab)
    weights = DecoderWeights(g, 2026)
    dec = HipDecoder(hip, weights)
    batch = HipBatch(dec, wl.batch, wl.max_length)
    lengths, starts = wl.lengths, wl.start_tokens
    for s in range(wl.batch):
        batch.fill_synthetic(s, *wl.kv_seeds(s), int(lengths[s]), wl.max_length)
    max_pos = int(lengths.max()) + steps - 1

    def launch(stream):
        batch.step(max_pos, mask_seed=wl.mask_seed, stream=stream)

    batch.set_state(starts, lengths, 0)
    timer = GraphTimer(torch, [launch])
    batch.set_state(starts, lengths, 0)
    for _ in range(warmup):
        timer.graph.replay()
    torch.cuda.synchronize()
    batch.set_state(starts, lengths, 0)
    ms_per_step, timed = timer.time(steps, 0)
    assert timed == steps
    ids, lps = batch.history(0, steps)
    tok_s = wl.batch / (ms_per_step * 1e-3)
    kv_tokens = float(np.sum(lengths.astype(np.float64) + (steps + 1) / 2.0))
    kv_bytes = kv_tokens * g.layers * g.kv_heads * (64 + 64 + 4 + 4)
    step_bytes = kv_bytes + decoder_weight_bytes(g) + wl.batch * ((g.vocab + 31) // 32) * 4
    gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
    part = {"sequences": wl.batch, "steps": steps, "ms_per_step": ms_per_step,
            "tokens_per_s": tok_s, "context_mean": float(lengths.mean()),
            "bytes_per_step": step_bytes, "GBps": gbs, "frac_hbm": gbs / HBM_PEAK_GBS}
    cpu = None
    if check or cpu_seconds > 0:
        ref = oracle.SynthDecoder(weights)
        caches = []
        for s in range(wl.batch):
            c = oracle.KvCache(g.layers, g.kv_heads, wl.max_length)
            oracle.kv_fill_synthetic(c, *wl.kv_seeds(s), int(lengths[s]), *PREFIX_SCALE)
            caches.append(c)
        t0 = time.perf_counter()
        want, want_lp = ref.decode_batch(caches, starts, lengths, steps, wl.mask_seed,
                                         MASK_THRESHOLD24, threads=threads)
        el = time.perf_counter() - t0
        cpu = {"value": wl.batch * steps / el, "unit": "tok/s", "cores": threads,
               "kind": "port",
               "sample": f"the whole workload: oracle decode of all {wl.batch} sequences x "
                         f"{steps} steps on {threads} threads ({el:.1f} s)"}
        part["cpu_tokens_per_s"] = cpu["value"]
        part["speedup_vs_cpu"] = tok_s / cpu["value"]
        part["greedy_identical"] = bool(np.array_equal(ids, want))
        part["greedy_mismatches"] = int(np.sum(ids != want))
        part["logprob_max_abs_err"] = float(np.max(np.abs(lps - want_lp)))
    batch.free()
    dec.free()
    return part, cpu


def bench_prefill(torch, hip, tokens_n, reps, check, threads):
    """Prefill of a 2048-token prompt through the synthetic 8-layer decoder:
    the median of `reps` graph replays of the whole pass, the kernel time by
    kind from one eager pass with an event after every kernel (int8 GEMM
    rate and attention rate each over its own time), and, as the CPU leg and
    the parity check, the oracle prefill (NeedleRuntime.prefill: 2048
    sequential steps' arithmetic, layer-major on `threads` threads) of the
    same prompt, whose last logits the device's are compared with."""
    import numpy as np

    import oracle
    from needle_hip import HipKvCache, synth
    from needle_hip.models import DecoderGeometry, DecoderWeights, HipDecoder, HipPrefill

    g = DecoderGeometry()
    weights = DecoderWeights(g, 2026)
    dec = HipDecoder(hip, weights)
    pre = HipPrefill(dec, tokens_n, tokens_n)
    cache = HipKvCache(hip, g.layers, g.kv_heads, max_length=tokens_n)
    tokens = synth.Stream(2026, "prefill-prompt").integers(tokens_n, 0, g.vocab - 1)
    pre.set_tokens(tokens, 0)
    timer = GraphTimer(torch, [lambda stream: pre.launch(cache, stream)])
    ms, timed = timer.time(reps, 1)
    logits = pre.logits()
    gemm_ms, attn_ms, other_ms = pre.phase_ms(cache)
    # Algorithmic int8 work: 2*M*N*K per projection (three digit planes are
    # executed; the figure counts the contraction once).  Attention: QK^T and
    # PV over the causal triangle, 4 flops per (query, key, dim).
    per_layer = 2 * tokens_n * g.dim * ((g.heads + 2 * g.kv_heads) * 64 + g.dim + 2 * g.ffn)
    gemm_ops = g.layers * per_layer + 2 * g.vocab * g.dim
    attn_flops = g.layers * g.heads * 4 * 64 * tokens_n * (tokens_n + 1) / 2
    part = {"tokens": tokens_n, "replays": timed, "ms": ms, "tokens_per_s": tokens_n / (ms * 1e-3),
            "gemm_int8_ops": gemm_ops, "attention_flops": attn_flops,
            "phase_ms": {"gemm": gemm_ms, "attention": attn_ms, "other": other_ms},
            "gemm_int8_TOPS": gemm_ops / (gemm_ms * 1e-3) / 1e12,
            "attention_TFLOPs": attn_flops / (attn_ms * 1e-3) / 1e12,
            "kv_bytes_written": g.layers * g.kv_heads * tokens_n * (64 * 2 + 8)}
    part["last_logit_argmax"] = int(np.argmax(logits))
    cpu = None
    if check:
        ref = oracle.SynthDecoder(weights)
        rc = ref.new_cache(tokens_n)
        t0 = time.perf_counter()
        want = ref.prefill(rc, tokens, 0, threads=threads)
        el = time.perf_counter() - t0
        cpu = {"value": tokens_n / el, "unit": "tok/s", "cores": threads, "kind": "port",
               "sample": f"the whole workload: oracle prefill of all {tokens_n} positions, "
                         f"layer-major on {threads} threads ({el:.1f} s)"}
        part["cpu_tokens_per_s"] = cpu["value"]
        err = float(np.max(np.abs(logits.astype(np.float64) - want)))
        part["logit_max_abs_err"] = err
        part["logit_max_abs"] = float(np.max(np.abs(want)))
        part["logit_err_over_scale"] = err / max(1e-30, part["logit_max_abs"])
        part["argmax_identical"] = int(np.argmax(want)) == part["last_logit_argmax"]
    pre.free()
    cache.free()
    dec.free()
    return part, cpu


def bench_read_ceiling(torch, hip, nbytes=1 << 30, blocks=(1024, 2048, 4096, 8192), reps=10):
    """The read-only streaming rate of nd_stream_read_d over `nbytes` (four
    times the Infinity Cache and more) at several workgroup counts: the
    matvec's load form with nothing else to do.  Median of `reps` launches
    per count, each bracketed by HIP events."""
    import ctypes as C

    src = torch.randint(0, 1 << 30, (nbytes // 4,), dtype=torch.int32, device="cuda")
    out = torch.empty(max(blocks), dtype=torch.int32, device="cuda")
    stream = torch.cuda.Stream()  # not the default stream: its handle is null
    torch.cuda.synchronize()
    best, per = 0.0, {}
    for nb in blocks:
        def launch():
            hip._check(hip.lib.nd_stream_read_d(hip.ctx, C.c_void_p(src.data_ptr()), nbytes, nb,
                                                C.c_void_p(out.data_ptr()),
                                                C.c_void_p(stream.cuda_stream)))
        launch()
        torch.cuda.synchronize()
        times = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            launch()
            b.record(stream)
            torch.cuda.synchronize()
            times.append(a.elapsed_time(b))
        ms = sorted(times)[len(times) // 2]
        gbs = nbytes / (ms * 1e-3) / 1e9
        per[str(nb)] = round(gbs, 1)
        best = max(best, gbs)
    del src
    return {"bytes": nbytes, "GBps_by_workgroups": per, "GBps": best, "frac_hbm": best / HBM_PEAK_GBS}


def bench_copy_ceiling(torch, bytes_moved, steps, warmup):
    """The runtime's own device copy moving the same number of bytes per
    launch (half read, half written) under the same rotation and graph
    timing: what one launch of this size reaches on this GPU."""
    half = bytes_moved // 2 // 4
    replicas = max(1, math.ceil(ROTATE_BYTES / (half * 4)))
    srcs = [torch.rand(half, device="cuda") for _ in range(replicas)]
    dst = torch.empty(half, device="cuda")

    def make(src):
        return lambda stream: dst.copy_(src)

    timer = GraphTimer(torch, [make(srcs[i % replicas]) for i in range(max(replicas, 32))])
    ms, _ = timer.time(math.ceil(steps / timer.n), warmup)
    gbs = half * 8 / (ms * 1e-3) / 1e9
    return {"bytes_per_launch": half * 8, "replicas": replicas, "ms_per_launch": ms,
            "GBps": gbs, "frac_hbm": gbs / HBM_PEAK_GBS}


def needle2_token_bytes(g, visible):
    """HBM bytes one Needle 2 token reads: int8 codes + f32 row scales of every
    matrix it multiplies, the engram rows it gathers and `visible` K/V rows
    (64 + 64 codes + two f32 scales) per layer and KV head."""
    qkvg = (2 * g.heads + 2 * g.kv_heads) * 64
    per_layer = (qkvg * (g.dim + 4) + g.dim * (g.heads * 64 + 4)
                 + (2 * g.lanes + g.lanes * g.lanes) * (g.lanes * g.dim + 4)
                 + visible * g.kv_heads * (64 * 2 + 8))
    cat = g.engram_tables * g.engram_sub
    engram = len(g.sites) * (2 * g.dim * (cat + 4) + g.engram_tables * (g.engram_sub + 4))
    return g.layers * per_layer + engram + g.vocab * (g.dim + 4)


def needle2_cq_token_bytes(g, visible, form):
    """HBM bytes one Needle 2 token reads with Cactus-Quant matrices, each in
    the (bits, group) that form(role, index) gives it: packed codes (bits per
    weight, ternary 2) + binary16 norms per group of every matrix it
    multiplies, the engram rows it gathers and `visible` K/V rows per layer
    and KV head."""

    def mat(n, k, role, index=0):
        bits, group = form(role, index)
        pb = 2 if bits == 5 else bits
        kpad = -(-k // group) * group
        return n * (kpad * pb // 8 + kpad // group * 2)

    total = 0
    hd, ln = 64, g.lanes
    for l in range(g.layers):
        total += (mat(g.heads * hd, g.dim, "wq", l) + mat(g.kv_heads * hd, g.dim, "wk", l)
                  + mat(g.kv_heads * hd, g.dim, "wv", l) + mat(g.heads * hd, g.dim, "wgate", l)
                  + mat(g.dim, g.heads * hd, "wo", l) + mat(ln, ln * g.dim, "phi_pre")
                  + mat(ln, ln * g.dim, "phi_post") + mat(ln * ln, ln * g.dim, "phi_res")
                  + visible * g.kv_heads * (64 * 2 + 8))
    cat = g.engram_tables * g.engram_sub
    for s in range(len(g.sites)):
        total += (mat(g.dim, cat, "eg_key", s) + mat(g.dim, cat, "eg_value", s)
                  + mat(g.engram_tables, g.engram_sub, "eg_tables", s))
    return total + mat(g.vocab, g.dim, "embedding")


def bench_needle2_cq(torch, hip, reps, bits=4, group=32):
    """The same generate (shipped geometry, 128-token prompt, 64 greedy
    tokens) with every matrix in the Cactus-Quant form of the shipped archive
    (CQ4, groups of 32; bits "mixed": each matrix in its own width and group,
    cact.mixed_form): products as cqMatvec, rows as dequantizeCqRow, the
    prompt as one batched pass (the CQ matvec over its 128 rows).  Timing
    only: the GPU tests hold its parity with the oracle."""
    import numpy as np

    from needle_hip import NeedleModel, synth
    from needle_hip.cact import mixed_form
    from needle_hip.needle2 import Needle2Geometry, Needle2Weights
    from needle_hip.runtime import EOS_TOKEN_ID

    g = Needle2Geometry()
    form = mixed_form if bits == "mixed" else (lambda role, index=0: (bits, group))
    model = NeedleModel(hip, Needle2Weights(g, 2026, cq_bits=bits, cq_group=group))
    prompt = synth.Stream(2026, "needle2.prompt").integers(128, 0, g.vocab - 1)
    new = 64
    model.generate_resident(prompt, new, eos=EOS_TOKEN_ID)
    model.generate_resident(prompt, 1, eos=EOS_TOKEN_ID)
    walls, walls1 = [], []
    res = None
    for _ in range(reps):
        t0 = time.perf_counter()
        res = model.generate_resident(prompt, new, eos=EOS_TOKEN_ID)
        walls.append(time.perf_counter() - t0)
        t0 = time.perf_counter()
        model.generate_resident(prompt, 1, eos=EOS_TOKEN_ID)
        walls1.append(time.perf_counter() - t0)
    wall, wall1 = float(np.median(walls)), float(np.median(walls1))
    n_gen = res.generated_tokens
    decode_ms = (wall - wall1) * 1e3 / max(1, n_gen - 1)
    bytes_tok = needle2_cq_token_bytes(g, min(g.kv_window, 128 + n_gen // 2), form)
    part = {"bits": bits, "group": group if bits != "mixed" else "mixed",
            "prompt_tokens": 128, "generated_tokens": n_gen,
            "reps": reps, "wall_ms": wall * 1e3, "tokens_per_s": n_gen / wall,
            "decode_ms_per_token": decode_ms, "decode_tokens_per_s": 1e3 / decode_ms,
            "prefill_128_ms": wall1 * 1e3, "prefill_tokens_per_s": 128 / wall1, "bytes_per_token": bytes_tok,
            "decode_GBps": bytes_tok / (decode_ms * 1e-3) / 1e9,
            "launches_per_token": model.resident.step_launches()}
    model.dispose()
    return part


def bench_needle2(torch, hip, reps, check, cpu_seconds):
    """Needle 2 at the shipped geometry (27 layers, vocab 8192, KV window
    256), batch 1: NeedleModel.generate of 64 greedy tokens from a 128-token
    prompt, tok/s as the reference reports it (generated tokens / wall time
    of the whole call, prefill included)."""
    import numpy as np

    import oracle
    from needle_hip import NeedleModel, synth
    from needle_hip.needle2 import Needle2Geometry, Needle2Weights
    from needle_hip.runtime import EOS_TOKEN_ID

    g = Needle2Geometry()
    weights = Needle2Weights(g, 2026)
    model = NeedleModel(hip, weights)
    prompt = synth.Stream(2026, "needle2.prompt").integers(128, 0, g.vocab - 1)
    new = 64
    model.generate_resident(prompt, new, eos=EOS_TOKEN_ID)  # captures the step graphs
    model.generate_resident(prompt, 1, eos=EOS_TOKEN_ID)
    walls, walls1 = [], []
    res = None
    for _ in range(reps):
        t0 = time.perf_counter()
        res = model.generate_resident(prompt, new, eos=EOS_TOKEN_ID)
        walls.append(time.perf_counter() - t0)
        t0 = time.perf_counter()
        model.generate_resident(prompt, 1, eos=EOS_TOKEN_ID)
        walls1.append(time.perf_counter() - t0)
    wall = float(np.median(walls))
    wall1 = float(np.median(walls1))
    n_gen = res.generated_tokens
    decode_ms = (wall - wall1) * 1e3 / max(1, n_gen - 1)
    prefill_ms = wall1 * 1e3
    visible = min(g.kv_window, 128 + n_gen // 2)
    bytes_tok = needle2_token_bytes(g, visible)
    part = {"prompt_tokens": 128, "generated_tokens": n_gen, "reps": reps,
            "wall_ms": wall * 1e3, "tokens_per_s": n_gen / wall,
            "decode_ms_per_token": decode_ms, "decode_tokens_per_s": 1e3 / decode_ms,
            "prefill_128_ms": prefill_ms, "prefill_tokens_per_s": 128 / wall1,
            "bytes_per_token": bytes_tok,
            "decode_GBps": bytes_tok / (decode_ms * 1e-3) / 1e9,
            # counted in the decode-step graph: begin, engram projections +
            # convolution, per layer one launch (the previous layer's Wo,
            # the mix, this layer's QKV and attention), the final mix (with
            # the last Wo), lm head and selection, and the confidence pool
            # (the head is on, as the reference's default)
            "launches_per_token": model.resident.step_launches(),
            "confidence_pool": model.resident.has_confidence}
    part["decode_frac_hbm"] = part["decode_GBps"] / HBM_PEAK_GBS
    # The same call through NeedleRuntime driving the session methods
    # (nd_needle_begin_token ... nd_needle_finish_token per step, a host round
    # trip per token), as a host of the reference's session contract runs it.
    model.generate(prompt, new, eos=EOS_TOKEN_ID)
    sess = []
    for _ in range(max(1, reps // 2)):
        r = model.generate(prompt, new, eos=EOS_TOKEN_ID)
        sess.append(r.elapsed_ms)
        part["session_greedy_identical_to_graph"] = r.token_ids == res.token_ids
    part["session_path_wall_ms"] = float(np.median(sess))
    part["session_path_tokens_per_s"] = n_gen / (part["session_path_wall_ms"] * 1e-3)
    cpu = None
    if check or cpu_seconds > 0:
        # The whole generate call on the oracle, one thread: 128 prompt steps
        # and the decode steps, timed together.
        ref = oracle.Needle2(weights)
        t0 = time.perf_counter()
        rt = ref.runtime(128 + new, 0)
        for t in prompt[:-1]:
            rt.step(int(t), want_logits=False)
        logits = rt.step(int(prompt[-1]))
        ids = []
        for k in range(new):
            tok = oracle.argmax(logits)
            if tok == EOS_TOKEN_ID:
                break
            ids.append(tok)
            if k + 1 < new:
                logits = rt.step(tok)
        el = time.perf_counter() - t0
        cpu = {"value": len(ids) / el, "unit": "tok/s", "cores": 1, "kind": "port",
               "sample": f"the whole generate call: oracle NeedleRuntime steps over the "
                         f"128-token prompt and {len(ids)} generated tokens, one thread "
                         f"({el:.1f} s)"}
        part["cpu_tokens_per_s"] = cpu["value"]
        part["speedup_vs_cpu"] = part["tokens_per_s"] / cpu["value"]
        part["greedy_identical"] = ids == res.token_ids
    model.dispose()
    return part, cpu


def traffic_workload(torch, hip, n, k, g, launches=64):
    """The launches a pair of rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE)
    measure: a 256 MiB device-to-device tensor copy (known bytes, to scale
    the counters) and `launches` batch-1 matvecs over rotated HBM replicas."""
    import ctypes as C

    from needle_hip import lib as L
    from needle_hip import synth

    src = torch.rand(64 << 20, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    per = matvec_bytes(n, k, g, 1)
    replicas = max(1, math.ceil(ROTATE_BYTES / per))
    w, sc = synth.int8_matrix(2026, f"bench-w{n}x{k}", n, k, g)
    mats = []
    for _ in range(replicas):
        h = C.c_void_p()
        hip._check(hip.lib.nd_mat_upload_i8(hip.ctx, L.ptr(w), L.ptr(sc), n, k, g, C.byref(h)))
        mats.append(h)
    x = torch.from_numpy(synth.Stream(2026, "bench-x").normal((1, k))).cuda()
    y = torch.empty((1, n), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    for i in range(launches):
        hip._check(hip.lib.nd_matvec_d(hip.ctx, mats[i % replicas], x.data_ptr(), 1, 0, n,
                                        y.data_ptr(), C.c_void_p(stream)))
    torch.cuda.synchronize()
    for h in mats:
        hip.lib.nd_mat_free(hip.ctx, h)
    return {"copy_bytes_each_way": src.numel() * 4, "copies": 4, "matvec_launches": launches,
            "matvec_bytes_per_launch": per}


def attention_traffic_workload(torch, hip, length=8192, heads=8, launches=64):
    """The launches a pair of rocprofv3 --pmc passes measure for the
    single-query attention: a 256 MiB device-to-device tensor copy (known
    bytes, to scale the counters) and `launches` attention calls over rotated
    HBM replicas of an 8-head cache of `length` positions."""
    import ctypes as C

    from needle_hip import HipKvCache, synth

    src = torch.rand(64 << 20, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    per = attention_bytes(length, heads)
    replicas = max(1, math.ceil(ROTATE_BYTES / per))
    st = synth.Stream(7, f"bench-att{length}")
    K, V = st.normal((length, heads, 64)), st.normal((length, heads, 64))
    caches = []
    for _ in range(replicas):
        kv = HipKvCache(hip, 1, heads, max_length=length)
        kv.store(0, 0, K, V)
        caches.append(kv)
    q = torch.from_numpy(st.normal((heads * 64,))).cuda()
    out = torch.empty(heads * 64, dtype=torch.float32, device="cuda")
    stream = torch.cuda.Stream()  # not the default stream: its handle is null
    torch.cuda.synchronize()
    for i in range(launches):
        hip._check(hip.lib.nd_attention_d(hip.ctx, caches[i % replicas].handle, 0, length - 1,
                                          q.data_ptr(), heads, out.data_ptr(),
                                          C.c_void_p(stream.cuda_stream)))
    torch.cuda.synchronize()
    for kv in caches:
        kv.free()
    return {"copy_bytes_each_way": 256 << 20, "copies": 4, "attention_launches": launches,
            "attention_bytes_per_call": per}


def measured_traffic():
    """HBM bytes per matvec launch from the committed rocprofv3 --pmc summary
    (profiles/matvec_i8_4096x4096_g32_b1_traffic.md, line 'traffic_bytes_per_launch: N'),
    or None when it is absent."""
    path = ROOT / "profiles" / "matvec_i8_4096x4096_g32_b1_traffic.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1].strip())
    return None


def cpu_baseline_matvec(n, k, g, seconds):
    """The oracle (one thread) on the same matvec workload, timed on this host."""
    import numpy as np

    import oracle
    from needle_hip import synth

    w, s = synth.int8_matrix(2026, f"bench-w{n}x{k}", n, k, g)
    x = synth.Stream(2026, "bench-x").normal((1, k))
    oracle.matvec_i8(w, s, g, x)  # warm
    calls = 0
    t0 = time.perf_counter()
    while True:
        oracle.matvec_i8(w, s, g, x)
        calls += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    per = matvec_bytes(n, k, g, 1)
    return {"value": per * calls / el / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{calls} calls of the oracle int8 matvec N={n} K={k} G={g} batch 1 "
                      f"({el:.1f} s, host has {os.cpu_count()} cores)"}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3200,
                    help="timed matvec launches (at least; >= 5 graph replays, median reported)")
    ap.add_argument("--warmup", type=int, default=3, help="untimed graph replays")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="length of the matvec CPU sample (the model legs run whole)")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-decode", action="store_true")
    ap.add_argument("--skip-prefill", action="store_true")
    ap.add_argument("--skip-needle2", action="store_true")
    ap.add_argument("--needle2-reps", type=int, default=5)
    ap.add_argument("--only", choices=["matvec", "matvec8", "attention", "decode", "prefill",
                                       "needle2", "needle2cq", "needle2mixed", "traffic", "attention_traffic", "cq",
                                       "grammar", "ceiling", "matvec_span", "copy_matvec",
                                       "attention_span", "needle2_span", "needle2_span_cq4"],
                    help="run one part alone and print its JSON (for profiling)")
    ap.add_argument("--decode-steps", type=int, default=128)
    ap.add_argument("--no-check", action="store_true",
                    help="skip the full-size greedy identity check against the oracle")
    ap.add_argument("--check-threads", type=int, default=min(16, os.cpu_count() or 1))
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the multi-GPU "
              "design is documented but not built.", file=sys.stderr)
        sys.exit(2)

    import torch

    from needle_hip import HipBackend

    hip = HipBackend(device=0)
    n = k = 4096
    g = 32
    if args.only:
        if args.only == "matvec":
            part = bench_matvec(torch, hip, n, k, g, 1, args.steps, args.warmup)
        elif args.only == "matvec8":
            part = bench_matvec(torch, hip, n, k, g, 8, args.steps, args.warmup)
        elif args.only == "attention":
            part = bench_attention(torch, hip, 8192, 8, args.steps // 2, args.warmup)
        elif args.only == "decode":
            part, _ = bench_constrained_decode(torch, hip, args.decode_steps, 2, False, 1, 0)
        elif args.only == "needle2":
            part, _ = bench_needle2(torch, hip, args.needle2_reps, False, 0)
        elif args.only == "needle2cq":
            part = bench_needle2_cq(torch, hip, args.needle2_reps)
        elif args.only == "needle2mixed":
            part = bench_needle2_cq(torch, hip, args.needle2_reps, bits="mixed")
        elif args.only == "ceiling":
            part = bench_read_ceiling(torch, hip)
        elif args.only == "traffic":
            part = traffic_workload(torch, hip, n, k, g)
        elif args.only == "attention_traffic":
            part = attention_traffic_workload(torch, hip)
        elif args.only == "matvec_span":
            part = bench_matvec_span(torch, hip, n, k, g, args.steps, args.warmup)
        elif args.only == "needle2_span":
            part = bench_needle2_span(torch, hip, 8)
        elif args.only == "needle2_span_cq4":
            part = bench_needle2_span(torch, hip, 8, cq_bits=4)
        elif args.only == "attention_span":
            part = bench_attention_span(torch, hip, 8192, 8, args.steps, args.warmup)
        elif args.only == "copy_matvec":
            part = bench_copy_ceiling(torch, matvec_bytes(n, k, g, 1), args.steps, args.warmup)
        elif args.only == "grammar":
            part, _ = bench_grammar_mask(torch, hip, 20, 0 if args.skip_cpu else args.cpu_seconds)
        elif args.only == "cq":
            part = {f"cq{bits}_matvec_b1_hbm": bench_cq_matvec(torch, hip, n, k, g, bits, 1,
                                                                 args.steps, args.warmup)
                    for bits in (2, 3, 4, 5)}
        else:
            part, _ = bench_prefill(torch, hip, 2048, 5, False, 1)
        print(json.dumps({args.only: part}))
        return
    main_mv = bench_matvec(torch, hip, n, k, g, 1, args.steps, args.warmup)
    print(f"[bench] matvec b1 HBM {main_mv['GBps']:.0f} GB/s "
          f"{main_mv['ms_per_launch'] * 1e3:.2f} us/launch", file=sys.stderr, flush=True)
    parts = {"matvec_b1_hbm": main_mv}
    parts["matvec_b8_hbm"] = bench_matvec(torch, hip, n, k, g, 8, args.steps, args.warmup)
    parts["matvec_b1_mall"] = bench_matvec(torch, hip, n, k, g, 1, args.steps, args.warmup,
                                           rotate=False)
    print(f"[bench] matvec b8 {parts['matvec_b8_hbm']['GBps']:.0f} GB/s, b1 MALL "
          f"{parts['matvec_b1_mall']['GBps']:.0f} GB/s", file=sys.stderr, flush=True)
    for bits in (2, 3, 4, 5):
        part = bench_cq_matvec(torch, hip, n, k, g, bits, 1, args.steps, args.warmup)
        parts[f"cq{bits}_matvec_b1_hbm"] = part
        print(f"[bench] CQ{bits if bits < 5 else ' ternary'} matvec b1 {part['GBps']:.0f} GB/s "
              f"{part['ms_per_call'] * 1e3:.2f} us/call", file=sys.stderr, flush=True)
    for length in (512, 2048, 8192):
        parts[f"attention_L{length}_hbm"] = bench_attention(torch, hip, length, 8,
                                                            args.steps // 2, args.warmup)
        print(f"[bench] attention L={length} "
              f"{parts[f'attention_L{length}_hbm']['GBps']:.0f} GB/s", file=sys.stderr, flush=True)
    parts["attention_L8192_mall"] = bench_attention(torch, hip, 8192, 8, args.steps // 2,
                                                    args.warmup, rotate=False)
    parts["read_ceiling_1GiB"] = bench_read_ceiling(torch, hip)
    print(f"[bench] read-only stream ceiling {parts['read_ceiling_1GiB']['GBps']:.0f} GB/s",
          file=sys.stderr, flush=True)
    for name, nbytes in (("copy_ceiling_matvec_bytes", main_mv["bytes_per_launch"]),
                         ("copy_ceiling_attention_L8192_bytes",
                          parts["attention_L8192_hbm"]["bytes_per_call"])):
        parts[name] = bench_copy_ceiling(torch, nbytes, args.steps, args.warmup)
        print(f"[bench] {name}: {parts[name]['GBps']:.0f} GB/s "
              f"({parts[name]['ms_per_launch'] * 1e3:.2f} us)", file=sys.stderr, flush=True)
    if not args.skip_decode:
        part, cpu_dec = bench_constrained_decode(
            torch, hip, args.decode_steps, 2, not args.no_check, args.check_threads,
            0 if args.skip_cpu else args.cpu_seconds)
        parts["constrained_decode_b64"] = part
        if cpu_dec:
            parts["constrained_decode_b64"]["cpu_baseline"] = cpu_dec
        print(f"[bench] constrained decode b64 {part['tokens_per_s']:.0f} tok/s "
              f"{part['ms_per_step']:.3f} ms/step greedy_identical="
              f"{part.get('greedy_identical')}", file=sys.stderr, flush=True)

    if not args.skip_prefill:
        part, cpu_pre = bench_prefill(torch, hip, 2048, 5, not (args.no_check and args.skip_cpu),
                                      args.check_threads)
        if cpu_pre:
            part["cpu_baseline"] = cpu_pre
        parts["prefill_2048"] = part
        print(f"[bench] prefill 2048 {part['ms']:.2f} ms {part['tokens_per_s']:.0f} tok/s, GEMM "
              f"{part['gemm_int8_TOPS']:.1f} int8 TOPS, attention {part['attention_TFLOPs']:.1f} "
              f"TFLOP/s, logit err {part.get('logit_max_abs_err')}", file=sys.stderr, flush=True)

    if not args.skip_needle2:
        part, cpu_n2 = bench_needle2(torch, hip, args.needle2_reps, not args.no_check,
                                     0 if args.skip_cpu else args.cpu_seconds)
        if cpu_n2:
            part["cpu_baseline"] = cpu_n2
        parts["needle2_generate_b1"] = part
        print(f"[bench] needle2 generate b1 {part['tokens_per_s']:.0f} tok/s, decode "
              f"{part['decode_ms_per_token']:.3f} ms/token, greedy_identical="
              f"{part.get('greedy_identical')}", file=sys.stderr, flush=True)
        part = bench_needle2_cq(torch, hip, args.needle2_reps)
        parts["needle2_cq4_generate_b1"] = part
        print(f"[bench] needle2 cq4 generate b1 {part['tokens_per_s']:.0f} tok/s, decode "
              f"{part['decode_ms_per_token']:.3f} ms/token", file=sys.stderr, flush=True)
        part = bench_needle2_cq(torch, hip, args.needle2_reps, bits="mixed")
        parts["needle2_cq_mixed_generate_b1"] = part
        print(f"[bench] needle2 mixed-width generate b1 {part['tokens_per_s']:.0f} tok/s, decode "
              f"{part['decode_ms_per_token']:.3f} ms/token", file=sys.stderr, flush=True)

    part, cpu_gm = bench_grammar_mask(torch, hip, 20, 0 if args.skip_cpu else 5.0)
    if cpu_gm:
        part["cpu_baseline"] = cpu_gm
    parts["grammar_mask_v8192"] = part
    print(f"[bench] grammar mask: kernel {part['kernel_ms_per_mask'] * 1e3:.1f} us/mask, host call "
          f"{part['host_call_ms_per_mask']:.2f} ms/mask (resident "
          f"{part['resident_call_ms_per_mask']:.3f}), undecided mean "
          f"{part['mean_undecided']:.2f}, agent loop "
          f"{part.get('cpu_ms_per_mask', float('nan')):.1f} ms/mask", file=sys.stderr, flush=True)

    cpu = None
    if not args.skip_cpu:
        cpu = cpu_baseline_matvec(n, k, g, args.cpu_seconds)

    ms = main_mv["ms_per_launch"]
    line = {
        "metric": "decode tok/s (batch 1 & 64) + int8 matvec/attn GB/s as % of HBM peak",
        "value": round(main_mv["GBps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": main_mv["launches"],
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "vs_baseline": None,
        "dtype": "int8xf32",
        "data": "synthetic",
        "config": {"workload": "int8 matvec N=4096 K=4096 G=32 batch 1 (fp32 scales, fp32 x/y)",
                   "rotation_replicas": main_mv["replicas"]},
        "roofline": {"bound": "hbm", "achieved": round(main_mv["GBps"], 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(main_mv["frac_hbm"], 4),
                     "traffic": measured_traffic(),
                     "kernel": "matvec_i8_kernel<B=1,SPT=1,RACC=8>",
                     "bytes_per_launch": main_mv["bytes_per_launch"]},
        "cpu_baseline": cpu,
        "parts": parts,
    }
    hip.dispose()
    print(json.dumps(line))


if __name__ == "__main__":
    main()
