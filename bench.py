"""Benchmark of the W8A16 linear on one MI355X.

Headline (`value`): decode GB/s on BASELINE config 1 -- a Qwen3-8B decoder
layer's seven W8A16 projections (q, k, v, o, gate, up, down) at batch
M in {1, 4, 16}.  One step computes all 21 projection outputs (7 x 3 batch
sizes) the way a decoder layer issues them: per batch size, q/k/v in one
`linear_multi` launch (they share the input, like the reference's fused QKV
W8A16 kernel), o, gate/up in one `linear_multi` launch, then down -- 12
launches.  The same step as 21 single-projection launches is reported as
`config.per_op_GBps`.
Each batch size's pass reads a different copy of the layer's weights (4
copies, 772 MB, rotated so the 256 MB Infinity Cache never serves a repeat).
Inputs are synthetic (weights N(0, 0.02) quantized per channel, activations
N(0, 1)) and resident in HBM before the timed region.

value = algorithmic bytes of the timed steps / their wall time, with bytes
per launch B = N*K + 2N + 2MK + 2MN (int8 weights, fp16 scales, fp16
activations and outputs).  HIP events on the launch stream bracket the timed
steps (preceded and followed by a device synchronize).  The steps are
launched eagerly through the torch op.

Graph replay: the same fused step captured GRAPH_STEPS at a time in one HIP
graph and replayed (`config.graph_replay`), as a serving loop would run it;
under a kernel tracer its dispatches run back to back.

Distribution: a second pass of DIST_REPS steps records an event after every
step; `stats` gives the median, p10 and p90 of the per-step rates (decode and
prefill).  Per-launch rows (configs 0, 2, 4 and each projection) replay HIP
graphs of back-to-back launches on rotating weight copies, i.e. GPU time per
launch, averaged over at least 50 launches.

The same JSON line carries
  * roofline      -- the decode GEMV kernel (every launch in the timed
                     region): algorithmic bytes per launch / average launch
                     duration (timed region / launches, 12 per step) against the 8 TB/s
                     HBM peak; `traffic` is the measured HBM bytes per launch
                     from profiles/gemv_decode_traffic.json when present;
  * prefill       -- BASELINE config 3 (Qwen3-8B MLP prefill, M=2048) in
                     TFLOP/s against the 2.5166 PFLOP/s dense FP16 MFMA peak:
                     gate/up in one launch, then down, on four rotated layer
                     copies (604 MB), timed after >= 0.25 s of the same steps
                     (the clock's sustained-load level);
  * other_configs -- per-launch timings of configs 0, 2 and 4 with their
                     roofline fraction and the kernel configuration the
                     planner ran (rf_w8a16_plan), and W4A16 rows;
  * read_envelope -- the same 12-launch step with a plain streaming read of
                     the same bytes in place of the GEMV (lib/librf_bench.so):
                     the bound the launch structure itself puts on `value`,
                     also per batch size;
  * cpu_baseline  -- the reference's CPU path (fp16 dequantize, then torch's
                     CPU F.linear, adapters/qwen3.py:617-623) timed on the
                     host cores: config 1 at M=1 (B/t), a 128-row sample of
                     config 3 (F/t), and config 2's 1000 rows once, whose
                     greedy tokens are compared with the GPU's fused argmax
                     (`cfg2_argmax_agreement`).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2516.6
METRIC = "W8A16 linear: decode GB/s (% HBM peak) + prefill TFLOP/s (% MFMA peak)"

QWEN3_8B = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
            ("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288)]
QWEN3_VL_32B = [("q", 8192, 5120), ("k", 1024, 5120), ("v", 1024, 5120), ("o", 5120, 8192),
                ("gate", 25600, 5120), ("up", 25600, 5120), ("down", 5120, 25600)]
DECODE_M = (1, 4, 16)
LAYER_COPIES = 4
# The decode step's launches per M: projections sharing the input run as one launch.
DECODE_GROUPS = ((0, 1, 2), (3,), (4, 5), (6,))
PREFILL = [("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288)]
PREFILL_M = 2048
PREFILL_COPIES = 4          # 4 x 151 MB: past the 256 MB Infinity Cache
PREFILL_SETTLE_S = 0.25
CFG0_COPIES = 192           # 192 x 3.1 MB = 605 MB
LM_HEAD = (151936, 5120)
ARGMAX_ROWS = 1000
DIST_REPS = 60
GRAPH_STEPS = 16            # decode steps per HIP graph (a multiple of the 4-copy rotation)
GRAPH_REPLAYS = 3


def nbytes(m, n, k, bias=False):
    return n * k + 2 * n + 2 * m * k + 2 * m * n + (2 * n if bias else 0)


def group_bytes(m, idxs, specs=QWEN3_8B):
    """Algorithmic bytes of one launch over projections idxs sharing x: x read once."""
    k = specs[idxs[0]][2]
    return sum(nbytes(m, specs[i][1], k) - 2 * m * k for i in idxs) + 2 * m * k


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_layer(torch, rf, specs, seed, keep_rowmajor=False):
    """Quantized + packed weights of one layer, generated on the device:
    (name, n, k, packed, scale) per projection (+ the row-major q on request)."""
    layer = []
    for i, (name, n, k) in enumerate(specs):
        g = torch.Generator(device="cuda").manual_seed(seed * 100 + i)
        w = torch.randn(n, k, generator=g, device="cuda", dtype=torch.float32) * 0.02
        q, s = rf.quantize_linear_per_channel(w)
        del w
        entry = (name, n, k, rf.pack_weight(q), s)
        layer.append(entry + (q,) if keep_rowmajor else entry)
        del q
    return layer


class Timer:
    """HIP events on the launch stream around a region, device-synchronized on both sides."""

    def __init__(self, torch):
        self.torch = torch
        self.stream = torch.cuda.current_stream()

    def __enter__(self):
        self.torch.cuda.synchronize()
        self.a = self.torch.cuda.Event(enable_timing=True)
        self.b = self.torch.cuda.Event(enable_timing=True)
        self.a.record(self.stream)
        return self

    def __exit__(self, *exc):
        self.b.record(self.stream)
        self.b.synchronize()
        self.torch.cuda.synchronize()
        self.ms = self.a.elapsed_time(self.b)


def step_times(torch, step, n, start=0):
    """Per-step durations (ms) of n back-to-back steps: an event on the launch
    stream after every step (device-synchronized before and after)."""
    stream = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    torch.cuda.synchronize()
    ev[0].record(stream)
    for i in range(n):
        step(start + i)
        ev[i + 1].record(stream)
    ev[-1].synchronize()
    torch.cuda.synchronize()
    return [ev[i].elapsed_time(ev[i + 1]) for i in range(n)]


def rate_stats(ms, work, scale):
    """Median / p10 / p90 of per-step rates work / t (work per step, scaled to
    the unit by `scale`), and the per-step times they come from."""
    import numpy as np
    rates = np.asarray([work / (t * 1e-3) / scale for t in ms])
    t = np.asarray(ms)
    return {"reps": len(ms), "median": round(float(np.median(rates)), 1),
            "p10": round(float(np.percentile(rates, 10)), 1),
            "p90": round(float(np.percentile(rates, 90)), 1),
            "median_ms_per_step": round(float(np.median(t)), 4)}


def capture(torch, fn):
    """HIP graph of fn()'s launches.  fn runs once eagerly on the capture stream
    first, so any workspace it needs exists before capture."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        fn()
    torch.cuda.synchronize()
    return g


def per_launch_us(torch, fn, copies, reps, graph=True, replays=3):
    """Average duration of back-to-back launches of fn(copy), rotating copies;
    replayed from a HIP graph unless graph=False."""
    def run():
        for i in range(reps):
            fn(copies[i % len(copies)])
    if not graph:
        run()
        with Timer(torch) as t:
            run()
        return t.ms * 1e3 / reps
    g = capture(torch, run)
    g.replay()
    with Timer(torch) as t:
        for _ in range(replays):
            g.replay()
    return t.ms * 1e3 / (replays * reps)


def plan_name(m, ns, k, fmt=0):
    from rhinoforge_amd import capi
    return capi.plan(m, ns, k, fmt=fmt)["name"]


def bench_decode(torch, rf, steps, warmup):
    layers = [make_layer(torch, rf, QWEN3_8B, seed=c) for c in range(LAYER_COPIES)]
    xs = {m: torch.randn(m, 12288, device="cuda").half() for m in DECODE_M}
    outs = {(m, n): torch.empty(m, n, device="cuda", dtype=torch.float16)
            for m in DECODE_M for _, n, _ in QWEN3_8B}

    def step(i):
        for j, m in enumerate(DECODE_M):
            layer = layers[(i * len(DECODE_M) + j) % LAYER_COPIES]
            x = xs[m]
            for name, n, k, wp, s in layer:
                rf.linear_into(x[:, :k], wp, s, None, outs[(m, n)])

    for i in range(warmup):
        step(i)
    with Timer(torch) as t:
        for i in range(steps):
            step(warmup + i)
    launches = steps * len(DECODE_M) * len(QWEN3_8B)
    step_bytes = sum(nbytes(m, n, k) for m in DECODE_M for _, n, k in QWEN3_8B)

    # The step with the projections that share an input fused into one launch
    # each (q/k/v and gate/up; o and down stay single): 4 launches per M.
    def launches_of(layer, m):
        x = xs[m][:, :4096]
        q, k_, v, o, gate, up, down = layer
        rf.linear_multi(x, [q[3], k_[3], v[3]], [q[4], k_[4], v[4]])
        rf.linear_into(x, o[3], o[4], None, outs[(m, 4096)])
        rf.linear_multi(x, [gate[3], up[3]], [gate[4], up[4]])
        rf.linear_into(xs[m][:, :12288], down[3], down[4], None, outs[(m, 4096)])

    def step_fused(i):
        for j, m in enumerate(DECODE_M):
            launches_of(layers[(i * len(DECODE_M) + j) % LAYER_COPIES], m)

    for i in range(warmup):
        step_fused(i)
    with Timer(torch) as tf:
        for i in range(steps):
            step_fused(warmup + i)
    fused_launches = steps * len(DECODE_M) * len(DECODE_GROUPS)
    fused_bytes = sum(group_bytes(m, g) for m in DECODE_M for g in DECODE_GROUPS)

    dist = step_times(torch, step_fused, DIST_REPS, warmup + steps)

    # The fused step per batch size (its 4 launches, same rotation), so the
    # headline can be read per M against the read envelope's per-M rate.
    per_m_fused = {}
    for m in DECODE_M:
        def step_m(i, m=m):
            launches_of(layers[i % LAYER_COPIES], m)
        for i in range(warmup):
            step_m(i)
        with Timer(torch) as tm:
            for i in range(steps):
                step_m(i)
        b = sum(group_bytes(m, g) for g in DECODE_GROUPS)
        per_m_fused[str(m)] = round(b * steps / (tm.ms * 1e-3) / 1e9, 1)

    rows = []
    for m in DECODE_M:
        for idx, (name, n, k) in enumerate(QWEN3_8B):
            copies = [layer[idx] for layer in layers]
            x, out = xs[m][:, :k], outs[(m, n)]
            us = per_launch_us(torch, lambda c: rf.linear_into(x, c[3], c[4], None, out),
                               copies, 40)
            rows.append({"M": m, "proj": name, "N": n, "K": k, "us": round(us, 2),
                         "GBps": round(nbytes(m, n, k) / (us * 1e-6) / 1e9, 1),
                         "plan": plan_name(m, n, k)})
    for m in DECODE_M:
        x = xs[m][:, :4096]
        for name, idxs in (("qkv", (0, 1, 2)), ("gate_up", (4, 5))):
            copies = [[layer[i] for i in idxs] for layer in layers]
            us = per_launch_us(torch, lambda c: rf.linear_multi(x, [p[3] for p in c],
                                                                [p[4] for p in c]), copies, 40)
            ns = [QWEN3_8B[i][1] for i in idxs]
            rows.append({"M": m, "proj": name, "N": sum(ns), "K": 4096, "us": round(us, 2),
                         "GBps": round(group_bytes(m, idxs) / (us * 1e-6) / 1e9, 1),
                         "plan": plan_name(m, ns, 4096) + " (one launch)"})
    per_m_per_op = {}
    for m in DECODE_M:
        sel = [r for r in rows if r["M"] == m and r["proj"] in dict((p, 1) for p, _, _ in QWEN3_8B)]
        per_m_per_op[str(m)] = round(sum(nbytes(m, r["N"], r["K"]) for r in sel)
                                     / sum(r["us"] * 1e-6 for r in sel) / 1e9, 1)
    # The same step replayed from one HIP graph of GRAPH_STEPS steps (last:
    # eager launches after graph replays measured slower in the same process): the
    # launches a serving loop would capture once and replay.  Under a kernel
    # tracer these dispatches run back to back (eager ones are traced one at a
    # time), so their trace bounds the step without per-dispatch isolation.
    def run_graph():
        for i in range(GRAPH_STEPS):
            step_fused(i)
    g = capture(torch, run_graph)
    g.replay()
    with Timer(torch) as tg:
        for _ in range(GRAPH_REPLAYS):
            g.replay()
    del g
    graph_steps = GRAPH_STEPS * GRAPH_REPLAYS

    del layers
    torch.cuda.empty_cache()
    return {
        "GBps": fused_bytes * steps / (tf.ms * 1e-3) / 1e9,
        "ms_per_step": tf.ms / steps,
        "launches": fused_launches,
        "avg_launch_us": tf.ms * 1e3 / fused_launches,
        "avg_bytes_per_launch": fused_bytes / (len(DECODE_M) * len(DECODE_GROUPS)),
        "dist": rate_stats(dist, fused_bytes, 1e9),
        "graph": {"GBps": round(fused_bytes * graph_steps / (tg.ms * 1e-3) / 1e9, 1),
                  "ms_per_step": round(tg.ms / graph_steps, 4),
                  "steps_per_graph": GRAPH_STEPS, "replays": GRAPH_REPLAYS},
        "per_M_fused_GBps": per_m_fused,
        "per_op_GBps": step_bytes * steps / (t.ms * 1e-3) / 1e9,
        "per_op_ms_per_step": t.ms / steps,
        "per_op_avg_launch_us": t.ms * 1e3 / launches,
        "per_M_per_op_GBps": per_m_per_op,
        "per_launch": rows,
    }


def read_envelope(torch, steps, warmup):
    """The decode step's launch structure with the GEMV replaced by a plain
    streaming read (lib/librf_bench.so): 12 launches per step reading the
    same algorithmic byte counts, rotated over LAYER_COPIES buffer sets, eager
    on one stream and timed like the GEMV step (also per batch size).  Launch
    gaps, ramp-up and drain bound the decode step no matter what kernel runs;
    this is that bound on the device at hand."""
    import ctypes
    path = os.path.join(ROOT, "rhinoforge_amd", "lib", "librf_bench.so")
    if not os.path.isfile(path):
        log(f"read envelope skipped: {path} not built")
        return None
    lib = ctypes.CDLL(path)
    lib.rf_bench_stream_read.restype = ctypes.c_int
    lib.rf_bench_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                         ctypes.c_void_p]
    sizes = {m: [(group_bytes(m, g) + 15) // 16 * 16 for g in DECODE_GROUPS] for m in DECODE_M}
    bufs = [{m: [torch.empty(b, dtype=torch.uint8, device="cuda") for b in sizes[m]]
             for m in DECODE_M} for _ in range(LAYER_COPIES)]
    for c in bufs:
        for m in DECODE_M:
            for t in c[m]:
                t.fill_(1)
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream

    def read_m(copy, m):
        for b, buf in zip(sizes[m], copy[m]):
            st = lib.rf_bench_stream_read(buf.data_ptr(), b, sink.data_ptr(), stream)
            if st != 0:
                raise RuntimeError(f"rf_bench_stream_read: hipError {st}")

    def step(i):
        for j, m in enumerate(DECODE_M):
            read_m(bufs[(i * len(DECODE_M) + j) % LAYER_COPIES], m)

    for i in range(warmup):
        step(i)
    with Timer(torch) as t:
        for i in range(steps):
            step(warmup + i)
    per_m = {}
    for m in DECODE_M:
        for i in range(warmup):
            read_m(bufs[i % LAYER_COPIES], m)
        with Timer(torch) as tm:
            for i in range(steps):
                read_m(bufs[i % LAYER_COPIES], m)
        per_m[str(m)] = round(sum(sizes[m]) * steps / (tm.ms * 1e-3) / 1e9, 1)
    del bufs
    torch.cuda.empty_cache()
    total = sum(sum(v) for v in sizes.values())
    return {"GBps": total * steps / (t.ms * 1e-3) / 1e9, "ms_per_step": t.ms / steps,
            "launches_per_step": sum(len(v) for v in sizes.values()), "per_M_GBps": per_m}


def settle(torch, step, seconds, min_steps):
    """Run step(i) back to back for at least `seconds` of wall time (and
    min_steps steps) so the GPU clock reaches its sustained-load level before a
    timed region: a compute-bound GEMM runs ~20% slower in the first ~20 ms of
    load than in steady state.  Returns the number of steps run."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    i = 0
    while i < min_steps or time.perf_counter() - t0 < seconds:
        step(i)
        i += 1
        if i % 4 == 0:
            torch.cuda.synchronize()  # keep the host clock tied to GPU progress
    torch.cuda.synchronize()
    return i


def bench_prefill(torch, rf, steps, warmup):
    """the Qwen3-8B MLP at M=2048.  One step = gate and up in
    one linear_multi launch (they share the input), then down: 2 launches,
    rotating PREFILL_COPIES layer copies.  The same step as 3 single-projection
    launches is reported as per_op."""
    copies = [make_layer(torch, rf, PREFILL, seed=50 + c) for c in range(PREFILL_COPIES)]
    x = torch.randn(PREFILL_M, 12288, device="cuda").half()
    outs = {n: torch.empty(PREFILL_M, n, device="cuda", dtype=torch.float16) for _, n, _ in PREFILL}

    def step_fused(i):
        gate, up, down = copies[i % PREFILL_COPIES]
        rf.linear_multi(x[:, :4096], [gate[3], up[3]], [gate[4], up[4]])
        rf.linear_into(x[:, :12288], down[3], down[4], None, outs[4096])

    def step_per_op(i):
        for name, n, k, wp, s in copies[i % PREFILL_COPIES]:
            rf.linear_into(x[:, :k], wp, s, None, outs[n])

    step_flops = sum(2 * PREFILL_M * n * k for _, n, k in PREFILL)
    settled = settle(torch, step_fused, PREFILL_SETTLE_S, max(2, warmup))
    with Timer(torch) as t:
        for i in range(steps):
            step_fused(i)
    dist = step_times(torch, step_fused, DIST_REPS, steps)
    settle(torch, step_per_op, PREFILL_SETTLE_S / 4, max(2, warmup))
    with Timer(torch) as tp:
        for i in range(steps):
            step_per_op(i)
    per = []
    for idx, (name, n, k) in enumerate(PREFILL):
        cs = [c[idx] for c in copies]
        xx, out = x[:, :k], outs[n]
        us = per_launch_us(torch, lambda c: rf.linear_into(xx, c[3], c[4], None, out), cs, 12)
        per.append({"proj": name, "M": PREFILL_M, "N": n, "K": k, "us": round(us, 1),
                    "TFLOPs": round(2 * PREFILL_M * n * k / (us * 1e-6) / 1e12, 1),
                    "plan": plan_name(PREFILL_M, n, k)})
    cs = [[c[0], c[1]] for c in copies]
    xx = x[:, :4096]
    us = per_launch_us(torch, lambda c: rf.linear_multi(xx, [p[3] for p in c], [p[4] for p in c]),
                       cs, 12)
    per.append({"proj": "gate_up", "M": PREFILL_M, "N": 2 * 12288, "K": 4096, "us": round(us, 1),
                "TFLOPs": round(2 * PREFILL_M * 2 * 12288 * 4096 / (us * 1e-6) / 1e12, 1),
                "plan": plan_name(PREFILL_M, [12288, 12288], 4096) + " (one launch)"})
    del copies
    torch.cuda.empty_cache()
    launches = steps * 2
    return {"TFLOPs": step_flops * steps / (t.ms * 1e-3) / 1e12, "ms_per_step": t.ms / steps,
            "avg_launch_us": t.ms * 1e3 / launches, "flops_per_launch": step_flops / 2,
            "dist": rate_stats(dist, step_flops, 1e12),
            "per_op_TFLOPs": step_flops * steps / (tp.ms * 1e-3) / 1e12, "settle_steps": settled,
            "steps": steps, "per_launch": per}


def roofline_row(row, bound, bytes_, flops):
    """Add the roofline fraction of a per-launch row: HBM-bound rows against
    8 TB/s, MFMA-bound rows against the dense fp16 peak."""
    us = row["us"]
    row["GBps"] = round(bytes_ / (us * 1e-6) / 1e9, 1)
    if bound == "mfma":
        row["TFLOPs"] = round(flops / (us * 1e-6) / 1e12, 1)
        row["frac"] = round(row["TFLOPs"] / MFMA_FP16_PEAK_TFLOPS, 4)
    else:
        row["frac"] = round(row["GBps"] / HBM_PEAK_GBS, 4)
    row["bound"] = bound
    return row


def bench_cfg0(torch, rf):
    """cfg0: Qwen3-0.6B-shaped single op, M=1, K=1024, N=3072 (192 x 3.1 MB copies)."""
    cfg0 = [make_layer(torch, rf, [("cfg0", 3072, 1024)], seed=900 + c)[0]
            for c in range(CFG0_COPIES)]
    x = torch.randn(1, 1024, device="cuda").half()
    y = torch.empty(1, 3072, device="cuda", dtype=torch.float16)
    us = per_launch_us(torch, lambda c: rf.linear_into(x, c[3], c[4], None, y), cfg0, CFG0_COPIES)
    del cfg0
    return roofline_row({"M": 1, "N": 3072, "K": 1024, "us": round(us, 2), "copies": CFG0_COPIES,
                         "plan": plan_name(1, 3072, 1024)},
                        "hbm", nbytes(1, 3072, 1024), 2 * 3072 * 1024)


def bench_cfg2(torch, rf):
    """cfg2: the Qwen3-14B lm_head, one 778 MB copy (three times the Infinity
    Cache), at M 1 and 8; and the GPU half of the 1000-row argmax agreement
    (the CPU half is in cpu_baseline)."""
    n, k = LM_HEAD
    head = make_layer(torch, rf, [("lm_head", n, k)], seed=914, keep_rowmajor=True)[0]
    rows = []
    for m in (1, 8):
        x = torch.randn(m, k, device="cuda").half()
        y = torch.empty(m, n, device="cuda", dtype=torch.float16)
        us = per_launch_us(torch, lambda c: rf.linear_into(x, c[3], c[4], None, y), [head], 50,
                           replays=1)
        # greedy decode: the token ids, by the fused-argmax launch, and by the logits
        # launch followed by torch.argmax
        us_am = per_launch_us(torch, lambda c: rf.linear_argmax(x, c[3], c[4]), [head], 50,
                              replays=1)
        us_two = per_launch_us(torch, lambda c: (rf.linear_into(x, c[3], c[4], None, y),
                                                  y.argmax(-1)), [head], 50, replays=1)
        rows.append(roofline_row({"M": m, "us": round(us, 1), "plan": plan_name(m, n, k),
                                  "argmax_fused_us": round(us_am, 1),
                                  "logits_then_argmax_us": round(us_two, 1)},
                                 "hbm", nbytes(m, n, k), 2 * m * n * k))
    # 1000 seeded RMS-normalized rows through the fused argmax, in decode batches of 8
    g = torch.Generator(device="cuda").manual_seed(2)
    z = torch.randn(ARGMAX_ROWS, k, generator=g, device="cuda")
    xa = (z / z.pow(2).mean(dim=1, keepdim=True).sqrt()).half()
    ids = torch.cat([rf.linear_argmax(xa[i:i + 8], head[3], head[4])
                     for i in range(0, ARGMAX_ROWS, 8)])
    argmax_case = {"x": xa.cpu(), "ids": ids.cpu(), "q": head[5].cpu(), "s": head[4].cpu()}
    del head, z, xa
    torch.cuda.empty_cache()
    return rows, argmax_case


def bench_cfg4(torch, rf):
    """cfg4: Qwen3-VL-32B projections at M in {1, 32, 512}, four layer copies
    (1.96 GB): every projection's copies together exceed the 256 MB Infinity
    Cache.  M 1 and 32 are judged against HBM, M 512 against MFMA."""
    copies = [make_layer(torch, rf, QWEN3_VL_32B, seed=940 + c) for c in range(4)]
    rows = []
    for m in (1, 32, 512):
        x = torch.randn(m, 25600, device="cuda").half()
        bound = "mfma" if m >= 512 else "hbm"
        reps = 52 if m < 512 else 12
        for idx, (name, n, k) in enumerate(QWEN3_VL_32B):
            y = torch.empty(m, n, device="cuda", dtype=torch.float16)
            cs = [c[idx] for c in copies]
            xx = x[:, :k]
            us = per_launch_us(torch, lambda c: rf.linear_into(xx, c[3], c[4], None, y), cs, reps)
            rows.append(roofline_row({"M": m, "proj": name, "N": n, "K": k, "us": round(us, 2),
                                      "plan": plan_name(m, n, k)},
                                     bound, nbytes(m, n, k), 2 * m * n * k))
        xx = x[:, :5120]
        for name, idxs in (("qkv", (0, 1, 2)), ("gate_up", (4, 5))):
            cs = [[c[i] for i in idxs] for c in copies]
            us = per_launch_us(torch, lambda c: rf.linear_multi(xx, [p[3] for p in c],
                                                                [p[4] for p in c]), cs, reps)
            ns = [QWEN3_VL_32B[i][1] for i in idxs]
            rows.append(roofline_row({"M": m, "proj": name, "N": sum(ns), "K": 5120,
                                      "us": round(us, 2),
                                      "plan": plan_name(m, ns, 5120) + " (one launch)"},
                                     bound, group_bytes(m, idxs, QWEN3_VL_32B),
                                     2 * m * sum(ns) * 5120))
    del copies
    torch.cuda.empty_cache()
    return rows


# Launches of few tiles across M (the GEMV's 16-wavefront rule at M 17..32,
# the GEMM's two-K-group rules above): Qwen3-8B and Qwen3-VL-32B projections
# that leave most CUs without a whole tile.
FEW_TILES = [(24, "8b k", 1024, 4096), (32, "8b k", 1024, 4096), (32, "vl k", 1024, 5120),
             (48, "8b q", 4096, 4096), (48, "8b k", 1024, 4096), (64, "8b q", 4096, 4096),
             (96, "8b q", 4096, 4096), (96, "8b k", 1024, 4096), (96, "vl k", 1024, 5120),
             (1024, "8b k", 1024, 4096), (1024, "vl k", 1024, 5120),
             (2048, "8b k", 1024, 4096), (2048, "vl k", 1024, 5120)]


def bench_few_tiles(torch, rf):
    """Per-launch times of FEW_TILES through linear_into (AUTO), rotating
    weight copies of >= 320 MB per shape (past the 256 MB Infinity Cache);
    M >= 512 judged against MFMA, smaller M against HBM."""
    rows = []
    for m, name, n, k in FEW_TILES:
        ncopies = max(4, -(-(320 << 20) // (n * k)))
        cs = [make_layer(torch, rf, [(name, n, k)], seed=970 + c)[0] for c in range(ncopies)]
        x = torch.randn(m, k, device="cuda").half()
        y = torch.empty(m, n, device="cuda", dtype=torch.float16)
        us = per_launch_us(torch, lambda c: rf.linear_into(x, c[3], c[4], None, y), cs,
                           2 * ncopies)
        rows.append(roofline_row({"M": m, "proj": name, "N": n, "K": k, "us": round(us, 2),
                                  "plan": plan_name(m, n, k)},
                                 "mfma" if m >= 512 else "hbm", nbytes(m, n, k), 2 * m * n * k))
        del cs
    torch.cuda.empty_cache()
    return rows


# Decode projections of the reference's model families (hidden / q / k,v /
# MLP widths from each model's config), q/k/v and gate/up fused as a decoder
# layer issues them: (family, projection, output widths, K).
MODEL_SHAPES = [
    ("Qwen3-0.6B", "qkv", [2048, 1024, 1024], 1024), ("Qwen3-0.6B", "o", [1024], 2048),
    ("Qwen3-0.6B", "gate_up", [3072, 3072], 1024), ("Qwen3-0.6B", "down", [1024], 3072),
    ("Qwen3-1.7B", "qkv", [2048, 1024, 1024], 2048), ("Qwen3-1.7B", "o", [2048], 2048),
    ("Qwen3-1.7B", "gate_up", [6144, 6144], 2048), ("Qwen3-1.7B", "down", [2048], 6144),
    ("Qwen3-4B", "qkv", [4096, 1024, 1024], 2560), ("Qwen3-4B", "o", [2560], 4096),
    ("Qwen3-4B", "gate_up", [9728, 9728], 2560), ("Qwen3-4B", "down", [2560], 9728),
    ("Qwen3-8B", "qkv", [4096, 1024, 1024], 4096), ("Qwen3-8B", "o", [4096], 4096),
    ("Qwen3-8B", "gate_up", [12288, 12288], 4096), ("Qwen3-8B", "down", [4096], 12288),
    ("Qwen3-14B", "qkv", [5120, 1024, 1024], 5120), ("Qwen3-14B", "o", [5120], 5120),
    ("Qwen3-14B", "gate_up", [17408, 17408], 5120), ("Qwen3-14B", "down", [5120], 17408),
    ("Qwen3-(VL-)32B", "qkv", [8192, 1024, 1024], 5120), ("Qwen3-(VL-)32B", "o", [5120], 8192),
    ("Qwen3-(VL-)32B", "gate_up", [25600, 25600], 5120), ("Qwen3-(VL-)32B", "down", [5120], 25600),
    ("Qwen2.5-VL-3B", "qkv", [2048, 256, 256], 2048), ("Qwen2.5-VL-3B", "o", [2048], 2048),
    ("Qwen2.5-VL-3B", "gate_up", [11008, 11008], 2048), ("Qwen2.5-VL-3B", "down", [2048], 11008),
    ("Qwen2.5-VL-7B", "qkv", [3584, 512, 512], 3584), ("Qwen2.5-VL-7B", "o", [3584], 3584),
    ("Qwen2.5-VL-7B", "gate_up", [18944, 18944], 3584), ("Qwen2.5-VL-7B", "down", [3584], 18944),
    ("Pi0.5 Gemma 2B", "qkv", [2048, 256, 256], 2048), ("Pi0.5 Gemma 2B", "o", [2048], 2048),
    ("Pi0.5 Gemma 2B", "gate_up", [16384, 16384], 2048), ("Pi0.5 Gemma 2B", "down", [2048], 16384),
    ("Pi0.5 expert", "qkv", [2048, 256, 256], 1024), ("Pi0.5 expert", "o", [1024], 2048),
    ("Pi0.5 expert", "gate_up", [4096, 4096], 1024), ("Pi0.5 expert", "down", [1024], 4096),
]
MODEL_SHAPES_M = (1, 4, 8, 16, 24, 32)


def bench_model_shapes(torch, rf):
    """Per-launch times of MODEL_SHAPES at M in MODEL_SHAPES_M (decode sizes
    and the GEMV / GEMM crossover) through linear_into / linear_multi
    (AUTO), replayed from a HIP graph, rotating
    weight copies of >= 320 MB per shape (random int8 tiles: the timing does
    not depend on the values), against HBM."""
    from rhinoforge_amd import capi
    from rhinoforge_amd.ops import packed_shape
    rows = []
    for fam, proj, ns, k in MODEL_SHAPES:
        wbytes = sum(n * k for n in ns)
        ncopies = max(4, -(-(320 << 20) // wbytes))
        cs = [[torch.randint(-127, 128, packed_shape(n, k), dtype=torch.int8, device="cuda")
               for n in ns] for _ in range(ncopies)]
        sc = [torch.full((n,), 1e-3, dtype=torch.float16, device="cuda") for n in ns]
        for m in MODEL_SHAPES_M:
            x = torch.randn(m, k, device="cuda").half()
            if len(ns) == 1:
                y = torch.empty(m, ns[0], device="cuda", dtype=torch.float16)
                fn = lambda c: rf.linear_into(x, c[0], sc[0], None, y)  # noqa: E731
            else:
                fn = lambda c: rf.linear_multi(x, c, sc)  # noqa: E731
            us = per_launch_us(torch, fn, cs, max(2 * ncopies, 48))
            p = capi.plan(m, ns, k)
            b = sum(nbytes(m, n, k) for n in ns) - (len(ns) - 1) * 2 * m * k
            rows.append(roofline_row({"family": fam, "proj": proj, "M": m, "N": ns, "K": k,
                                      "us": round(us, 2),
                                      "plan": f"{p['name']}, {p['splits']} split(s)"},
                                     "hbm", b, 2 * m * sum(ns) * k))
        log(f"  {fam} {proj}: " + ", ".join(f"M{r['M']} {r['us']}" for r in rows[-len(MODEL_SHAPES_M):]))
        del cs
        torch.cuda.empty_cache()
    return rows


def bench_other_configs(torch, rf):
    """Per-launch timings of BASELINE configs 0, 2 and 4 and the W4A16 rows (not
    part of `value`); returns them and config 2's argmax case for cpu_baseline."""
    out = {"cfg0": bench_cfg0(torch, rf)}
    out["cfg2_lm_head"], argmax_case = bench_cfg2(torch, rf)
    out["cfg4_vl32b"] = bench_cfg4(torch, rf)
    out["w4a16"] = bench_w4a16(torch, rf)
    return out, argmax_case


def nbytes_w4(m, n, k, gs):
    """Algorithmic bytes of one W4A16 call: int4 weight, scales, x, y."""
    scale = 2 * n * (k // gs if gs else 1)
    return n * k // 2 + scale + 2 * m * k + 2 * m * n


def bench_w4a16(torch, rf):
    """W4A16 on the same Qwen3-8B shapes: decode projections at M 1 and 16 and the
    M=2048 MLP prefill, per-channel and group-wise (32, 128); random int4 values
    and scales, four rotated layer copies (384 MB, past the Infinity Cache)."""
    rows = []
    for gs in (0, 32, 128):
        copies = []
        for c in range(LAYER_COPIES):
            g = torch.Generator(device="cuda").manual_seed(7000 + 10 * gs + c)
            layer = []
            for name, n, k in QWEN3_8B:
                q = torch.randint(-8, 8, (n, k), generator=g, device="cuda", dtype=torch.int8)
                sshape = (k // gs, n) if gs else (n,)
                sc = (torch.rand(sshape, generator=g, device="cuda") * 0.01 + 1e-3).half()
                layer.append((name, n, k, rf.pack_weight_int4(q), sc))
                del q
            copies.append(layer)
        fmt = 2 if gs else 1
        for m in (1, 16):
            x = torch.randn(m, 12288, device="cuda").half()
            step_bytes, step_us = 0, 0.0
            for idx, (name, n, k) in enumerate(QWEN3_8B):
                xx = x[:, :k]
                us = per_launch_us(torch, lambda c: rf.linear_w4a16(xx, c[3], c[4]),
                                   [layer[idx] for layer in copies], 40)
                b = nbytes_w4(m, n, k, gs)
                step_bytes, step_us = step_bytes + b, step_us + us
                rows.append({"group_size": gs, "M": m, "proj": name, "N": n, "K": k,
                             "us": round(us, 2), "GBps": round(b / (us * 1e-6) / 1e9, 1),
                             "plan": plan_name(m, n, k, fmt)})
            rows.append({"group_size": gs, "M": m, "proj": "layer (7 launches)",
                         "us": round(step_us, 2),
                         "GBps": round(step_bytes / (step_us * 1e-6) / 1e9, 1)})
            # the layer as a decoder issues it: q/k/v and gate/up each in one
            # w4a16.linear_multi launch (they share the input), o, down -- 4 launches

            def layer4(c, x=x):
                for idxs in DECODE_GROUPS:
                    xx = x[:, :QWEN3_8B[idxs[0]][2]]
                    if len(idxs) == 1:
                        rf.linear_w4a16(xx, c[idxs[0]][3], c[idxs[0]][4])
                    else:
                        rf.linear_multi_w4a16(xx, [c[i][3] for i in idxs], [c[i][4] for i in idxs])
            us4 = per_launch_us(torch, layer4, copies, 12)
            # x is read once per launch
            b4 = step_bytes - sum(2 * m * QWEN3_8B[g[0]][2] * (len(g) - 1) for g in DECODE_GROUPS)
            rows.append({"group_size": gs, "M": m, "proj": "layer (4 launches: qkv, o, gate_up, down)",
                         "us": round(us4, 2), "GBps": round(b4 / (us4 * 1e-6) / 1e9, 1)})
        if gs in (0, 32):
            x = torch.randn(PREFILL_M, 12288, device="cuda").half()
            for idx in (4, 6):  # gate (12288x4096) and down (4096x12288)
                name, n, k = QWEN3_8B[idx]
                xx = x[:, :k]
                us = per_launch_us(torch, lambda c: rf.linear_w4a16(xx, c[3], c[4]),
                                   [layer[idx] for layer in copies], 8)
                rows.append({"group_size": gs, "M": PREFILL_M, "proj": name, "N": n, "K": k,
                             "us": round(us, 1),
                             "TFLOPs": round(2 * PREFILL_M * n * k / (us * 1e-6) / 1e12, 1),
                             "plan": plan_name(PREFILL_M, n, k, fmt)})
        del copies
        torch.cuda.empty_cache()
    return rows


def cpu_baseline(torch, argmax_case=None, reps=5):
    """The reference's CPU path, timed on the host cores (torch's CPU kernels,
    torch.set_num_threads(T) with T = the box's CPU share, OMP_NUM_THREADS, else
    os.cpu_count()):
      dequant  W16 = fp16(s)[:, None] * fp16(q), in fp16 (quant/_common.py:39-41;
               the lm_head form fp16(f32(q) * f32(s)), adapters/qwen3.py:617-621,
               is bit-identical);
      matmul   y = F.linear(x16, W16) (adapters/qwen3.py:623).
    The reference caches its dequantized lm_head (adapters/qwen3.py:616-622), so
    the headline CPU figure is the matmul on a cached W16; the dequant is timed
    separately.  Median and p90 over `reps` runs after one warmup:
      * config 1 at M=1 (seven projections), GB/s of algorithmic bytes;
      * config 3 on a 128-row sample of its 2048 rows, TFLOP/s;
      * config 2's 1000 RMS-normalized rows, timed once, whose argmax is
        compared with the GPU's fused argmax on the same weights and rows."""
    import numpy as np
    F = torch.nn.functional
    threads = int(os.environ.get("OMP_NUM_THREADS") or 0) or (os.cpu_count() or 1)
    torch.set_num_threads(threads)

    def med_p90(v):
        return float(np.median(v)), float(np.percentile(v, 90))

    g = torch.Generator().manual_seed(0)

    def rand_layer(specs):
        out = []
        for _, n, k in specs:
            q = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=g)
            s = (torch.rand(n, generator=g) * 1e-3 + 1e-4).half()
            out.append((q, s))
        return out

    def dequant(layer):
        return [s[:, None] * q.half() for q, s in layer]

    # config 1, M = 1
    layer = rand_layer(QWEN3_8B)
    x = torch.randn(1, 12288, generator=g).half()
    t_deq, t_mm = [], []
    for rep in range(reps + 1):
        a = time.perf_counter()
        ws = dequant(layer)
        b = time.perf_counter()
        for w in ws:
            F.linear(x[:, :w.shape[1]], w)
        c = time.perf_counter()
        if rep:
            t_deq.append(b - a)
            t_mm.append(c - b)
    layer_bytes = sum(nbytes(1, n, k) for _, n, k in QWEN3_8B)
    mm_med, mm_p90 = med_p90(t_mm)
    deq_med, _ = med_p90(t_deq)
    del layer, ws
    # config 3, a 128-row sample
    rows3 = 128
    layer = rand_layer(PREFILL)
    ws = dequant(layer)
    x3 = torch.randn(rows3, 12288, generator=g).half()
    flops3 = sum(2 * rows3 * n * k for _, n, k in PREFILL)
    t3 = []
    for rep in range(reps + 1):
        a = time.perf_counter()
        for w in ws:
            F.linear(x3[:, :w.shape[1]], w)
        if rep:
            t3.append(time.perf_counter() - a)
    t3_med, t3_p90 = med_p90(t3)
    del layer, ws, x3
    res = {
        "value": round(layer_bytes / mm_med / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"cfg1 Qwen3-8B layer, 7 projections at M=1: torch CPU F.linear on a cached "
                   f"fp16 dequantized weight, median of {reps} runs (p90 "
                   f"{layer_bytes / mm_p90 / 1e9:.3f} GB/s); dequant alone {deq_med * 1e3:.1f} ms "
                   f"per layer; dequant + matmul {layer_bytes / (mm_med + deq_med) / 1e9:.3f} GB/s"),
        "p90_GBps": round(layer_bytes / mm_p90 / 1e9, 3),
        "dequant_ms_per_layer": round(deq_med * 1e3, 2),
        "cfg3_rows128_TFLOPs": {"median": round(flops3 / t3_med / 1e12, 3),
                                "p90": round(flops3 / t3_p90 / 1e12, 3), "reps": reps},
        "cpu_count": os.cpu_count(),
        "torch": torch.__version__,
        "cpu_model": "",
    }
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    res["cpu_model"] = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    agreement = None
    if argmax_case is not None:
        # config 2: 1000 rows against the lm_head the GPU ran, timed once
        q, s, xa = argmax_case["q"], argmax_case["s"], argmax_case["x"]
        n, k = q.shape
        a = time.perf_counter()
        w16 = (q.float() * s.float()[:, None]).half()  # adapters/qwen3.py:617-621
        b = time.perf_counter()
        y = F.linear(xa, w16)
        c = time.perf_counter()
        del w16
        res["cfg2_1000_rows"] = {"dequant_s": round(b - a, 2), "matmul_s": round(c - b, 2),
                                 "TFLOPs": round(2 * xa.shape[0] * n * k / (c - b) / 1e12, 3)}
        a_cpu = y.float().argmax(1)
        a_gpu = argmax_case["ids"].long()
        bad = (a_cpu != a_gpu).nonzero().flatten().tolist()
        ties = []
        for r in bad:
            v_c, v_g = float(y[r, a_cpu[r]]), float(y[r, a_gpu[r]])
            # a near-tie: the two logits lie within 2 fp16 ulps of each other
            # (docs/validation_policy.md:124-128 counts these apart)
            if abs(v_c - v_g) <= 2 * float(np.spacing(np.float16(abs(v_c)))):
                ties.append(r)
        agreement = {"rows": int(xa.shape[0]), "agree": int(xa.shape[0]) - len(bad),
                     "near_ties": len(ties), "disagree_beyond_ties": len(bad) - len(ties),
                     "gpu": "rf_w8a16_linear_argmax, batches of 8 rows",
                     "cpu": "fp16(f32(q)*f32(s)) then F.linear, argmax (lowest index)"}
    return res, agreement


def measured_traffic():
    """HBM bytes per GEMV launch from the committed rocprofv3 --pmc summary, if any."""
    path = os.path.join(ROOT, "profiles", "gemv_decode_traffic.json")
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip configs 0, 2 and 4")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="first run three device-to-device copies of this many MB (the "
                         "known-size reference kernel for rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--only", choices=("decode", "prefill", "cfg0", "cfg2", "cfg4", "w4a16",
                                       "few_tiles", "model_shapes"),
                    help="run one section alone and print its result (a profiling aid: "
                         "its JSON line is not the benchmark line)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build runs the W8A16 path on a single "
              "MI355X (no collectives, no multi-GPU figure); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    import rhinoforge_amd as rf

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    torch.cuda.synchronize()
    log(f"device: {torch.cuda.get_device_name(0)}")

    if args.copy_calibration_mb > 0:
        n = args.copy_calibration_mb << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy calibration: 3 x {n} bytes read + written")
        del src, dst
    if args.only:
        log(f"only {args.only}...")
        sections = {
            "decode": lambda: bench_decode(torch, rf, args.steps, args.warmup),
            "prefill": lambda: bench_prefill(torch, rf, max(10, args.steps // 2), args.warmup),
            "cfg0": lambda: bench_cfg0(torch, rf),
            "cfg2": lambda: bench_cfg2(torch, rf)[0],
            "cfg4": lambda: bench_cfg4(torch, rf),
            "w4a16": lambda: bench_w4a16(torch, rf),
            "few_tiles": lambda: bench_few_tiles(torch, rf),
            "model_shapes": lambda: bench_model_shapes(torch, rf),
        }
        print(json.dumps({"only": args.only, "result": sections[args.only]()}), flush=True)
        return
    log("decode (cfg1)...")
    dec = bench_decode(torch, rf, args.steps, args.warmup)
    log(f"decode: {dec['GBps']:.1f} GB/s ({dec['avg_launch_us']:.2f} us/launch, q/k/v and "
        f"gate/up fused); per-step median {dec['dist']['median']} GB/s; one launch per "
        f"projection: {dec['per_op_GBps']:.1f} GB/s")
    env = read_envelope(torch, args.steps, args.warmup)
    if env:
        log(f"read envelope of the same 12 launches: {env['GBps']:.1f} GB/s")
    pre = None
    if not args.no_prefill:
        log("prefill (cfg3)...")
        pre = bench_prefill(torch, rf, max(10, args.steps // 2), args.warmup)
        log(f"prefill: {pre['TFLOPs']:.1f} TFLOP/s (gate/up fused); per-step median "
            f"{pre['dist']['median']}; one launch per projection: {pre['per_op_TFLOPs']:.1f}")
    extra, argmax_case = None, None
    if not args.no_extra:
        log("configs 0, 2, 4...")
        extra, argmax_case = bench_other_configs(torch, rf)
    cpu, agreement = None, None
    if not args.no_cpu:
        log("cpu baseline...")
        cpu, agreement = cpu_baseline(torch, argmax_case)
        log(f"cpu: {cpu['value']} GB/s on {cpu['cores']} threads; argmax agreement {agreement}")

    achieved = dec["avg_bytes_per_launch"] / (dec["avg_launch_us"] * 1e-6) / 1e9
    traffic = measured_traffic()
    per_m = {m: {"GBps": dec["per_M_fused_GBps"][m],
                 "envelope_GBps": env["per_M_GBps"][m] if env else None,
                 "value_over_envelope": (round(dec["per_M_fused_GBps"][m] / env["per_M_GBps"][m], 4)
                                         if env else None),
                 "per_op_GBps": dec["per_M_per_op_GBps"][m]} for m in dec["per_M_fused_GBps"]}
    line = {
        "metric": METRIC,
        "value": round(dec["GBps"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (weights N(0,0.02) int8 per-channel quantized, activations N(0,1) fp16)",
        "config": {
            "workload": "cfg1: Qwen3-8B decode layer, 7 W8A16 projections x M in {1,4,16}",
            "layer_copies_rotated": LAYER_COPIES,
            "weight_dtype": "int8",
            "per_M": per_m,
            "launch": ("per M: q/k/v in one linear_multi launch, o, gate/up in one "
                       "linear_multi launch, down (12 launches per step); eager torch-op "
                       "launches on one stream"),
            "per_op_GBps": round(dec["per_op_GBps"], 1),
            "per_op_ms_per_step": round(dec["per_op_ms_per_step"], 4),
            "per_op_note": "the same step as 21 single-projection launches",
            "graph_replay": dec["graph"],
        },
        "stats": {"decode_GBps": dec["dist"],
                  "prefill_TFLOPs": pre["dist"] if pre else None,
                  "note": (f"{DIST_REPS} steps with an event after every step, after the "
                           "headline's timed region; p10/p90 of the per-step rates")},
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic.get("hbm_bytes_per_launch") if traffic else None,
            "kernel": "w8a16_gemv_kernel (all instances)",
            "avg_launch_us": round(dec["avg_launch_us"], 3),
            "algorithmic_bytes_per_launch": round(dec["avg_bytes_per_launch"]),
        },
        "prefill": None if pre is None else {
            "workload": "cfg3: Qwen3-8B MLP prefill M=2048 (gate, up, down)",
            "value": round(pre["TFLOPs"], 1),
            "unit": "TFLOP/s",
            "steps": pre["steps"],
            "ms_per_step": round(pre["ms_per_step"], 4),
            "launch": ("gate/up in one linear_multi launch, then down (2 launches per step), "
                       f"{PREFILL_COPIES} rotated layer copies (604 MB); timed after "
                       f"{pre['settle_steps']} untimed steps (>= {PREFILL_SETTLE_S:.2f} s) bring "
                       "the GPU clock to its sustained level"),
            "per_op_TFLOPs": round(pre["per_op_TFLOPs"], 1),
            "roofline": {"bound": "mfma", "achieved": round(pre["TFLOPs"], 1),
                         "peak": MFMA_FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(pre["TFLOPs"] / MFMA_FP16_PEAK_TFLOPS, 4),
                         "kernel": "w8a16_gemm_v3_kernel (all instances)",
                         "avg_launch_us": round(pre["avg_launch_us"], 2),
                         "flops_per_launch": pre["flops_per_launch"]},
            "per_launch": pre["per_launch"],
        },
        "read_envelope": None if env is None else {
            "GBps": round(env["GBps"], 1),
            "frac_of_peak": round(env["GBps"] / HBM_PEAK_GBS, 4),
            "value_over_envelope": round(dec["GBps"] / env["GBps"], 4),
            "ms_per_step": round(env["ms_per_step"], 4),
            "per_M_GBps": env["per_M_GBps"],
            "what": ("the decode step's 12 launches with the GEMV replaced by a plain "
                     "non-temporal streaming read of the same byte counts (rotated buffers, "
                     "eager, same stream and timer): the rate this launch structure allows"),
        },
        "cpu_baseline": cpu,
        "cfg2_argmax_agreement": agreement,
        "decode_per_launch": dec["per_launch"],
        "other_configs": extra,
    }
    if traffic:
        log(json.dumps({"traffic_source": traffic}))
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
