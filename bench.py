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
launched eagerly through the torch op; the per-projection rows replay HIP
graphs of 40 back-to-back launches, i.e. GPU-side time per launch.

The same JSON line carries
  * roofline      -- the decode GEMV kernel (every launch in the timed
                     region): algorithmic bytes per launch / average launch
                     duration (timed region / launches, 12 per step) against the 8 TB/s
                     HBM peak; `traffic` is the measured HBM bytes per launch
                     from profiles/gemv_decode_traffic.json when present;
  * prefill       -- BASELINE config 3 (Qwen3-8B MLP prefill, M=2048) in
                     TFLOP/s against the 2.5166 PFLOP/s dense FP16 MFMA peak:
                     gate/up in one launch, then down, timed after >= 0.25 s
                     of the same steps (the clock's sustained-load level);
  * configs       -- per-launch timings of configs 0, 2 and 4 and of each
                     config-1 projection (back-to-back launches on rotating
                     weight copies);
  * read_envelope -- the same 12-launch step with a plain streaming read of
                     the same bytes in place of the GEMV (lib/librf_bench.so):
                     the bound the launch structure itself puts on `value`;
  * cpu_baseline  -- the CPU restatement of the reference's dequantize-then-
                     matmul path (oracle, numpy/BLAS on the host cores) on a
                     bounded sample of config 1 at M=1.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
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
PREFILL = [("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288)]
PREFILL_M = 2048
PREFILL_SETTLE_S = 0.25


def nbytes(m, n, k, bias=False):
    return n * k + 2 * n + 2 * m * k + 2 * m * n + (2 * n if bias else 0)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_layer(torch, rf, specs, seed):
    """Quantized + packed weights of one layer, generated on the device."""
    layer = []
    for i, (name, n, k) in enumerate(specs):
        g = torch.Generator(device="cuda").manual_seed(seed * 100 + i)
        w = torch.randn(n, k, generator=g, device="cuda", dtype=torch.float32) * 0.02
        q, s = rf.quantize_linear_per_channel(w)
        del w
        layer.append((name, n, k, rf.pack_weight(q), s))
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


def per_launch_us(torch, fn, copies, reps, graph=True):
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
        for _ in range(3):
            g.replay()
    return t.ms * 1e3 / (3 * reps)


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

    # The same step with the projections that share an input fused into one
    # launch each (q/k/v and gate/up; o and down stay single): 4 launches per M.
    def step_fused(i):
        for j, m in enumerate(DECODE_M):
            layer = layers[(i * len(DECODE_M) + j) % LAYER_COPIES]
            x = xs[m][:, :4096]
            q, k_, v, o, gate, up, down = layer
            rf.linear_multi(x, [q[3], k_[3], v[3]], [q[4], k_[4], v[4]])
            rf.linear_into(x, o[3], o[4], None, outs[(m, 4096)])
            g, u = rf.linear_multi(x, [gate[3], up[3]], [gate[4], up[4]])
            rf.linear_into(xs[m][:, :12288], down[3], down[4], None, outs[(m, 4096)])

    for i in range(warmup):
        step_fused(i)
    with Timer(torch) as tf:
        for i in range(steps):
            step_fused(warmup + i)

    rows = []
    for m in DECODE_M:
        for idx, (name, n, k) in enumerate(QWEN3_8B):
            copies = [layer[idx] for layer in layers]
            x, out = xs[m][:, :k], outs[(m, n)]
            us = per_launch_us(torch, lambda c: rf.linear_into(x, c[3], c[4], None, out),
                               copies, 40)
            rows.append({"M": m, "proj": name, "N": n, "K": k, "us": round(us, 2),
                         "GBps": round(nbytes(m, n, k) / (us * 1e-6) / 1e9, 1),
                         "kernel": "gemv" if rf.select_kernel(m, n, k) == rf.KERNEL_GEMV
                         else "gemm"})
    for m in DECODE_M:
        x = xs[m][:, :4096]
        for name, idxs in (("qkv", (0, 1, 2)), ("gate_up", (4, 5))):
            copies = [[layer[i] for i in idxs] for layer in layers]
            us = per_launch_us(torch, lambda c: rf.linear_multi(x, [p[3] for p in c],
                                                                [p[4] for p in c]), copies, 40)
            b = sum(nbytes(m, QWEN3_8B[i][1], 4096) - 2 * m * 4096 for i in idxs) + 2 * m * 4096
            rows.append({"M": m, "proj": name, "N": sum(QWEN3_8B[i][1] for i in idxs), "K": 4096,
                         "us": round(us, 2), "GBps": round(b / (us * 1e-6) / 1e9, 1),
                         "kernel": "gemv (one launch)"})
    per_m = {}
    for m in DECODE_M:
        sel = [r for r in rows if r["M"] == m and r["proj"] in dict((p, 1) for p, _, _ in QWEN3_8B)]
        per_m[str(m)] = round(sum(nbytes(m, r["N"], r["K"]) for r in sel)
                              / sum(r["us"] * 1e-6 for r in sel) / 1e9, 1)
    del layers
    torch.cuda.empty_cache()
    fused_launches = steps * len(DECODE_M) * 4
    # Algorithmic bytes of the fused step: a shared input is read once per launch.
    fused_bytes = 0
    for m in DECODE_M:
        for idxs in ((0, 1, 2), (3,), (4, 5), (6,)):
            k = QWEN3_8B[idxs[0]][2]
            fused_bytes += sum(nbytes(m, QWEN3_8B[i][1], k) - 2 * m * k for i in idxs) + 2 * m * k
    return {
        "GBps": fused_bytes * steps / (tf.ms * 1e-3) / 1e9,
        "ms_per_step": tf.ms / steps,
        "launches": fused_launches,
        "avg_launch_us": tf.ms * 1e3 / fused_launches,
        "avg_bytes_per_launch": fused_bytes / (len(DECODE_M) * 4),
        "per_op_GBps": step_bytes * steps / (t.ms * 1e-3) / 1e9,
        "per_op_ms_per_step": t.ms / steps,
        "per_op_avg_launch_us": t.ms * 1e3 / launches,
        "per_M_GBps": per_m,
        "per_launch": rows,
    }


def read_envelope(torch, steps, warmup):
    """The decode step's launch structure with the GEMV replaced by a plain
    streaming read (lib/librf_bench.so): 12 launches per step reading the
    same algorithmic byte counts, rotated over LAYER_COPIES buffer sets, eager
    on one stream and timed like the GEMV step.  Launch gaps, ramp-up and
    drain bound the decode step no matter what kernel runs; this is that
    bound on the device at hand."""
    import ctypes
    path = os.path.join(ROOT, "rhinoforge_amd", "lib", "librf_bench.so")
    if not os.path.isfile(path):
        log(f"read envelope skipped: {path} not built")
        return None
    lib = ctypes.CDLL(path)
    lib.rf_bench_stream_read.restype = ctypes.c_int
    lib.rf_bench_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                         ctypes.c_void_p]
    sizes = []  # algorithmic bytes of the fused step's launches, in launch order
    for m in DECODE_M:
        for idxs in ((0, 1, 2), (3,), (4, 5), (6,)):
            k = QWEN3_8B[idxs[0]][2]
            b = sum(nbytes(m, QWEN3_8B[i][1], k) - 2 * m * k for i in idxs) + 2 * m * k
            sizes.append((b + 15) // 16 * 16)
    bufs = [[torch.empty(b, dtype=torch.uint8, device="cuda") for b in sizes]
            for _ in range(LAYER_COPIES)]
    for c in bufs:
        for t in c:
            t.fill_(1)
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream

    def step(i):
        for s, b in enumerate(sizes):
            buf = bufs[(i * len(DECODE_M) + s // 4) % LAYER_COPIES][s]
            st = lib.rf_bench_stream_read(buf.data_ptr(), b, sink.data_ptr(), stream)
            if st != 0:
                raise RuntimeError(f"rf_bench_stream_read: hipError {st}")

    for i in range(warmup):
        step(i)
    with Timer(torch) as t:
        for i in range(steps):
            step(warmup + i)
    del bufs
    torch.cuda.empty_cache()
    gbps = sum(sizes) * steps / (t.ms * 1e-3) / 1e9
    return {"GBps": gbps, "ms_per_step": t.ms / steps, "launches_per_step": len(sizes)}


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
    one linear_multi launch (they share the input), then down: 2 launches.  The
    same step as 3 single-projection launches is reported as per_op."""
    copies = [make_layer(torch, rf, PREFILL, seed=50 + c) for c in range(2)]
    x = torch.randn(PREFILL_M, 12288, device="cuda").half()
    outs = {n: torch.empty(PREFILL_M, n, device="cuda", dtype=torch.float16) for _, n, _ in PREFILL}

    def step_fused(i):
        gate, up, down = copies[i % 2]
        rf.linear_multi(x[:, :4096], [gate[3], up[3]], [gate[4], up[4]])
        rf.linear_into(x[:, :12288], down[3], down[4], None, outs[4096])

    def step_per_op(i):
        for name, n, k, wp, s in copies[i % 2]:
            rf.linear_into(x[:, :k], wp, s, None, outs[n])

    flops = sum(2 * PREFILL_M * n * k for _, n, k in PREFILL) * steps
    settled = settle(torch, step_fused, PREFILL_SETTLE_S, max(2, warmup))
    with Timer(torch) as t:
        for i in range(steps):
            step_fused(i)
    settle(torch, step_per_op, PREFILL_SETTLE_S / 4, max(2, warmup))
    with Timer(torch) as tp:
        for i in range(steps):
            step_per_op(i)
    per = []
    for idx, (name, n, k) in enumerate(PREFILL):
        cs = [c[idx] for c in copies]
        xx, out = x[:, :k], outs[n]
        us = per_launch_us(torch, lambda c: rf.linear_into(xx, c[3], c[4], None, out), cs, 10)
        per.append({"proj": name, "M": PREFILL_M, "N": n, "K": k, "us": round(us, 1),
                    "TFLOPs": round(2 * PREFILL_M * n * k / (us * 1e-6) / 1e12, 1)})
    cs = [[c[0], c[1]] for c in copies]
    xx = x[:, :4096]
    us = per_launch_us(torch, lambda c: rf.linear_multi(xx, [p[3] for p in c], [p[4] for p in c]),
                       cs, 10)
    per.append({"proj": "gate_up", "M": PREFILL_M, "N": 2 * 12288, "K": 4096, "us": round(us, 1),
                "TFLOPs": round(2 * PREFILL_M * 2 * 12288 * 4096 / (us * 1e-6) / 1e12, 1),
                "kernel": "one launch"})
    del copies
    torch.cuda.empty_cache()
    launches = steps * 2
    return {"TFLOPs": flops / (t.ms * 1e-3) / 1e12, "ms_per_step": t.ms / steps,
            "avg_launch_us": t.ms * 1e3 / launches, "flops_per_launch": flops / launches,
            "per_op_TFLOPs": flops / (tp.ms * 1e-3) / 1e12, "settle_steps": settled,
            "steps": steps, "per_launch": per}


def bench_other_configs(torch, rf):
    """Per-launch timings of BASELINE configs 0, 2 and 4 (not part of `value`)."""
    out = {}
    # cfg0: Qwen3-0.6B-shaped single op, M=1, K=1024, N=3072 (many copies: 3 MB each)
    cfg0 = [make_layer(torch, rf, [("cfg0", 3072, 1024)], seed=900 + c)[0] for c in range(96)]
    x = torch.randn(1, 1024, device="cuda").half()
    y = torch.empty(1, 3072, device="cuda", dtype=torch.float16)
    us = per_launch_us(torch, lambda c: rf.linear_into(x, c[3], c[4], None, y), cfg0, 96)
    out["cfg0"] = {"M": 1, "N": 3072, "K": 1024, "us": round(us, 2),
                   "GBps": round(nbytes(1, 3072, 1024) / (us * 1e-6) / 1e9, 1)}
    del cfg0
    # cfg2: Qwen3-14B lm_head, one 778 MB copy (larger than the Infinity Cache)
    head = make_layer(torch, rf, [("lm_head", 151936, 5120)], seed=914)[0]
    rows = []
    for m in (1, 8):
        x = torch.randn(m, 5120, device="cuda").half()
        y = torch.empty(m, 151936, device="cuda", dtype=torch.float16)
        us = per_launch_us(torch, lambda c: rf.linear_into(x, c[3], c[4], None, y), [head], 10)
        # greedy decode: the token ids, by the fused-argmax launch, and by the logits
        # launch followed by torch.argmax
        us_am = per_launch_us(torch, lambda c: rf.linear_argmax(x, c[3], c[4]), [head], 10)
        us_two = per_launch_us(torch, lambda c: (rf.linear_into(x, c[3], c[4], None, y),
                                                  y.argmax(-1)), [head], 10)
        rows.append({"M": m, "us": round(us, 1),
                     "GBps": round(nbytes(m, 151936, 5120) / (us * 1e-6) / 1e9, 1),
                     "argmax_fused_us": round(us_am, 1), "logits_then_argmax_us": round(us_two, 1)})
    out["cfg2_lm_head"] = rows
    del head
    torch.cuda.empty_cache()
    # cfg4: Qwen3-VL-32B projections at M in {1, 32, 512}, four layer copies (1.96 GB):
    # every projection's copies together exceed the 256 MB Infinity Cache (two
    # copies of a 131 MB gate/up/down weight would mostly be served from it)
    copies = [make_layer(torch, rf, QWEN3_VL_32B, seed=940 + c) for c in range(4)]
    rows = []
    for m in (1, 32, 512):
        x = torch.randn(m, 25600, device="cuda").half()
        for idx, (name, n, k) in enumerate(QWEN3_VL_32B):
            y = torch.empty(m, n, device="cuda", dtype=torch.float16)
            cs = [c[idx] for c in copies]
            xx = x[:, :k]
            us = per_launch_us(torch, lambda c: rf.linear_into(xx, c[3], c[4], None, y), cs,
                               20 if m < 512 else 6)
            kern = "gemv" if rf.select_kernel(m, n, k) == rf.KERNEL_GEMV else "gemm"
            r = {"M": m, "proj": name, "N": n, "K": k, "us": round(us, 2), "kernel": kern,
                 "GBps": round(nbytes(m, n, k) / (us * 1e-6) / 1e9, 1)}
            if kern == "gemm":
                r["TFLOPs"] = round(2 * m * n * k / (us * 1e-6) / 1e12, 1)
            rows.append(r)
        xx = x[:, :5120]
        for name, idxs in (("qkv", (0, 1, 2)), ("gate_up", (4, 5))):
            cs = [[c[i] for i in idxs] for c in copies]
            us = per_launch_us(torch, lambda c: rf.linear_multi(xx, [p[3] for p in c],
                                                                [p[4] for p in c]),
                               cs, 20 if m < 512 else 6)
            n = sum(QWEN3_VL_32B[i][1] for i in idxs)
            b = sum(nbytes(m, QWEN3_VL_32B[i][1], 5120) - 2 * m * 5120 for i in idxs) + 2 * m * 5120
            kern = "gemv" if rf.select_kernel(m, n, 5120) == rf.KERNEL_GEMV else "gemm"
            r = {"M": m, "proj": name, "N": n, "K": 5120, "us": round(us, 2),
                 "kernel": kern + " (one launch)", "GBps": round(b / (us * 1e-6) / 1e9, 1)}
            if kern == "gemm":
                r["TFLOPs"] = round(2 * m * n * 5120 / (us * 1e-6) / 1e12, 1)
            rows.append(r)
    out["cfg4_vl32b"] = rows
    del copies
    torch.cuda.empty_cache()
    out["w4a16"] = bench_w4a16(torch, rf)
    return out


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
                             "us": round(us, 2), "GBps": round(b / (us * 1e-6) / 1e9, 1)})
            rows.append({"group_size": gs, "M": m, "proj": "layer (7 launches)",
                         "us": round(step_us, 2),
                         "GBps": round(step_bytes / (step_us * 1e-6) / 1e9, 1)})
        if gs in (0, 32):
            x = torch.randn(PREFILL_M, 12288, device="cuda").half()
            for idx in (4, 6):  # gate (12288x4096) and down (4096x12288)
                name, n, k = QWEN3_8B[idx]
                xx = x[:, :k]
                us = per_launch_us(torch, lambda c: rf.linear_w4a16(xx, c[3], c[4]),
                                   [layer[idx] for layer in copies], 6)
                rows.append({"group_size": gs, "M": PREFILL_M, "proj": name, "N": n, "K": k,
                             "us": round(us, 1),
                             "TFLOPs": round(2 * PREFILL_M * n * k / (us * 1e-6) / 1e12, 1)})
        del copies
        torch.cuda.empty_cache()
    return rows


def cpu_baseline(budget_s=12.0):
    """Reference CPU path (oracle restatement: fp16 dequant, fp32-accumulate GEMM,
    fp16 round) over cfg1's seven projections at M=1, on the host cores."""
    import numpy as np

    sys.path.insert(0, ROOT)
    from oracle import w8a16 as o

    rng = np.random.default_rng(0)
    layer = []
    for name, n, k in QWEN3_8B:
        q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
        s = (rng.random(n).astype(np.float32) * 1e-3 + 1e-4).astype(np.float16)
        layer.append((q, s))
    x = o.make_activation(1, 1, 12288)
    t_deq = t_mm = 0.0
    passes = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s or passes == 0:
        for q, s in layer:
            a = time.perf_counter()
            w16 = o.dequantize_linear_per_channel(q, s)
            b = time.perf_counter()
            o.cpu_path(x[:, :q.shape[1]], q, s, w16=w16)
            c = time.perf_counter()
            t_deq += b - a
            t_mm += c - b
        passes += 1
    layer_bytes = sum(nbytes(1, n, k) for _, n, k in QWEN3_8B)
    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(layer_bytes * passes / t_mm / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"cfg1 Qwen3-8B layer, 7 projections at M=1, {passes} passes "
                   f"(~{budget_s:.0f} s); value = GEMM on a cached fp16 dequantized "
                   f"weight (the reference caches its dequantized lm_head); "
                   f"dequant+GEMM = {layer_bytes * passes / (t_mm + t_deq) / 1e9:.3f} GB/s"),
        "cpu_model": model,
        "dequant_s_per_layer": round(t_deq / passes, 4),
        "gemm_s_per_layer": round(t_mm / passes, 4),
    }


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
    log("decode (cfg1)...")
    dec = bench_decode(torch, rf, args.steps, args.warmup)
    log(f"decode: {dec['GBps']:.1f} GB/s ({dec['avg_launch_us']:.2f} us/launch, q/k/v and "
        f"gate/up fused); one launch per projection: {dec['per_op_GBps']:.1f} GB/s")
    env = read_envelope(torch, args.steps, args.warmup)
    if env:
        log(f"read envelope of the same 12 launches: {env['GBps']:.1f} GB/s")
    pre = None
    if not args.no_prefill:
        log("prefill (cfg3)...")
        pre = bench_prefill(torch, rf, max(10, args.steps // 2), args.warmup)
        log(f"prefill: {pre['TFLOPs']:.1f} TFLOP/s (gate/up fused); one launch per "
            f"projection: {pre['per_op_TFLOPs']:.1f} TFLOP/s")
    extra = None
    if not args.no_extra:
        log("configs 0, 2, 4...")
        extra = bench_other_configs(torch, rf)
    cpu = None
    if not args.no_cpu:
        log("cpu baseline...")
        cpu = cpu_baseline()
        log(f"cpu: {cpu['value']} GB/s on {cpu['cores']} threads")

    achieved = dec["avg_bytes_per_launch"] / (dec["avg_launch_us"] * 1e-6) / 1e9
    traffic = measured_traffic()
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
            "per_M_GBps": dec["per_M_GBps"],
            "launch": ("per M: q/k/v in one linear_multi launch, o, gate/up in one "
                       "linear_multi launch, down (12 launches per step); eager torch-op "
                       "launches on one stream"),
            "per_op_GBps": round(dec["per_op_GBps"], 1),
            "per_op_ms_per_step": round(dec["per_op_ms_per_step"], 4),
            "per_op_note": "the same step as 21 single-projection launches",
        },
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
            "launch": ("gate/up in one linear_multi launch, then down (2 launches per step); "
                       f"timed after {pre['settle_steps']} untimed steps (>= "
                       f"{PREFILL_SETTLE_S:.2f} s) bring the GPU clock to its sustained level"),
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
            "what": ("the decode step's 12 launches with the GEMV replaced by a plain "
                     "non-temporal streaming read of the same byte counts (rotated buffers, "
                     "eager, same stream and timer): the rate this launch structure allows"),
        },
        "cpu_baseline": cpu,
        "decode_per_launch": dec["per_launch"],
        "other_configs": extra,
    }
    if traffic:
        log(json.dumps({"traffic_source": traffic}))
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
