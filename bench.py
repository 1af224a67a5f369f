"""Benchmark of the W8A16 linear on one MI355X.

Headline (`value`): decode GB/s on BASELINE config 1 -- a Qwen3-8B decoder
layer's seven W8A16 projections (q, k, v, o, gate, up, down) at batch
M in {1, 4, 16}.  One step = the 21 launches (7 projections x 3 batch sizes),
each pass over a different copy of the layer's weights (4 copies, 772 MB,
rotated so the 256 MB Infinity Cache never serves a repeat).  Inputs are
synthetic (weights N(0, 0.02) quantized per channel, activations N(0, 1))
and resident in HBM before the timed region.

value = sum of algorithmic bytes over the timed steps / wall time of the steps,
with bytes per launch B = N*K + 2N + 2MK + 2MN (int8 weights, fp16 scales,
fp16 activations and outputs).  The same line carries:
  * roofline          -- the decode GEMV kernel: algorithmic bytes per launch /
                         average launch duration (HIP events on the launch
                         stream over the timed region) vs the 8 TB/s HBM peak;
  * prefill           -- BASELINE config 3 (Qwen3-8B MLP prefill, M=2048) in
                         TFLOP/s vs the 2.5166 PFLOP/s dense FP16 MFMA peak;
  * cpu_baseline      -- the CPU restatement of the reference's
                         dequantize-then-matmul path (oracle, numpy/BLAS on all
                         host cores) on a bounded sample of config 1, M=1.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

HBM_PEAK_GBS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2516.6
METRIC = "W8A16 linear: decode GB/s (% HBM peak) + prefill TFLOP/s (% MFMA peak)"

QWEN3_8B = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
            ("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288)]
DECODE_M = (1, 4, 16)
LAYER_COPIES = 4
PREFILL = [("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288)]
PREFILL_M = 2048


def nbytes(m, n, k, bias=False):
    return n * k + 2 * n + 2 * m * k + 2 * m * n + (2 * n if bias else 0)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_layer(torch, rf, specs, seed):
    layer = []
    for i, (name, n, k) in enumerate(specs):
        g = torch.Generator(device="cuda").manual_seed(seed * 100 + i)
        w = torch.randn(n, k, generator=g, device="cuda", dtype=torch.float32) * 0.02
        q, s = rf.quantize_linear_per_channel(w)
        del w
        layer.append((name, n, k, rf.pack_weight(q), s))
        del q
    return layer


def bench_decode(torch, rf, steps, warmup):
    layers = [make_layer(torch, rf, QWEN3_8B, seed=c) for c in range(LAYER_COPIES)]
    xs = {m: torch.randn(m, 12288, device="cuda").half() for m in DECODE_M}
    outs = {(m, n): torch.empty(m, n, device="cuda", dtype=torch.float16)
            for m in DECODE_M for _, n, _ in QWEN3_8B}
    stream = torch.cuda.current_stream()

    def step(i):
        for j, m in enumerate(DECODE_M):
            layer = layers[(i * len(DECODE_M) + j) % LAYER_COPIES]
            for name, n, k, wp, s in layer:
                rf.linear_into(xs[m][:, :k], wp, s, None, outs[(m, n)])

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(steps):
        step(warmup + i)
    end.record(stream)
    end.synchronize()
    total_ms = start.elapsed_time(end)
    launches = steps * len(DECODE_M) * len(QWEN3_8B)
    step_bytes = sum(nbytes(m, n, k) for m in DECODE_M for _, n, k in QWEN3_8B)

    # Per-projection launch durations: events bracket each launch on its stream.
    per = {}
    reps = max(10, steps)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(reps * len(DECODE_M) * len(QWEN3_8B))]
    idx = 0
    for r in range(reps):
        for j, m in enumerate(DECODE_M):
            layer = layers[(r * len(DECODE_M) + j) % LAYER_COPIES]
            for name, n, k, wp, s in layer:
                a, b = ev[idx]
                a.record(stream)
                rf.linear_into(xs[m][:, :k], wp, s, None, outs[(m, n)])
                b.record(stream)
                per.setdefault((m, name, n, k), []).append((a, b))
                idx += 1
    torch.cuda.synchronize()
    rows = []
    for (m, name, n, k), lst in per.items():
        ts = sorted(a.elapsed_time(b) for a, b in lst)
        med = ts[len(ts) // 2] * 1e-3
        rows.append({"M": m, "proj": name, "N": n, "K": k, "us_median": med * 1e6,
                     "GBps": nbytes(m, n, k) / med / 1e9,
                     "kernel": "gemv" if rf.select_kernel(m, n, k) == rf.KERNEL_GEMV else "gemm"})
    kern_bytes = sum(nbytes(r["M"], r["N"], r["K"]) for r in rows)
    kern_time = sum(r["us_median"] * 1e-6 for r in rows)
    per_m = {}
    for m in DECODE_M:
        sel = [r for r in rows if r["M"] == m]
        per_m[str(m)] = round(sum(nbytes(m, r["N"], r["K"]) for r in sel)
                              / sum(r["us_median"] * 1e-6 for r in sel) / 1e9, 1)
    del layers
    return {
        "value_GBps": step_bytes * steps / (total_ms * 1e-3) / 1e9,
        "ms_per_step": total_ms / steps,
        "launches": launches,
        "kernel_GBps": kern_bytes / kern_time / 1e9,
        "kernel_avg_us": kern_time / len(rows) * 1e6,
        "kernel_avg_bytes": kern_bytes / len(rows),
        "per_M_GBps": per_m,
        "per_launch": rows,
    }


def bench_prefill(torch, rf, steps, warmup):
    copies = [make_layer(torch, rf, PREFILL, seed=50 + c) for c in range(2)]
    x = torch.randn(PREFILL_M, 12288, device="cuda").half()
    outs = {n: torch.empty(PREFILL_M, n, device="cuda", dtype=torch.float16) for _, n, _ in PREFILL}
    stream = torch.cuda.current_stream()

    def step(i):
        for name, n, k, wp, s in copies[i % 2]:
            rf.linear_into(x[:, :k], wp, s, None, outs[n])

    for i in range(max(2, warmup)):
        step(i)
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for i in range(steps):
        step(i)
    b.record(stream)
    b.synchronize()
    ms = a.elapsed_time(b)
    flops = sum(2 * PREFILL_M * n * k for _, n, k in PREFILL) * steps
    tflops = flops / (ms * 1e-3) / 1e12
    launches = steps * len(PREFILL)
    return {"TFLOPs": tflops, "ms_per_step": ms / steps, "avg_launch_us": ms * 1e3 / launches,
            "flops_per_launch": flops / launches}


def cpu_baseline(budget_s=12.0):
    """Reference CPU path (oracle restatement: fp16 dequant, fp32-accumulate GEMM,
    fp16 round) over cfg1's seven projections at M=1, on all host cores."""
    import numpy as np

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
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
                   f"weight; dequant+GEMM = {layer_bytes * passes / (t_mm + t_deq) / 1e9:.3f} GB/s"),
        "cpu_model": model,
        "dequant_s_per_layer": round(t_deq / passes, 4),
        "gemm_s_per_layer": round(t_mm / passes, 4),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-prefill", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build runs the W8A16 path on a single "
              "MI355X (no collectives); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    import rhinoforge_amd as rf

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    torch.cuda.synchronize()
    log(f"device: {torch.cuda.get_device_name(0)}")

    log("decode (cfg1)...")
    dec = bench_decode(torch, rf, args.steps, args.warmup)
    log(f"decode: {dec['value_GBps']:.1f} GB/s, kernel {dec['kernel_GBps']:.1f} GB/s")
    pre = None
    if not args.no_prefill:
        log("prefill (cfg3)...")
        pre = bench_prefill(torch, rf, max(5, args.steps // 5), args.warmup)
        log(f"prefill: {pre['TFLOPs']:.1f} TFLOP/s")
    cpu = None
    if not args.no_cpu:
        log("cpu baseline...")
        cpu = cpu_baseline()
        log(f"cpu: {cpu['value']} GB/s on {cpu['cores']} threads")

    achieved = dec["kernel_GBps"]
    line = {
        "metric": METRIC,
        "value": round(dec["value_GBps"], 1),
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
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "w8a16_gemv_kernel",
            "avg_launch_us": round(dec["kernel_avg_us"], 3),
            "avg_bytes_per_launch": round(dec["kernel_avg_bytes"]),
        },
        "prefill": None if pre is None else {
            "workload": "cfg3: Qwen3-8B MLP prefill M=2048 (gate, up, down)",
            "value": round(pre["TFLOPs"], 1),
            "unit": "TFLOP/s",
            "roofline": {"bound": "mfma", "achieved": round(pre["TFLOPs"], 1),
                         "peak": MFMA_FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(pre["TFLOPs"] / MFMA_FP16_PEAK_TFLOPS, 4),
                         "kernel": "w8a16_gemm_kernel",
                         "avg_launch_us": round(pre["avg_launch_us"], 2)},
        },
        "cpu_baseline": cpu,
        "host": platform.node(),
    }
    log(json.dumps({"per_launch": dec["per_launch"]}))
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
