"""Write the committed golden fixtures for the W8A16 path.

Run from the repository root:  python tests/golden/make_golden.py

Each fixture holds a seed, the sha256 of the inputs that seed generates with
the oracle's portable generator (SplitMix64 + Box-Muller), and the expected
outputs:
  * y_cpu  -- fp16, from torch.nn.functional.linear on the CPU over the fp16
              dequantized weight: the literal reference CPU path
              (adapters/qwen3.py:617-623; bias added in fp16 afterwards as in
              src/ops/rpu_linear.cpp:156-159);
  * y_star -- the fp64 oracle y* = f64(x).(f64(s) f64(q))^T (+ b), stored as fp64.
The quantized weight is produced by the oracle's quantizer, itself pinned by
the reference KAT (tests/test_quantization.py:14-29); its sha256 is stored
too, so a drift in either the generator or the quantizer is caught.

Inputs are not stored (they are regenerated from the seed); the fixtures are
small enough to commit (a few tens of KB, compressed).
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import w8a16 as o  # noqa: E402

OUT = Path(__file__).resolve().parent

# (name, M list, N, K, bias, outlier_frac, rms_normalize)
CASES = [
    ("cfg0_like_n80_k136", [1, 3, 16, 33, 64], 80, 136, False, 0.0, False),
    ("bias_n48_k256", [1, 5, 17], 48, 256, True, 0.0, False),
    ("outlier_n33_k512", [2, 31, 65], 33, 512, False, 0.01, False),
    ("rmsnorm_n128_k64", [1, 8], 128, 64, False, 0.0, True),
]
SEED = 0x5EED_0001


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def inputs(name: str, m: int, n: int, k: int, bias: bool, outlier: float, rmsn: bool):
    w = o.make_weight(o.derive_seed(SEED, name, "w"), n, k)
    q, s = o.quantize_linear_per_channel(w)
    x = o.make_activation(o.derive_seed(SEED, name, "x", m), m, k, rms_normalize=rmsn,
                          outlier_frac=outlier)
    b = (o.normal(o.derive_seed(SEED, name, "b"), (n,)) * 0.1).astype(np.float16) if bias else None
    return x, q, s, b


def torch_cpu_path(x, q, s, b):
    w16 = (torch.from_numpy(q).to(torch.float32) * torch.from_numpy(s).to(torch.float32)[:, None]
           ).to(torch.float16)
    y = torch.nn.functional.linear(torch.from_numpy(x), w16)
    if b is not None:
        y = y + torch.from_numpy(b)
    return y.numpy()


def main() -> None:
    for name, ms, n, k, bias, outlier, rmsn in CASES:
        rec = {"seed": np.uint64(SEED), "N": n, "K": k, "M_list": np.array(ms),
               "bias": bias, "outlier_frac": outlier, "rms_normalize": rmsn}
        for m in ms:
            x, q, s, b = inputs(name, m, n, k, bias, outlier, rmsn)
            rec[f"sha_x_{m}"] = sha(x)
            rec[f"y_cpu_{m}"] = torch_cpu_path(x, q, s, b)
            rec[f"y_star_{m}"] = o.oracle_fp64(x, q, s, b)
        rec["sha_q"] = sha(q)
        rec["sha_s"] = sha(s)
        if b is not None:
            rec["sha_b"] = sha(b)
        np.savez_compressed(OUT / f"{name}.npz", **rec)
        print(f"wrote {name}.npz")


if __name__ == "__main__":
    main()
