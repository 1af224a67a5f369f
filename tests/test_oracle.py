"""Pin the CPU oracle (oracle/w8a16.py) before trusting it.

Checks come from the reference's own KAT (tests/test_quantization.py:14-29),
closed forms, library routines (torch's CPU ops, which the reference calls),
brute force on tiny inputs, and planted mistakes that must be caught.
"""
from __future__ import annotations

import hashlib
import itertools
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import w8a16 as o

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---------------------------------------------------------------- quantizer
def test_reference_kat_matrix():
    """tests/test_quantization.py:14-29 of the reference, plus the explicit values."""
    w = np.array([[-2.0, -0.5, 0.5, 2.0], [-0.25, 0.0, 0.25, 0.5]], np.float32)
    q, s = o.quantize_linear_per_channel(w)
    assert q.dtype == np.int8 and s.dtype == np.float16 and s.shape == (2,)
    assert q.min() >= -128 and q.max() <= 127
    restored = o.dequantize_linear_per_channel(q, s).astype(np.float64)
    cos = (restored * w).sum(1) / (np.linalg.norm(restored, axis=1) * np.linalg.norm(w, axis=1))
    assert cos.min() > 0.999
    assert s.view(np.uint16).tolist() == [0x2408, 0x1C08]
    assert q.tolist() == [[-127, -32, 32, 127], [-64, 0, 64, 127]]


def test_round_half_even_and_cast_before_amax():
    # Row scale: amax = 1.27 -> s = fp16(0.01) ; entries chosen to land on .5 quotients
    s = np.float16(1.27 / 127)
    s32 = np.float32(s)
    halves = np.array([2.5, 3.5, -2.5, -3.5, 0.5, 1.5], np.float64)
    row = (halves * float(s32)).astype(np.float32)
    w = np.concatenate([row, [np.float32(1.27)]])[None, :].astype(np.float32)
    q, sc = o.quantize_linear_per_channel(w)
    quot = w.astype(np.float16).astype(np.float32) / np.float32(sc[0])
    # Ties to even where the fp32 quotient is exactly .5
    for qi, v in zip(q[0], quot[0]):
        if float(v) - np.floor(float(v)) == 0.5:
            assert qi % 2 == 0, (qi, v)
    # fp16 cast before amax: 1.0001 rounds to 1.0 in fp16 -> amax is 1.0
    q2, s2 = o.quantize_linear_per_channel(np.array([[1.0001, 0.5]], np.float32))
    assert s2[0] == np.float16(np.float32(1.0) / np.float32(127))
    assert q2[0, 0] == 127


def test_invariants_zero_row_and_range():
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((50, 300)) * 0.02).astype(np.float32)
    w[7] = 0.0
    w[9, :] = 1e-12  # below fp16 resolution: casts to 0
    q, s = o.quantize_linear_per_channel(w)
    assert np.abs(q.astype(int)).max() <= 127
    for n in range(50):
        if n in (7, 9):
            assert s[n] == np.float16(2.0 ** -14) and (q[n] == 0).all()
        else:
            assert np.abs(q[n].astype(int)).max() == 127


def _torch_quant(w):
    """The reference's quantizer steps written directly as torch ops."""
    w16 = torch.from_numpy(w).to(torch.float16)
    amax = w16.to(torch.float32).abs().amax(dim=1)
    sc = (amax / 127.0).to(torch.float16).clamp_min(torch.finfo(torch.float16).tiny)
    q = torch.round(w16.to(torch.float32) / sc.to(torch.float32).unsqueeze(1)).clamp_(-128, 127)
    return q.to(torch.int8).numpy(), sc.numpy()


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_quantizer_bit_exact_vs_torch_ops(seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((97, 513)) * 0.02).astype(np.float32)
    w[3] *= 1000.0  # large row
    w[4] *= 1e-4    # tiny row: scale near the fp16 normal limit
    q1, s1 = o.quantize_linear_per_channel(w)
    q2, s2 = _torch_quant(w)
    assert (q1 == q2).all()
    assert (s1.view(np.uint16) == s2.view(np.uint16)).all()


def test_bits4_range():
    rng = np.random.default_rng(3)
    w = rng.standard_normal((8, 64)).astype(np.float32)
    q, _ = o.quantize_linear_per_channel(w, bits=4)
    assert q.min() >= -8 and q.max() <= 7 and np.abs(q).max() == 7


def test_quantizer_rejects_bad_input():
    with pytest.raises(ValueError):
        o.quantize_linear_per_channel(np.zeros(4, np.float32))
    with pytest.raises(ValueError):
        o.quantize_linear_per_channel(np.zeros((2, 2), np.float32), bits=5)


# ---------------------------------------------------------------- dequant
def test_dequant_forms_equal_rounded_exact_product():
    q = np.arange(-128, 128, dtype=np.int8)[None, :].repeat(6, 0)
    s = np.array([2.0 ** -14, 0.0157470703125, 0.003936767578125, 1.0, 3.140625, 511.0],
                 np.float16)
    exact = s.astype(np.float64)[:, None] * q.astype(np.float64)
    a = o.dequantize_linear_per_channel(q, s)
    b = o.dequantize_fp32_then_fp16(q, s)
    assert (a.view(np.uint16) == b.view(np.uint16)).all()
    assert (a == exact.astype(np.float16)).all()  # RN of the exact product
    t = (torch.from_numpy(s).unsqueeze(1) * torch.from_numpy(q).to(torch.float16)).numpy()
    assert (a.view(np.uint16) == t.view(np.uint16)).all()


# ---------------------------------------------------------------- CPU path
def _case(m, n, k, seed=0, bias=False):
    w = o.make_weight(o.derive_seed(seed, "w"), n, k)
    q, s = o.quantize_linear_per_channel(w)
    x = o.make_activation(o.derive_seed(seed, "x", m), m, k)
    b = (o.normal(o.derive_seed(seed, "b"), (n,)) * 0.1).astype(np.float16) if bias else None
    return x, q, s, b


@pytest.mark.parametrize("m,n,k,bias", [(1, 64, 128, False), (7, 96, 256, True), (33, 40, 72, False)])
def test_cpu_path_matches_torch_linear(m, n, k, bias):
    x, q, s, b = _case(m, n, k, bias=bias)
    y = o.cpu_path(x, q, s, b)
    w16 = torch.from_numpy(o.dequantize_linear_per_channel(q, s))
    yt = torch.nn.functional.linear(torch.from_numpy(x), w16)
    if b is not None:
        yt = yt + torch.from_numpy(b)
    yt = yt.numpy()
    # Same fp32-accumulate / fp16-round contract; summation order may differ by 1 ulp.
    ulp = np.spacing(np.abs(yt).astype(np.float16)).astype(np.float32)
    assert (np.abs(y.astype(np.float32) - yt.astype(np.float32)) <= ulp).all()


def test_cpu_path_unit_vector_selects_column():
    x, q, s, _ = _case(1, 48, 64)
    for k in (0, 17, 63):
        e = np.zeros((1, 64), np.float16)
        e[0, k] = 1.0
        y = o.cpu_path(e, q, s)
        assert (y[0] == o.dequantize_linear_per_channel(q, s)[:, k]).all()
        ys = o.oracle_fp64(e, q, s)
        assert np.allclose(ys[0], s.astype(np.float64) * q[:, k], rtol=0, atol=0)


def test_cpu_path_flattens_leading_dims():
    x, q, s, _ = _case(6, 32, 64)
    y = o.cpu_path(x.reshape(2, 3, 64), q, s)
    assert y.shape == (2, 3, 32)
    assert (y.reshape(6, 32) == o.cpu_path(x, q, s)).all()


# ---------------------------------------------------------------- fp64 oracle
def test_oracle_brute_force_tiny():
    x, q, s, b = _case(3, 16, 32, bias=True)
    ref = np.zeros((3, 16))
    for i, j, kk in itertools.product(range(3), range(16), range(32)):
        ref[i, j] += float(x[i, kk]) * float(s[j]) * float(q[j, kk])
    ref += b.astype(np.float64)
    assert np.allclose(o.oracle_fp64(x, q, s, b), ref, rtol=1e-12, atol=1e-12)


def test_oracle_identity_blocks():
    n = k = 32
    q = np.zeros((n, k), np.int8)
    q[np.arange(n), np.arange(k)] = 127
    s = np.full(n, 0.5, np.float16)
    x = o.make_activation(5, 4, k)
    assert (o.oracle_fp64(x, q, s) == x.astype(np.float64) * 63.5).all()


def test_oracle_rows_subset():
    x, q, s, _ = _case(10, 16, 64)
    rows = np.array([0, 3, 9])
    assert (o.oracle_fp64(x, q, s, rows=rows) == o.oracle_fp64(x, q, s)[rows]).all()


# ---------------------------------------------------------------- tolerance checker
def test_check_tolerance_accepts_cpu_path():
    x, q, s, _ = _case(4, 256, 512)
    rep = o.check_tolerance(o.cpu_path(x, q, s), o.cpu_path(x, q, s), o.oracle_fp64(x, q, s))
    assert rep.ok, str(rep)


@pytest.mark.parametrize("mistake", ["sign", "transpose", "no_scale", "dropped_k", "wrong_row"])
def test_check_tolerance_catches_planted_mistakes(mistake):
    """A plausible bug planted in a CPU copy of the computation must fail."""
    x, q, s, _ = _case(4, 64, 64)
    y_cpu = o.cpu_path(x, q, s)
    y_star = o.oracle_fp64(x, q, s)
    w = s.astype(np.float32)[:, None] * q.astype(np.float32)
    x32 = x.astype(np.float32)
    if mistake == "sign":
        bad = -(x32 @ w.T)
    elif mistake == "transpose":
        bad = x32 @ w  # square N == K: runs, wrong answer
    elif mistake == "no_scale":
        bad = x32 @ q.astype(np.float32).T
    elif mistake == "dropped_k":
        bad = x32[:, :-8] @ w[:, :-8].T
    else:
        bad = (x32 @ w.T)[::-1]
    assert not o.check_tolerance(bad.astype(np.float16), y_cpu, y_star).ok


def test_check_tolerance_rejects_nonfinite():
    x, q, s, _ = _case(2, 32, 64)
    y = o.cpu_path(x, q, s).copy()
    y[0, 0] = np.float16(np.inf)
    assert not o.check_tolerance(y, o.cpu_path(x, q, s), o.oracle_fp64(x, q, s)).ok


# ---------------------------------------------------------------- generator
def test_splitmix64_known_values():
    # SplitMix64 reference outputs for seed 0 (Vigna's splitmix64.c):
    assert [int(v) for v in o.splitmix64(0, 3)] == [
        0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_normal_moments_and_determinism():
    a = o.normal(7, (200_000,))
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1.0) < 0.01
    assert (a == o.normal(7, (200_000,))).all()
    x = o.make_activation(9, 3, 5120, outlier_frac=0.01)
    big = np.abs(x.astype(np.float32)).max(axis=0) > 8
    assert 30 <= big.sum() <= 60  # 51 outlier channels x20 (a few may be small draws)


# ---------------------------------------------------------------- golden fixtures
def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _regen(name, rec, m):
    k, n = int(rec["K"]), int(rec["N"])
    seed = int(rec["seed"])
    w = o.make_weight(o.derive_seed(seed, name, "w"), n, k)
    q, s = o.quantize_linear_per_channel(w)
    x = o.make_activation(o.derive_seed(seed, name, "x", m), m, k,
                          rms_normalize=bool(rec["rms_normalize"]),
                          outlier_frac=float(rec["outlier_frac"]))
    b = ((o.normal(o.derive_seed(seed, name, "b"), (n,)) * 0.1).astype(np.float16)
         if bool(rec["bias"]) else None)
    return x, q, s, b


@pytest.mark.parametrize("path", sorted(GOLDEN.glob("*.npz")), ids=lambda p: p.stem)
def test_golden_fixtures_regenerate_and_match_oracle(path):
    rec = np.load(path)
    name = path.stem
    for m in rec["M_list"]:
        m = int(m)
        x, q, s, b = _regen(name, rec, m)
        assert _sha(x) == str(rec[f"sha_x_{m}"])
        assert _sha(q) == str(rec["sha_q"]) and _sha(s) == str(rec["sha_s"])
        y_cpu = rec[f"y_cpu_{m}"]
        y = o.cpu_path(x, q, s, b)
        ulp = np.spacing(np.abs(y_cpu).astype(np.float16)).astype(np.float32)
        assert (np.abs(y.astype(np.float32) - y_cpu.astype(np.float32)) <= ulp).all()
        assert np.allclose(o.oracle_fp64(x, q, s, b), rec[f"y_star_{m}"], rtol=1e-12, atol=1e-12)
        assert o.check_tolerance(y_cpu, y_cpu, rec[f"y_star_{m}"]).ok
