"""GPU parity of the W8A16 kernels against the CPU oracle (MI355X only).

Bar: max|y - y_cpu| <= 1e-2 * rms(y_cpu) and cosine(y, y*) >=
0.9999 against the fp64 oracle, outputs finite.  y_cpu is the reference's
dequantize-then-matmul CPU path (oracle.w8a16.cpu_path), y* the fp64 oracle.
Exact-arithmetic cases (one-hot activations) are compared bit for bit.
"""
from __future__ import annotations

import ctypes
import hashlib
from pathlib import Path

import numpy as np
import pytest
import torch

import rhinoforge_amd as rf
from rhinoforge_amd import capi
from oracle import w8a16 as o
import planner_cases
from conftest import fresh_hip_stream

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = Path(__file__).resolve().parent / "golden"
KERNELS = {"auto": rf.KERNEL_AUTO, "gemv": rf.KERNEL_GEMV, "gemm": rf.KERNEL_GEMM}


def _say(*a):
    print(*a, flush=True)


def _to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


_WEIGHTS: dict = {}


def make_weights(n, k, seed):
    """(q, s) numpy.  Small weights come from the oracle's portable generator and
    quantizer; large ones are drawn N(0, 0.02) on the GPU (torch, seeded) and
    quantized there by the package quantizer (bit-exact with the oracle's, see
    test_host.py and test_gpu_quantizer_matches_oracle)."""
    key = (n, k, seed)
    if key not in _WEIGHTS:
        if n * k <= (1 << 22):
            q, s = o.quantize_linear_per_channel(o.make_weight(o.derive_seed(seed, "w", n, k), n, k))
        else:
            g = torch.Generator(device=DEV).manual_seed(o.derive_seed(seed, "w", n, k) & 0x7FFFFFFF)
            w = torch.randn(n, k, generator=g, device=DEV, dtype=torch.float32) * 0.02
            qd, sd = rf.quantize_linear_per_channel(w)
            q, s = qd.cpu().numpy(), sd.cpu().numpy()
            del w, qd, sd
        _WEIGHTS.clear()  # keep at most one large weight resident
        _WEIGHTS[key] = (q, s)
    return _WEIGHTS[key]


def make_case(m, n, k, seed, *, bias=False, outlier=0.0, rmsn=False):
    q, s = make_weights(n, k, seed)
    x = o.make_activation(o.derive_seed(seed, "x", m, k), m, k, rms_normalize=rmsn,
                          outlier_frac=outlier)
    b = (o.normal(o.derive_seed(seed, "b", n), (n,)) * 0.1).astype(np.float16) if bias else None
    return x, q, s, b


def run_gpu(x, q, s, b, kernel=rf.KERNEL_AUTO, packed=None):
    wp = packed if packed is not None else rf.pack_weight(_to_dev(q))
    y = rf.linear(_to_dev(x), wp, _to_dev(s), None if b is None else _to_dev(b), kernel=kernel)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def assert_parity(y, x, q, s, b, rows=None, label=""):
    xs = x if rows is None else x[rows]
    ys = y if rows is None else y[rows]
    y_cpu = o.cpu_path(xs, q, s, b)
    y_star = o.oracle_fp64(xs, q, s, b)
    rep = o.check_tolerance(ys, y_cpu, y_star)
    _say(f"  {label}: {rep}")
    assert rep.ok, f"{label}: {rep}"
    return rep


# ---------------------------------------------------------------- exactness
@pytest.mark.parametrize("kernel,m", [("gemv", 1), ("gemv", 16), ("gemv", 40), ("gemm", 130)])
def test_one_hot_rows_are_exact(kernel, m):
    """x[r] = e_{k_r}: y[r, n] = fp16(s[n] * q[n, k_r]) exactly (one product, no sum)."""
    n, k = 80, 200
    _say(f"one-hot {kernel} M={m} N={n} K={k}")
    rng = np.random.default_rng(m)
    q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    s = (rng.random(n) * 0.05 + 1e-3).astype(np.float16)
    ks = rng.integers(0, k, size=m)
    x = np.zeros((m, k), np.float16)
    x[np.arange(m), ks] = 1.0
    y = run_gpu(x, q, s, None, KERNELS[kernel])
    expect = o.dequantize_linear_per_channel(q, s)[:, ks].T
    assert (y.view(np.uint16) == expect.view(np.uint16)).all()


# ---------------------------------------------------------------- golden fixtures
def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.mark.parametrize("kernel", sorted(KERNELS))
@pytest.mark.parametrize("path", sorted(GOLDEN.glob("*.npz")), ids=lambda p: p.stem)
def test_golden_fixtures(path, kernel):
    rec = np.load(path)
    name, n, k, seed = path.stem, int(rec["N"]), int(rec["K"]), int(rec["seed"])
    w = o.make_weight(o.derive_seed(seed, name, "w"), n, k)
    q, s = o.quantize_linear_per_channel(w)
    b = ((o.normal(o.derive_seed(seed, name, "b"), (n,)) * 0.1).astype(np.float16)
         if bool(rec["bias"]) else None)
    packed = rf.pack_weight(_to_dev(q))
    for m in (int(v) for v in rec["M_list"]):
        if kernel == "gemv" and m > 64:
            continue
        x = o.make_activation(o.derive_seed(seed, name, "x", m), m, k,
                              rms_normalize=bool(rec["rms_normalize"]),
                              outlier_frac=float(rec["outlier_frac"]))
        assert _sha(x) == str(rec[f"sha_x_{m}"])
        _say(f"golden {name} {kernel} M={m}")
        y = run_gpu(x, q, s, b, KERNELS[kernel], packed)
        rep = o.check_tolerance(y, rec[f"y_cpu_{m}"], rec[f"y_star_{m}"])
        assert rep.ok, f"{name} M={m} {kernel}: {rep}"


# ---------------------------------------------------------------- BASELINE configs
def test_cfg0_qwen3_06b_decode():
    x, q, s, b = make_case(1, 3072, 1024, seed=0)
    packed = rf.pack_weight(_to_dev(q))
    for kern in ("auto", "gemv", "gemm"):
        _say(f"cfg0 {kern}")
        assert_parity(run_gpu(x, q, s, b, KERNELS[kern], packed), x, q, s, b, label=f"cfg0 {kern}")


QWEN3_8B = {"q": (4096, 4096), "k": (1024, 4096), "v": (1024, 4096), "o": (4096, 4096),
            "gate": (12288, 4096), "up": (12288, 4096), "down": (4096, 12288)}
QWEN3_VL_32B = {"q": (8192, 5120), "k": (1024, 5120), "v": (1024, 5120), "o": (5120, 8192),
                "gate": (25600, 5120), "up": (25600, 5120), "down": (5120, 25600)}


@pytest.mark.parametrize("m", [1, 4, 16])
def test_cfg1_qwen3_8b_decode_layer(m):
    for proj, (n, k) in QWEN3_8B.items():
        _say(f"cfg1 M={m} {proj} N={n} K={k}")
        x, q, s, b = make_case(m, n, k, seed=1)
        assert rf.select_kernel(m, n, k) == rf.KERNEL_GEMV
        assert_parity(run_gpu(x, q, s, b), x, q, s, b, label=f"cfg1 M={m} {proj}")


@pytest.mark.parametrize("m", [1, 32, 512])
def test_cfg4_qwen3_vl_32b_projections(m):
    """Every row of every projection against the CPU path (fp16 dequant, fp32
    BLAS on the host) and the fp64 oracle."""
    for proj, (n, k) in QWEN3_VL_32B.items():
        _say(f"cfg4 M={m} {proj} N={n} K={k}")
        x, q, s, b = make_case(m, n, k, seed=4, outlier=0.01)
        assert_parity(run_gpu(x, q, s, b), x, q, s, b, label=f"cfg4 M={m} {proj}")


@pytest.mark.parametrize("m", [1, 32, 512])
def test_cfg4_fused_launches_as_benched(m):
    """The fused Qwen3-VL-32B launches the bench times: q/k/v in one
    linear_multi launch and gate/up in one (at M = 32 the latter runs the
    32x256 tile across both projections); every row of every output against
    the CPU path and the fp64 oracle."""
    x = o.make_activation(o.derive_seed(4, "fused", m), m, 5120, outlier_frac=0.01)
    xd = _to_dev(x)
    for group in (("q", "k", "v"), ("gate", "up")):
        ws = [make_weights(*QWEN3_VL_32B[p], seed=40 + i) for i, p in enumerate(group)]
        # make_weights keeps one large weight resident: copy the small ones out
        ws = [(q.copy(), s.copy()) for q, s in ws]
        _say(f"cfg4 fused {'/'.join(group)} M={m}: "
             f"{capi.plan(m, [QWEN3_VL_32B[p][0] for p in group], 5120)['name']}")
        ys = rf.linear_multi(xd, [rf.pack_weight(_to_dev(q)) for q, _ in ws],
                             [_to_dev(s) for _, s in ws])
        torch.cuda.synchronize()
        for p, (q, s), y in zip(group, ws, ys):
            assert_parity(y.cpu().numpy(), x, q, s, None, label=f"cfg4 fused M={m} {p}")


def test_cfg3_qwen3_8b_prefill_mlp():
    """Each MLP projection alone, every row against the CPU path and the fp64 oracle."""
    m = 2048
    for proj in ("gate", "up", "down"):
        n, k = QWEN3_8B[proj]
        _say(f"cfg3 M={m} {proj} N={n} K={k}")
        x, q, s, b = make_case(m, n, k, seed=3)
        assert rf.select_kernel(m, n, k) == rf.KERNEL_GEMM
        assert_parity(run_gpu(x, q, s, b), x, q, s, b, label=f"cfg3 {proj} all rows")


def test_cfg3_prefill_step_as_benched():
    """The two launches bench.py times for cfg3: gate and up in one linear_multi
    launch reading x[:, :4096] of a [2048, 12288] activation buffer (row stride
    12288), then down over the whole buffer; every row of the three outputs
    against the CPU path and the fp64 oracle."""
    m = 2048
    xfull = o.make_activation(o.derive_seed(3, "bench-step"), m, 12288)
    xd = _to_dev(xfull)
    weights = {}
    for i, proj in enumerate(("gate", "up", "down")):
        n, k = QWEN3_8B[proj]
        weights[proj] = make_weights(n, k, seed=300 + i)
    packed = {p: (rf.pack_weight(_to_dev(q)), _to_dev(s)) for p, (q, s) in weights.items()}
    _say("cfg3 fused gate/up launch M=2048 N=2x12288 K=4096 ldx=12288")
    ys = rf.linear_multi(xd[:, :4096], [packed["gate"][0], packed["up"][0]],
                         [packed["gate"][1], packed["up"][1]])
    yd = rf.linear(xd, *packed["down"])
    torch.cuda.synchronize()
    for proj, y in zip(("gate", "up"), ys):
        q, s = weights[proj]
        assert_parity(y.cpu().numpy(), xfull[:, :4096], q, s, None, label=f"bench step {proj}")
    q, s = weights["down"]
    assert_parity(yd.cpu().numpy(), xfull, q, s, None, label="bench step down")


def _lm_head_weights():
    n, k = 151936, 5120
    g = torch.Generator(device=DEV).manual_seed(14)
    w = torch.randn(n, k, generator=g, device=DEV, dtype=torch.float32) * 0.02
    q, s = rf.quantize_linear_per_channel(w)
    del w
    return q, s


@pytest.mark.parametrize("m", [1, 8])
def test_cfg2_qwen3_14b_lm_head(m):
    _say(f"cfg2 lm_head M={m}")
    q_dev, s_dev = _lm_head_weights()
    q, s = q_dev.cpu().numpy(), s_dev.cpu().numpy()
    x = o.make_activation(o.derive_seed(2, "x", m), m, 5120, rms_normalize=True)
    y = run_gpu(x, q, s, None, packed=rf.pack_weight(q_dev))
    assert_parity(y, x, q, s, None, label=f"cfg2 M={m}")


def test_cfg2_lm_head_argmax_agreement_1000_rows():
    """Greedy-token agreement with the CPU path over 1000 seeded rows, with near-tie accounting
    (a disagreement counts as a tie when the fp64 oracle's top-2 gap is below the output's
    fp16 rounding, docs/validation_policy.md:124-128)."""
    _say("cfg2 argmax 1000 rows")
    q_dev, s_dev = _lm_head_weights()
    packed = rf.pack_weight(q_dev)
    x = o.make_activation(o.derive_seed(2, "argmax"), 1000, 5120, rms_normalize=True)
    y = rf.linear(_to_dev(x), packed, s_dev)  # M=1000: GEMM
    y8 = torch.cat([rf.linear(_to_dev(x[i:i + 8]), packed, s_dev) for i in range(0, 1000, 8)])
    torch.cuda.synchronize()
    # CPU path: fp16 dequantized weight, fp32 accumulation (adapters/qwen3.py:617-623)
    w16 = o.dequantize_fp32_then_fp16(q_dev.cpu().numpy(), s_dev.cpu().numpy())
    y_cpu = (x.astype(np.float32) @ w16.astype(np.float32).T).astype(np.float16)
    a_cpu = y_cpu.astype(np.float32).argmax(1)
    for label, yy in (("gemm M=1000", y), ("gemv M=8 batches", y8)):
        a_gpu = yy.float().argmax(1).cpu().numpy()
        bad = np.nonzero(a_gpu != a_cpu)[0]
        ties = 0
        for r in bad:
            v_g = float(y_cpu[r, a_gpu[r]])
            v_c = float(y_cpu[r, a_cpu[r]])
            if abs(v_c - v_g) <= 2 * float(np.spacing(np.float16(abs(v_c)))):
                ties += 1
        _say(f"  {label}: agree {1000 - len(bad)}/1000, near-ties {ties}")
        assert len(bad) - ties == 0


# ---------------------------------------------------------------- fused argmax (lm_head, greedy decode)
def _argmax_first(y):
    """Row argmax of fp16 logits, lowest index among equal values (torch.argmax's rule)."""
    return y.float().argmax(-1).to(torch.int32)


def _same_bits_or_nan(a, b):
    """Bitwise equality where NaN positions must match (NaN compares unequal to itself)."""
    return bool((a.isnan() == b.isnan()).all()) and torch.equal(a.nan_to_num(0.0), b.nan_to_num(0.0))


@pytest.mark.parametrize("m", [1, 8])
def test_linear_argmax_cfg2_lm_head(m):
    """cfg2 lm_head (151936 x 5120): the fused argmax equals the argmax of the op's own
    fp16 logits exactly, and the logits it optionally returns are the linear op's, bit for bit."""
    _say(f"linear_argmax cfg2 M={m}")
    q_dev, s_dev = _lm_head_weights()
    packed = rf.pack_weight(q_dev)
    x = _to_dev(o.make_activation(o.derive_seed(2, "amax", m), m, 5120, rms_normalize=True))
    idx = rf.linear_argmax(x, packed, s_dev)
    idx2, logits = rf.linear_argmax(x, packed, s_dev, return_logits=True)
    y = rf.linear(x, packed, s_dev)
    torch.cuda.synchronize()
    assert idx.dtype == torch.int32 and idx.shape == (m,)
    assert torch.equal(logits, y)
    assert torch.equal(idx, _argmax_first(y)), (idx, _argmax_first(y))
    assert torch.equal(idx2, idx)


def test_linear_argmax_agreement_1000_rows_with_cpu_path():
    """Greedy-token agreement of the fused argmax (batches of 8 rows) with the reference
    CPU path over 1000 seeded rows, with the same near-tie accounting as the logits test."""
    _say("linear_argmax 1000 rows")
    q_dev, s_dev = _lm_head_weights()
    packed = rf.pack_weight(q_dev)
    x = o.make_activation(o.derive_seed(2, "argmax"), 1000, 5120, rms_normalize=True)
    xd = _to_dev(x)
    a_gpu = torch.cat([rf.linear_argmax(xd[i:i + 8], packed, s_dev) for i in range(0, 1000, 8)])
    torch.cuda.synchronize()
    w16 = o.dequantize_fp32_then_fp16(q_dev.cpu().numpy(), s_dev.cpu().numpy())
    y_cpu = (x.astype(np.float32) @ w16.astype(np.float32).T).astype(np.float16)
    a_cpu = y_cpu.astype(np.float32).argmax(1)
    a_gpu = a_gpu.cpu().numpy()
    bad = np.nonzero(a_gpu != a_cpu)[0]
    ties = sum(1 for r in bad if abs(float(y_cpu[r, a_cpu[r]]) - float(y_cpu[r, a_gpu[r]]))
               <= 2 * float(np.spacing(np.float16(abs(float(y_cpu[r, a_cpu[r]]))))))
    _say(f"  fused argmax: agree {1000 - len(bad)}/1000, near-ties {ties}")
    assert len(bad) - ties == 0


def test_linear_argmax_ties_nan_and_repeats():
    """Equal maxima resolve to the lowest index; a NaN logit counts as the largest (torch.argmax's
    rule); -0 equals +0; repeated calls (the workspace keys are reset) and a bias all agree with
    argmax of the op's own logits."""
    n, k = 700, 512
    rng = np.random.default_rng(7)
    q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    s = (rng.random(n) * 0.01 + 1e-3).astype(np.float16)
    for dup in (650, 300, 5):  # identical channels: 5 must win over 300 and 650
        q[dup] = q[123]
        s[dup] = s[123]
    s[[5, 123, 300, 650]] = np.float16(0.05)  # and make them the largest by far
    packed, sd = rf.pack_weight(_to_dev(q)), _to_dev(s)
    x = o.make_activation(31, 6, k)
    x[:, :] = np.abs(x).astype(np.float16) * np.sign(q[123].astype(np.float32)).astype(np.float16)
    x[3] = 0.0                 # all logits +0 (bias none): index 0
    x[4, 7] = np.float16(np.nan)  # a NaN activation: every logit of row 4 is NaN -> index 0
    x[5] = -x[5]               # row 5: channel 123's group is now the smallest; plain argmax
    xd = _to_dev(x)
    idx, y = rf.linear_argmax(xd, packed, sd, return_logits=True)
    torch.cuda.synchronize()
    assert idx[0].item() == 5 and idx[1].item() == 5 and idx[2].item() == 5
    assert idx[3].item() == 0 and idx[4].item() == 0
    assert torch.equal(idx, _argmax_first(y.nan_to_num(nan=float("inf"))))
    b = _to_dev((o.normal(32, (n,)) * 0.1).astype(np.float16))
    for _ in range(3):
        i2, y2 = rf.linear_argmax(xd, packed, sd, b, return_logits=True)
        i3 = rf.linear_argmax(xd, packed, sd)
        torch.cuda.synchronize()
        assert _same_bits_or_nan(y2, rf.linear(xd, packed, sd, b))
        assert torch.equal(i2, _argmax_first(y2.nan_to_num(nan=float("inf"))))
        assert torch.equal(i3, idx)


@pytest.mark.parametrize("m,n,k", [(16, 1000, 8192), (40, 3000, 1024), (64, 2000, 640), (3, 100, 136),
                                   (1, 1000, 4096)])
def test_linear_argmax_planner_paths(m, n, k):
    """Split-K (the argmax runs in the last split's reduction), multi-row m-tiles, the
    LDS-staged x configuration and a K tail: index == argmax of the op's own logits."""
    _say(f"linear_argmax M={m} N={n} K={k}")
    x, q, s, b = make_case(m, n, k, seed=33, bias=True)
    packed = rf.pack_weight(_to_dev(q))
    xd, sd, bd = _to_dev(x), _to_dev(s), _to_dev(b)
    idx, y = rf.linear_argmax(xd, packed, sd, bd, return_logits=True)
    torch.cuda.synchronize()
    assert torch.equal(y, rf.linear(xd, packed, sd, bd, kernel=rf.KERNEL_GEMV))
    assert torch.equal(idx, _argmax_first(y))
    assert_parity(y.cpu().numpy(), x, q, s, b, label=f"argmax logits {m}x{n}x{k}")


def test_linear_argmax_capi_and_errors():
    """The C ABI entry point through ctypes (no logits), and the op's refusals."""
    m, n, k = 4, 5000, 1024
    x, q, s, _ = make_case(m, n, k, seed=34)
    packed = rf.pack_weight(_to_dev(q))
    xd, sd = _to_dev(x), _to_dev(s)
    lib = capi.load()
    ws_bytes = lib.rf_w8a16_workspace_bytes_argmax(m, n, k)
    assert ws_bytes > 0 and lib.rf_w8a16_workspace_bytes_argmax(65, n, k) == 0
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=DEV)
    idx = torch.full((m,), -1, dtype=torch.int32, device=DEV)
    for _ in range(2):
        st = lib.rf_w8a16_linear_argmax(xd.data_ptr(), k, packed.data_ptr(), capi.LAYOUT_TILE16X64,
                                        sd.data_ptr(), None, None, 0, idx.data_ptr(), m, n, k,
                                        ws.data_ptr(), ws_bytes,
                                        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        capi.check(st, "rf_w8a16_linear_argmax")
        torch.cuda.synchronize()
        assert torch.equal(idx, _argmax_first(rf.linear(xd, packed, sd)))
        assert int(ws[:capi.WS_COUNTER_BYTES].count_nonzero()) == 0  # counters left zero
    big = torch.zeros(65, k, dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError, match="at most 64 rows"):
        rf.linear_argmax(big, packed, sd)
    st = lib.rf_w8a16_linear_argmax(big.data_ptr(), k, packed.data_ptr(), capi.LAYOUT_TILE16X64,
                                    sd.data_ptr(), None, None, 0, idx.data_ptr(), 65, n, k,
                                    ws.data_ptr(), ws_bytes, None)
    assert st == capi.EKERNEL


# ---------------------------------------------------------------- edge cases
EDGE = [(1, 1, 8), (1, 17, 72), (2, 100, 136), (16, 16, 64), (17, 33, 520), (33, 48, 1024),
        (64, 80, 200), (65, 33, 520), (3, 5, 4104), (200, 130, 264), (1, 4000, 16)]


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("m,n,k", EDGE)
def test_edge_shapes(m, n, k, bias):
    _say(f"edge M={m} N={n} K={k} bias={bias}")
    x, q, s, b = make_case(m, n, k, seed=11, bias=bias)
    packed = rf.pack_weight(_to_dev(q))
    kernels = ["auto", "gemm"] + (["gemv"] if m <= 64 else [])
    for kern in kernels:
        assert_parity(run_gpu(x, q, s, b, KERNELS[kern], packed), x, q, s, b,
                      label=f"edge {m}x{n}x{k} {kern}")


# One shape per rule of the GEMV planner (w8a16_gemv.hip plan_gemv), so every
# kernel configuration it can pick runs at least once.
GEMV_POLICY = [row[:3] for row in planner_cases.GEMV_POLICY]  # one shape per GEMV planner rule


@pytest.mark.parametrize("m,n,k", GEMV_POLICY)
def test_gemv_every_planner_rule(m, n, k):
    _say(f"gemv policy M={m} N={n} K={k}")
    x, q, s, b = make_case(m, n, k, seed=16, bias=True)
    if m <= 16:
        assert rf.select_kernel(m, n, k) == rf.KERNEL_GEMV
    packed = rf.pack_weight(_to_dev(q))
    y1 = run_gpu(x, q, s, b, kernel=rf.KERNEL_GEMV, packed=packed)
    assert_parity(y1, x, q, s, b, label=f"gemv policy {m}x{n}x{k}")
    y2 = run_gpu(x, q, s, b, kernel=rf.KERNEL_GEMV, packed=packed)  # split-K counters left zeroed
    assert (y1.view(np.uint16) == y2.view(np.uint16)).all()


# One shape per rule of the GEMM planner (w8a16_gemm.hip plan_gemm), with a
# 256-CU MI355X: tiles = ceil(M/BM) * ceil(N/BN); a K split below one tile per
# CU (>= 16 or 24 blocks of 64 per split), or for K >= 12288 at one tile per CU
# or a CU share of 1.25..1.75 / 2.25..2.75 tiles.
GEMM_POLICY = [row[:3] for row in planner_cases.GEMM_POLICY]  # one shape per GEMM planner rule


@pytest.mark.parametrize("m,n,k", GEMM_POLICY)
def test_gemm_every_planner_rule(m, n, k):
    _say(f"gemm policy M={m} N={n} K={k}")
    x, q, s, b = make_case(m, n, k, seed=18, bias=True)
    if m >= 65:
        assert rf.select_kernel(m, n, k) == rf.KERNEL_GEMM
    rows = None if m <= 300 else np.random.default_rng(m).choice(m, 128, replace=False)
    packed = rf.pack_weight(_to_dev(q))
    y1 = run_gpu(x, q, s, b, kernel=rf.KERNEL_GEMM, packed=packed)
    assert_parity(y1, x, q, s, b, rows=rows, label=f"gemm policy {m}x{n}x{k}")
    y2 = run_gpu(x, q, s, b, kernel=rf.KERNEL_GEMM, packed=packed)  # split-K: same sum order
    assert (y1.view(np.uint16) == y2.view(np.uint16)).all()


def test_gemm_split_k_matches_unsplit_order_free():
    """The K-split GEMM sums its fp32 partials in split order: bit-identical over
    repeated calls and interleaved with other shapes, and within tolerance of the
    GEMV on the same inputs (M=64: 16 tiles of 64x64, 8-way split)."""
    m, n, k = 64, 1024, 8192
    _say(f"gemm split-K vs gemv M={m} N={n} K={k}")
    x, q, s, b = make_case(m, n, k, seed=31, bias=True)
    packed = rf.pack_weight(_to_dev(q))
    xd, sd, bd = _to_dev(x), _to_dev(s), _to_dev(b)
    first = rf.linear(xd, packed, sd, bd, kernel=rf.KERNEL_GEMM)
    for i in range(3):
        other = make_case(150, 300, 2048, seed=32 + i)
        run_gpu(*other)  # another split shape on the same workspace in between
        again = rf.linear(xd, packed, sd, bd, kernel=rf.KERNEL_GEMM)
        assert torch.equal(first, again)
    y = first.cpu().numpy()
    assert_parity(y, x, q, s, b, label="gemm split-K")
    g = rf.linear(xd, packed, sd, bd, kernel=rf.KERNEL_GEMV).cpu().numpy()
    rep = o.check_tolerance(y, g, o.oracle_fp64(x, q, s, b))
    assert rep.ok, f"gemm split-K vs gemv: {rep}"


def _strided_rows(x, ldx):
    """x [m, k] copied into rows ldx halves apart (one device allocation)."""
    m, k = x.shape
    big = torch.empty((m - 1) * ldx + k, dtype=torch.float16, device=DEV)
    view = big.as_strided((m, k), (ldx, 1))
    view.copy_(_to_dev(x))
    return view


def _capi_linear(xv, ldx, packed, sd, y, m, n, k, kernel):
    """rf_w8a16_linear through ctypes on the current stream; returns the status."""
    lib = capi.load()
    ws_bytes = lib.rf_w8a16_workspace_bytes(m, n, k)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=DEV)
    st = lib.rf_w8a16_linear(xv.data_ptr(), ldx, packed.data_ptr(), capi.LAYOUT_TILE16X64,
                             sd.data_ptr(), None, y.data_ptr(), n, m, n, k, kernel, ws.data_ptr(),
                             ws_bytes, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return st


def test_gemm_fallback_when_row_stride_overflows_32bit_offsets():
    """Rows 2**24 + 8 halves apart: the 128-row tile spans more than 4 GB, so the
    GEMM called through the C ABI must take its 64-bit-address kernel; results
    must not change.  The torch op copies such a view to contiguous rows."""
    m, n, k = 130, 256, 200
    ldx = (1 << 24) + 8
    _say(f"gemm fallback M={m} N={n} K={k} ldx={ldx}")
    x, q, s, b = make_case(m, n, k, seed=19)
    view = _strided_rows(x, ldx)
    packed, sd = rf.pack_weight(_to_dev(q)), _to_dev(s)
    ref = rf.linear(_to_dev(x), packed, sd)
    y = torch.empty(m, n, dtype=torch.float16, device=DEV)
    capi.check(_capi_linear(view, ldx, packed, sd, y, m, n, k, capi.KERNEL_GEMM), "gemm fallback")
    assert torch.equal(y, ref)
    assert_parity(y.cpu().numpy(), x, q, s, None, label="gemm fallback")
    y2 = rf.linear(view, packed, sd)
    torch.cuda.synchronize()
    assert torch.equal(y2, ref)
    del view


@pytest.mark.parametrize("m,kernel", [(64, "gemv"), (64, "auto"), (16, "auto"), (40, "gemv")])
def test_gemv_rows_far_apart(m, kernel):
    """Activation rows 2**25 + 8 halves apart: (M-1) * ldx * 2 bytes exceed 2**32,
    so a per-lane 32-bit offset from row 0 would wrap.  The GEMV addresses each
    16-row m-tile from its own 64-bit base; called through the C ABI (no copy)
    it must match the oracle and the contiguous call bit for bit."""
    n, k = 1024, 512
    ldx = (1 << 25) + 8
    _say(f"gemv rows far apart M={m} kernel={kernel} ldx={ldx}")
    x, q, s, _ = make_case(m, n, k, seed=41 + m)
    view = _strided_rows(x, ldx)
    packed, sd = rf.pack_weight(_to_dev(q)), _to_dev(s)
    y = torch.empty(m, n, dtype=torch.float16, device=DEV)
    capi.check(_capi_linear(view, ldx, packed, sd, y, m, n, k, KERNELS[kernel]), "far rows")
    ref = torch.empty_like(y)
    capi.check(_capi_linear(_to_dev(x), k, packed, sd, ref, m, n, k, KERNELS[kernel]), "contig")
    assert torch.equal(y, ref)
    assert_parity(y.cpu().numpy(), x, q, s, None, label=f"far rows M={m} {kernel}")
    # the fused argmax (a GEMV epilogue: compared with the argmax of the GEMV's
    # own logits) and the torch op on the same view
    ref_v = torch.empty_like(y)
    capi.check(_capi_linear(_to_dev(x), k, packed, sd, ref_v, m, n, k, capi.KERNEL_GEMV), "gemv")
    idx = torch.empty(m, dtype=torch.int32, device=DEV)
    lib = capi.load()
    ws_bytes = lib.rf_w8a16_workspace_bytes_argmax(m, n, k)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=DEV)
    st = lib.rf_w8a16_linear_argmax(view.data_ptr(), ldx, packed.data_ptr(), capi.LAYOUT_TILE16X64,
                                    sd.data_ptr(), None, None, 0, idx.data_ptr(), m, n, k,
                                    ws.data_ptr(), ws_bytes,
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    capi.check(st, "argmax far rows")
    torch.cuda.synchronize()
    assert torch.equal(idx, _argmax_first(ref_v))
    assert torch.equal(rf.linear(view, packed, sd, kernel=KERNELS[kernel]), ref)
    del view


def test_gemv_refuses_rows_beyond_32bit_reach():
    """Two rows 2**31 halves apart (4 GB): no 16-row span fits a 32-bit offset.
    A forced GEMV is refused before launch; AUTO runs the GEMM's 64-bit kernel."""
    m, n, k = 2, 256, 128
    ldx = 1 << 31
    _say(f"gemv beyond reach M={m} ldx={ldx}")
    x, q, s, _ = make_case(m, n, k, seed=47)
    view = _strided_rows(x, ldx)
    packed, sd = rf.pack_weight(_to_dev(q)), _to_dev(s)
    y = torch.empty(m, n, dtype=torch.float16, device=DEV)
    assert _capi_linear(view, ldx, packed, sd, y, m, n, k, capi.KERNEL_GEMV) == capi.EKERNEL
    capi.check(_capi_linear(view, ldx, packed, sd, y, m, n, k, capi.KERNEL_AUTO), "auto far")
    ref = rf.linear(_to_dev(x), packed, sd)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)
    assert torch.equal(rf.linear(view, packed, sd, kernel=rf.KERNEL_GEMV), ref)
    del view


def test_zero_rows_and_extreme_scales():
    n, k = 64, 256
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w[0] = 0.0
    w[1] *= 1e4
    w[2] *= 1e-5
    q, s = o.quantize_linear_per_channel(w)
    x = o.make_activation(6, 4, k)
    for kern in ("gemv", "gemm"):
        y = run_gpu(x, q, s, None, KERNELS[kern])
        assert (y[:, 0] == 0).all()
        assert_parity(y, x, q, s, None, label=f"extreme scales {kern}")


def test_split_k_deterministic_and_reusable():
    """Small-N shapes take the split-K path; repeated calls are bitwise identical
    (fixed reduction order) and keep working (counters are left zeroed)."""
    x, q, s, b = make_case(4, 1024, 4096, seed=12)
    packed = rf.pack_weight(_to_dev(q))
    xd, sd = _to_dev(x), _to_dev(s)
    first = rf.linear(xd, packed, sd)
    for _ in range(50):
        again = rf.linear(xd, packed, sd)
    torch.cuda.synchronize()
    assert torch.equal(first, again)
    assert_parity(first.cpu().numpy(), x, q, s, b, label="split-K")


def test_gpu_quantizer_matches_oracle():
    w = o.make_weight(31, 300, 1000)
    w[3] = 0
    qd, sd = rf.quantize_linear_per_channel(_to_dev(w))
    q, s = o.quantize_linear_per_channel(w)
    assert (qd.cpu().numpy() == q).all()
    assert (sd.cpu().numpy().view(np.uint16) == s.view(np.uint16)).all()


def test_device_pack_equals_host_pack():
    for n, k in [(17, 72), (3072, 1024), (100, 8)]:
        q = torch.randint(-128, 128, (n, k), dtype=torch.int8)
        packed = rf.pack_weight(q.to(DEV))
        assert torch.equal(packed.cpu(), rf.pack_weight(q))
        # the inverse on the device (what state_dict() uses) and on the host
        back = rf.ops.unpack_weight_on_device(packed, n, k)
        assert back.device == packed.device and torch.equal(back.cpu(), q)
        assert torch.equal(rf.unpack_weight(packed, n, k), q)


def test_module_state_dict_on_device_is_row_major():
    q = torch.randint(-128, 128, (96, 320), dtype=torch.int8)
    s = (torch.rand(96) * 0.01 + 1e-3).half()
    mod = rf.W8A16Linear.from_quantized(q, s, device=DEV)
    sd = mod.state_dict()
    assert sd["weight"].device == mod.weight.device and torch.equal(sd["weight"].cpu(), q)
    fresh = rf.W8A16Linear(320, 96, device=DEV)
    fresh.load_state_dict(sd)
    assert torch.equal(fresh.weight, mod.weight)


def test_input_views_3d_empty_and_linear_into():
    x, q, s, b = make_case(6, 96, 128, seed=13, bias=True)
    packed, sd, bd = rf.pack_weight(_to_dev(q)), _to_dev(s), _to_dev(b)
    ref = rf.linear(_to_dev(x), packed, sd, bd)
    y3 = rf.linear(_to_dev(x).view(2, 3, 128), packed, sd, bd)
    assert y3.shape == (2, 3, 96) and torch.equal(y3.view(6, 96), ref)
    wide = torch.zeros(6, 256, dtype=torch.float16, device=DEV)
    wide[:, 64:192] = _to_dev(x)
    assert torch.equal(rf.linear(wide[:, 64:192], packed, sd, bd), ref)  # strided rows
    odd = torch.zeros(6 * 128 + 1, dtype=torch.float16, device=DEV)[1:].view(6, 128)
    odd.copy_(_to_dev(x))  # misaligned base address -> copied internally
    assert torch.equal(rf.linear(odd, packed, sd, bd), ref)
    out = torch.empty(6, 96, dtype=torch.float16, device=DEV)
    rf.linear_into(_to_dev(x), packed, sd, bd, out)
    assert torch.equal(out, ref)
    empty = rf.linear(torch.zeros(0, 128, dtype=torch.float16, device=DEV), packed, sd, bd)
    assert empty.shape == (0, 96)


def test_op_errors_on_device():
    # A row-major weight is refused, whatever its shape: the packed form is
    # the 3-D tiles [ceil(N/16), ceil(K/64), 1024].
    x, q, s, _ = make_case(2, 40, 120, seed=14)
    packed, sd = rf.pack_weight(_to_dev(q)), _to_dev(s)
    with pytest.raises(RuntimeError, match="packed int8 tiles"):
        rf.linear(_to_dev(x), _to_dev(q), sd)  # row-major weight, not packed
    x2, q2, s2, _ = make_case(2, 64, 128, seed=15)   # row-major [64, 128]: aligned shape
    for call in (lambda w: rf.linear(_to_dev(x2), w, _to_dev(s2)),
                 lambda w: rf.linear_multi(_to_dev(x2), [w], [_to_dev(s2)]),
                 lambda w: rf.linear_argmax(_to_dev(x2), w, _to_dev(s2))):
        with pytest.raises(RuntimeError, match="packed int8 tiles"):
            call(_to_dev(q2))
    with pytest.raises(RuntimeError, match="GEMV|cannot run"):
        rf.linear(torch.zeros(65, 120, dtype=torch.float16, device=DEV), packed, sd,
                  kernel=rf.KERNEL_GEMV)
    with pytest.raises(RuntimeError, match="bias"):
        rf.linear(_to_dev(x), packed, sd, torch.zeros(39, dtype=torch.float16, device=DEV))


@pytest.mark.parametrize("m,n,k", [(16, 1024, 8192), (1, 4096, 1024), (300, 384, 1024),
                                   (48, 5120, 8192), (32, 8192, 5120), (32, 25600, 320),
                                   (128, 2048, 4104)])
def test_graph_capture_replays_match_eager(m, n, k):
    """The op inside a HIP graph: every replay (with eager work between replays)
    equals the eager result bit for bit.  (16, 1024, 8192) takes the split-K
    GEMV path, (48, 5120, 8192) the 8-way split mid-M GEMM, (32, 8192, 5120)
    the 4-way split 32x64 tile and (128, 2048, 4104) the 4-way split 64x64
    tile with two K groups, whose counters must be left zeroed for the next
    replay; (32, 25600, 320) the unsplit 32x128 tile, (300, 384, 1024) the
    unsplit 64x64 tile with two K groups."""
    _say(f"graph capture M={m} N={n} K={k}")
    x, q, s, b = make_case(m, n, k, seed=17, bias=True)
    xd, packed, sd, bd = _to_dev(x), rf.pack_weight(_to_dev(q)), _to_dev(s), _to_dev(b)
    eager = rf.linear(xd, packed, sd, bd)
    out = torch.empty_like(eager)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        rf.linear_into(xd, packed, sd, bd, out)  # warm-up: workspace for this stream
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        rf.linear_into(xd, packed, sd, bd, out)
    for i in range(5):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        other = rf.linear(xd, packed, sd, bd)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(other, eager)
    assert_parity(out.cpu().numpy(), x, q, s, b, label=f"graph {m}x{n}x{k}")


@pytest.mark.parametrize("m", [1, 4, 16, 40, 100])
def test_linear_multi_qkv_and_gate_up(m):
    """q/k/v (4096/1024/1024 x 4096, q with a bias) and gate/up (12288 x 4096) in one
    call each: every output against the oracle, and against separate calls."""
    groups = [[(4096, True), (1024, False), (1024, False)], [(12288, False), (12288, False)]]
    k = 4096
    for gi, group in enumerate(groups):
        _say(f"linear_multi M={m} group {gi}")
        x = o.make_activation(o.derive_seed(20, "x", m, gi), m, k)
        cases = []
        for pi, (n, has_bias) in enumerate(group):
            q, s = make_weights(n, k, seed=200 + 10 * gi + pi)
            b = (o.normal(o.derive_seed(21, "b", n, pi), (n,)) * 0.1).astype(np.float16) if has_bias else None
            cases.append((q, s, b, rf.pack_weight(_to_dev(q))))
        xd = _to_dev(x)
        ys = rf.linear_multi(xd, [c[3] for c in cases], [_to_dev(c[1]) for c in cases],
                             [None if c[2] is None else _to_dev(c[2]) for c in cases])
        torch.cuda.synchronize()
        for pi, (q, s, b, packed) in enumerate(cases):
            y = ys[pi].cpu().numpy()
            assert_parity(y, x, q, s, b, label=f"multi M={m} g{gi} p{pi}")
            single = rf.linear(xd, packed, _to_dev(s), None if b is None else _to_dev(b)).cpu().numpy()
            rep = o.check_tolerance(y, single, o.oracle_fp64(x, q, s, b))
            assert rep.ok, f"multi vs single: {rep}"


def test_linear_multi_gemm_one_launch_ragged_split():
    """M=1030 (GEMM), three projections of ragged widths sharing K=4104 (K tail)
    in one launch: 117 tiles of 128x128 take a 4-way K split; one projection
    has a bias.  Each output against the oracle and against a single call."""
    m, k = 1030, 4104
    ns = [(1000, False), (264, True), (136, False)]
    x = o.make_activation(o.derive_seed(24, "x", m, k), m, k)
    rows = np.random.default_rng(24).choice(m, 96, replace=False)
    cases = []
    for pi, (n, has_bias) in enumerate(ns):
        q, s = make_weights(n, k, seed=240 + pi)
        b = (o.normal(o.derive_seed(25, "b", n, pi), (n,)) * 0.1).astype(np.float16) if has_bias else None
        cases.append((q, s, b, rf.pack_weight(_to_dev(q))))
    xd = _to_dev(x)
    _say(f"linear_multi gemm M={m} K={k} Ns={[n for n, _ in ns]}")
    ys = rf.linear_multi(xd, [c[3] for c in cases], [_to_dev(c[1]) for c in cases],
                         [None if c[2] is None else _to_dev(c[2]) for c in cases])
    again = rf.linear_multi(xd, [c[3] for c in cases], [_to_dev(c[1]) for c in cases],
                            [None if c[2] is None else _to_dev(c[2]) for c in cases])
    torch.cuda.synchronize()
    for pi, (q, s, b, packed) in enumerate(cases):
        assert torch.equal(ys[pi], again[pi])
        y = ys[pi].cpu().numpy()
        assert_parity(y, x, q, s, b, rows=rows, label=f"multi gemm p{pi}")
        single = rf.linear(xd, packed, _to_dev(s), None if b is None else _to_dev(b)).cpu().numpy()
        rep = o.check_tolerance(y[rows], single[rows], o.oracle_fp64(x[rows], q, s, b))
        assert rep.ok, f"multi gemm vs single: {rep}"


def test_linear_multi_gemm_whole_rounds_two_projections():
    """M=1024, gate/up-like pair N = 8200 (ragged) and 7936, K = 520 (K tail):
    8 x (33 + 31) = 512 tiles of 128x256 fill two whole rounds.  Each output
    against the oracle and against a single call."""
    m, k = 1024, 520
    ns = [(8200, True), (7936, False)]
    x = o.make_activation(o.derive_seed(26, "x", m, k), m, k)
    rows = np.random.default_rng(26).choice(m, 96, replace=False)
    cases = []
    for pi, (n, has_bias) in enumerate(ns):
        q, s = make_weights(n, k, seed=260 + pi)
        b = (o.normal(o.derive_seed(27, "b", n, pi), (n,)) * 0.1).astype(np.float16) if has_bias else None
        cases.append((q, s, b, rf.pack_weight(_to_dev(q))))
    xd = _to_dev(x)
    _say(f"linear_multi gemm whole rounds M={m} K={k} Ns={[n for n, _ in ns]}")
    ys = rf.linear_multi(xd, [c[3] for c in cases], [_to_dev(c[1]) for c in cases],
                         [None if c[2] is None else _to_dev(c[2]) for c in cases])
    torch.cuda.synchronize()
    for pi, (q, s, b, packed) in enumerate(cases):
        y = ys[pi].cpu().numpy()
        assert_parity(y, x, q, s, b, rows=rows, label=f"multi gemm whole rounds p{pi}")
        single = rf.linear(xd, packed, _to_dev(s), None if b is None else _to_dev(b)).cpu().numpy()
        rep = o.check_tolerance(y[rows], single[rows], o.oracle_fp64(x[rows], q, s, b))
        assert rep.ok, f"multi gemm whole rounds vs single: {rep}"


def test_linear_multi_split_k_and_capi():
    """M=16, K=12288: the shared launch takes the 4-way K split; also via ctypes."""
    m, k = 16, 12288
    ns = [1024, 512, 256]
    x = o.make_activation(22, m, k)
    cases = []
    for pi, n in enumerate(ns):
        q, s = make_weights(n, k, seed=230 + pi)
        cases.append((q, s, rf.pack_weight(_to_dev(q)), _to_dev(s)))
    xd = _to_dev(x)
    ys = rf.linear_multi(xd, [c[2] for c in cases], [c[3] for c in cases])
    again = rf.linear_multi(xd, [c[2] for c in cases], [c[3] for c in cases])
    torch.cuda.synchronize()
    for pi, (q, s, _, _) in enumerate(cases):
        assert torch.equal(ys[pi], again[pi])
        assert_parity(ys[pi].cpu().numpy(), x, q, s, None, label=f"multi split-K p{pi}")
    lib = capi.load()
    outs = [torch.empty(m, n, dtype=torch.float16, device=DEV) for n in ns]
    arr = (capi.Proj * len(ns))()
    for i, (c, y) in enumerate(zip(cases, outs)):
        arr[i] = capi.Proj(c[2].data_ptr(), c[3].data_ptr(), None, y.data_ptr(), ns[i], ns[i])
    nsc = (ctypes.c_int64 * len(ns))(*ns)
    ws_bytes = lib.rf_w8a16_workspace_bytes_multi(m, nsc, len(ns), k)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=DEV)
    st = lib.rf_w8a16_linear_multi(xd.data_ptr(), k, capi.LAYOUT_TILE16X64, arr, len(ns), m, k,
                                   capi.KERNEL_AUTO, ws.data_ptr(), ws_bytes,
                                   ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    capi.check(st, "rf_w8a16_linear_multi")
    torch.cuda.synchronize()
    for y, ref in zip(outs, ys):
        assert torch.equal(y, ref)


def test_opcheck_on_device_tensors():
    """torch.library.opcheck with device tensors: schema, autograd registration
    (the input requires grad; autograd falls through, outputs carry no graph),
    FakeTensor and AOT dispatch with dynamic shapes, for every compute op."""
    from torch.library import opcheck
    n, k = 96, 256
    x = torch.randn(2, 5, k, device=DEV).half().requires_grad_()
    q = torch.randint(-128, 128, (n, k), dtype=torch.int8, device=DEV)
    w, s = rf.pack_weight(q), (torch.rand(n, device=DEV) * 0.01 + 1e-3).half()
    b = torch.randn(n, device=DEV).half()
    out = torch.empty(2, 5, n, dtype=torch.float16, device=DEV)
    q4 = torch.randint(-8, 8, (n, k), dtype=torch.int8, device=DEV)
    w4, s4 = rf.pack_weight_int4(q4), (torch.rand(k // 32, n, device=DEV) * 0.01 + 1e-3).half()
    cases = [
        (torch.ops.w8a16.linear.default, (x, w, s, b)),
        (torch.ops.w8a16.linear_into.default, (x, w, s, b, out)),
        (torch.ops.w8a16.linear_multi.default, (x, [w, w], [s, s], [b, None])),
        (torch.ops.w8a16.linear_argmax.default, (x, w, s, None, True)),
        (torch.ops.w8a16.pack_weight.default, (q,)),
        (torch.ops.w4a16.linear.default, (x, w4, s4)),
        (torch.ops.w4a16.linear_multi.default, (x, [w4, w4], [s4, s4], [b, None])),
        (torch.ops.w4a16.pack_weight.default, (q4,)),
    ]
    for op, args in cases:
        _say(f"opcheck {op}")
        report = opcheck(op, args, raise_exception=False)
        failed = {key: v for key, v in report.items() if v != "SUCCESS"}
        assert not failed, f"{op}: {failed}"
    y = rf.linear(x, w, s, b)
    assert not y.requires_grad


def test_w8a16_linear_module_forward():
    torch.manual_seed(0)
    lin = torch.nn.Linear(512, 200, bias=True)
    mod = rf.W8A16Linear.from_linear(lin).to(DEV)
    x = o.make_activation(21, 5, 512)
    y = mod(_to_dev(x)).cpu().numpy()
    q, s = rf.quantize_linear_per_channel(lin.weight.detach())
    assert_parity(y, x, q.numpy(), s.numpy(), lin.bias.detach().half().numpy(), label="module")


def test_capi_direct_call():
    """Call rf_w8a16_linear through ctypes, as a non-torch host would."""
    lib = capi.load()
    x, q, s, _ = make_case(3, 1024, 4096, seed=15)
    xd, sd = _to_dev(x), _to_dev(s)
    packed = rf.pack_weight(_to_dev(q))
    y = torch.empty(3, 1024, dtype=torch.float16, device=DEV)
    ws_bytes = lib.rf_w8a16_workspace_bytes(3, 1024, 4096)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    for kern in (capi.KERNEL_GEMV, capi.KERNEL_GEMM):
        st = lib.rf_w8a16_linear(xd.data_ptr(), 4096, packed.data_ptr(), capi.LAYOUT_TILE16X64,
                                 sd.data_ptr(), None, y.data_ptr(), 1024, 3, 1024, 4096, kern,
                                 ws.data_ptr(), ws_bytes, ctypes.c_void_p(stream))
        capi.check(st, "rf_w8a16_linear")
        torch.cuda.synchronize()
        assert_parity(y.cpu().numpy(), x, q, s, None, label=f"ctypes kernel={kern}")
    assert lib.rf_w8a16_linear(xd.data_ptr(), 4096, packed.data_ptr(), capi.LAYOUT_TILE16X64,
                               sd.data_ptr(), None, y.data_ptr(), 1024, 3, 1024, 4096,
                               capi.KERNEL_GEMV, None, 0, ctypes.c_void_p(stream)) in (
        capi.EWORKSPACE, capi.OK)


# ------------------------------------------- several projections, 3..7 strips per workgroup
@pytest.mark.parametrize("case", planner_cases.STRIP_GROUP_LAUNCHES, ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}")
def test_linear_multi_strip_groups(case):
    """linear_multi where the planner gives each workgroup three to seven
    strips: every row of every projection within the bar, and a second call
    bit-identical to the first."""
    m, ns, k, name = case
    _say(f"strip groups M={m} N={ns} K={k}")
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert capi.plan(m, ns, k)["name"] == name
    x = o.make_activation(o.derive_seed(91, "x", m, k), m, k)
    qs = [o.quantize_linear_per_channel(o.make_weight(o.derive_seed(91, "w", j, n, k), n, k))
          for j, n in enumerate(ns)]
    bs = [(o.normal(o.derive_seed(91, "b", j, n), (n,)) * 0.1).astype(np.float16) if j == 1 else None
          for j, n in enumerate(ns)]
    args = ([rf.pack_weight(_to_dev(q)) for q, _ in qs], [_to_dev(s) for _, s in qs],
            [None if b is None else _to_dev(b) for b in bs])
    ys = rf.linear_multi(_to_dev(x), *args)
    ys2 = rf.linear_multi(_to_dev(x), *args)
    torch.cuda.synchronize()
    for j, ((q, s), b, y, y2) in enumerate(zip(qs, bs, ys, ys2)):
        assert torch.equal(y, y2), f"proj {j}: second call differs"
        assert_parity(y.cpu().numpy(), x, q, s, b, label=f"proj {j} N={ns[j]}")


# ---------------------------------------------------------------- seeded random shapes
def _random_launches(seed=2026, count=48):
    """Shapes drawn around the planners' boundaries: M on both sides of
    16 / 32 / 64 / 128 / 256, 1..4 projections sharing x, N multiples of 16
    or ragged, K multiples of 64 or a K tail, forced GEMV / GEMM or AUTO."""
    rng = np.random.default_rng(seed)
    ms = [1, 2, 3, 4, 5, 8, 15, 16, 17, 24, 31, 32, 33, 48, 63, 64, 65, 96, 127, 128, 129,
          200, 255, 256, 300, 513]
    out = []
    for i in range(count):
        m = int(rng.choice(ms))
        ns = [int(rng.integers(1, 64)) * 16 + (int(rng.integers(1, 16)) if rng.random() < 0.3 else 0)
              for _ in range(int(rng.integers(1, 5)))]
        k = int(rng.integers(1, 97)) * 64 + (int(rng.integers(1, 8)) * 8 if rng.random() < 0.3 else 0)
        kernel = str(rng.choice(["auto", "gemv", "gemm"] if m <= 64 else ["auto", "gemm"]))
        out.append((i, m, ns, k, kernel))
    return out


@pytest.mark.parametrize("case", _random_launches(), ids=lambda c: f"r{c[0]}-{c[1]}x{c[2]}x{c[3]}-{c[4]}")
def test_random_launch_shapes(case):
    """linear_multi over seeded random shapes: every projection within the bar
    (the fp64 oracle on at most 64 rows: the first and last 32)."""
    i, m, ns, k, kernel = case
    _say(f"random launch {i}: M={m} N={ns} K={k} kernel={kernel}")
    x = o.make_activation(o.derive_seed(77, "x", i, m, k), m, k)
    qs = [o.quantize_linear_per_channel(o.make_weight(o.derive_seed(77, "w", i, j, n, k), n, k))
          for j, n in enumerate(ns)]
    bs = [(o.normal(o.derive_seed(77, "b", i, j), (n,)) * 0.1).astype(np.float16) if j % 2 else None
          for j, n in enumerate(ns)]
    ys = rf.linear_multi(_to_dev(x), [rf.pack_weight(_to_dev(q)) for q, _ in qs],
                         [_to_dev(s) for _, s in qs], [None if b is None else _to_dev(b) for b in bs],
                         kernel=KERNELS[kernel])
    torch.cuda.synchronize()
    rows = None if m <= 64 else np.r_[0:32, m - 32:m]
    for j, ((q, s), b, y) in enumerate(zip(qs, bs, ys)):
        assert tuple(y.shape) == (m, ns[j])
        assert_parity(y.cpu().numpy(), x, q, s, b, rows=rows, label=f"proj {j} N={ns[j]}")


def _random_wide_launches(seed=4099, count=24):
    """Wide launches: 1..4 projections summing to 513..32768 columns (the
    planners' many-strip rules, three to seven strips per workgroup among
    them), M 1..64, ragged N and K tails, AUTO or forced GEMV."""
    rng = np.random.default_rng(seed)
    ms = [1, 2, 3, 4, 5, 6, 8, 9, 12, 13, 16, 24, 32, 48, 64]
    out = []
    for i in range(count):
        m = int(rng.choice(ms))
        total = int(rng.integers(513, 2049)) * 16
        parts = int(rng.integers(1, 5))
        cuts = np.sort(rng.choice(np.arange(1, total // 16), parts - 1, replace=False)) * 16
        ns = [int(b - a) for a, b in zip(np.r_[0, cuts], np.r_[cuts, total])]
        if rng.random() < 0.5:
            ns[-1] -= int(rng.integers(1, 16))  # a ragged last projection
        k = int(rng.integers(2, 33)) * 64 + (int(rng.integers(1, 8)) * 8 if rng.random() < 0.3 else 0)
        kernel = str(rng.choice(["auto", "gemv"]))
        out.append((i, m, ns, k, kernel))
    return out


@pytest.mark.parametrize("case", _random_wide_launches(),
                         ids=lambda c: f"w{c[0]}-{c[1]}x{sum(c[2])}x{c[3]}-{c[4]}")
def test_random_wide_launch_shapes(case):
    """linear_multi over seeded wide random launches: every projection within
    the bar on its first and last rows (all rows up to M = 16)."""
    i, m, ns, k, kernel = case
    _say(f"wide random launch {i}: M={m} N={ns} K={k} kernel={kernel} "
         f"plan={capi.plan(m, ns, k, kernel=KERNELS[kernel])['name']}")
    x = o.make_activation(o.derive_seed(78, "x", i, m, k), m, k)
    qs = [o.quantize_linear_per_channel(o.make_weight(o.derive_seed(78, "w", i, j, n, k), n, k))
          for j, n in enumerate(ns)]
    bs = [(o.normal(o.derive_seed(78, "b", i, j), (n,)) * 0.1).astype(np.float16) if j % 2 else None
          for j, n in enumerate(ns)]
    ys = rf.linear_multi(_to_dev(x), [rf.pack_weight(_to_dev(q)) for q, _ in qs],
                         [_to_dev(s) for _, s in qs], [None if b is None else _to_dev(b) for b in bs],
                         kernel=KERNELS[kernel])
    torch.cuda.synchronize()
    rows = None if m <= 16 else np.r_[0:8, m - 8:m]
    for j, ((q, s), b, y) in enumerate(zip(qs, bs, ys)):
        assert tuple(y.shape) == (m, ns[j])
        assert_parity(y.cpu().numpy(), x, q, s, b, rows=rows, label=f"proj {j} N={ns[j]}")



def test_linear_multi_two_k_groups():
    """Three ragged projections at M = 256 (K = 4104, a K tail) in one launch of
    the 64x64 tile with two K groups: every row of every output against the
    oracle, and bit-identical to a second call."""
    m, k = 256, 4104
    ns = [1000, 520, 520]
    plan = capi.plan(m, ns, k, cus=256)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert plan["name"] == "gemm 64x64 two K groups", plan
    _say(f"linear_multi two K groups M={m} N={ns} K={k}")
    cases = [make_case(m, n, k, seed=40 + i, bias=(i == 0)) for i, n in enumerate(ns)]
    x = cases[0][0]
    xd = _to_dev(x)
    packed = [rf.pack_weight(_to_dev(c[1])) for c in cases]
    scales = [_to_dev(c[2]) for c in cases]
    biases = [None if c[3] is None else _to_dev(c[3]) for c in cases]
    ys = rf.linear_multi(xd, packed, scales, biases)
    again = rf.linear_multi(xd, packed, scales, biases)
    torch.cuda.synchronize()
    for i, (c, y, y2) in enumerate(zip(cases, ys, again)):
        assert torch.equal(y, y2), i
        assert_parity(y.cpu().numpy(), x, c[1], c[2], c[3], label=f"two K groups proj {i}")


def test_linear_multi_long_k_two_k_groups():
    """Two ragged projections at M = 1000 with K = 12296 (a K tail) in one
    launch of the 128x256 register-B tile with two K groups and two K splits:
    sampled rows (first and last included) of both outputs against the
    oracle, and bit-identical to a second call."""
    m, k = 1000, 12296
    ns = [2056, 1000]
    plan = capi.plan(m, ns, k, cus=256)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert (plan["name"], plan["splits"]) == ("gemm 128x256 two K groups, B-in-registers", 2), plan
    _say(f"linear_multi long-K two K groups M={m} N={ns} K={k}")
    cases = [make_case(m, n, k, seed=60 + i, bias=(i == 0)) for i, n in enumerate(ns)]
    x = cases[0][0]
    xd = _to_dev(x)
    packed = [rf.pack_weight(_to_dev(c[1])) for c in cases]
    scales = [_to_dev(c[2]) for c in cases]
    biases = [None if c[3] is None else _to_dev(c[3]) for c in cases]
    ys = rf.linear_multi(xd, packed, scales, biases)
    again = rf.linear_multi(xd, packed, scales, biases)
    torch.cuda.synchronize()
    rows = np.concatenate([[0, m - 1], np.random.default_rng(m).choice(np.arange(1, m - 1), 62, replace=False)])
    for i, (c, y, y2) in enumerate(zip(cases, ys, again)):
        assert torch.equal(y, y2), i
        assert_parity(y.cpu().numpy(), x, c[1], c[2], c[3], rows=rows, label=f"long-K two K groups proj {i}")


def test_workspace_grows_on_a_fresh_stream():
    """The torch ops call the C ABI with the stream's cached workspace first
    (16 MB on a new stream) and grow it only when the call is refused with
    EWORKSPACE.  (600, 4096, 8192) plans a 3-way split 128x128 GEMM whose
    partials take 30 MB: on a fresh stream the first call of each op is
    refused, grown and repeated.  Checked against the oracle on sampled rows
    and, for every op, bit-identical to the same call on the default stream."""
    m, n, k = 600, 4096, 8192
    plan = capi.plan(m, [n], k, cus=256)
    assert plan["workspace_bytes"] > (16 << 20), plan
    _say(f"workspace growth M={m} N={n} K={k}: {plan['name']}, {plan['splits']} splits")
    x, q, s, b = make_case(m, n, k, seed=23, bias=True)
    xd, packed, sd, bd = _to_dev(x), rf.pack_weight(_to_dev(q)), _to_dev(s), _to_dev(b)
    ref = rf.linear(xd, packed, sd, bd)
    ref_multi = rf.linear_multi(xd, [packed, packed], [sd, sd], [bd, None])
    torch.cuda.synchronize()
    for op in ("linear", "linear_into", "linear_multi"):
        with fresh_hip_stream() as stream:  # its workspace starts at the 16 MB default
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(stream):
                if op == "linear":
                    outs = [rf.linear(xd, packed, sd, bd)]
                elif op == "linear_into":
                    outs = [torch.empty_like(ref)]
                    rf.linear_into(xd, packed, sd, bd, outs[0])
                else:
                    outs = rf.linear_multi(xd, [packed, packed], [sd, sd], [bd, None])
            torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        want = ref_multi if op == "linear_multi" else [ref]
        for got, exp in zip(outs, want):
            assert torch.equal(got, exp), op
    rows = np.r_[0:8, m - 8:m]
    assert_parity(ref.cpu().numpy(), x, q, s, b, rows=rows, label="workspace growth")
    assert_parity(ref_multi[1].cpu().numpy(), x, q, s, None, rows=rows, label="workspace growth multi")
