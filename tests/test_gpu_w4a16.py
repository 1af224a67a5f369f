"""W4A16 parity on the GPU: packed int4 weights through the GEMV and GEMM kernels.

Tolerance (the same bar as W8A16): max|y - y_cpu| <= 1e-2 * rms(y_cpu) and
cos(y, y*) >= 0.9999 per row and overall, with y_cpu the fp16-dequantize-then-
GEMM CPU path and y* the fp64 oracle (oracle/w4a16.py).  Unit-vector inputs
are exact: with x = e_k the result is the dequantized column RN_fp16(s*q[:,k]).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import rhinoforge_amd as rf
from rhinoforge_amd import capi
from oracle import w4a16 as o4
from oracle import w8a16 as o8
import planner_cases
from conftest import fresh_hip_stream

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(*a):
    print(*a, flush=True)


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


_W: dict = {}


def make_w4(n, k, gs, seed):
    key = (n, k, gs, seed)
    if key not in _W:
        w = o8.make_weight(o8.derive_seed(seed, "w4", n, k), n, k)
        if gs:
            q, s = o4.quantize_int4_group_wise(w, gs)
        else:
            q, s = o4.quantize_int4_per_channel(w)
        _W.clear()
        _W[key] = (q, s)
    return _W[key]


def run(x, q, s, b=None, kernel=rf.KERNEL_AUTO, packed=None):
    wp = packed if packed is not None else rf.pack_weight_int4(_dev(q))
    y = rf.linear_w4a16(_dev(x), wp, _dev(s), None if b is None else _dev(b), kernel=kernel)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def check(y, x, q, s, b=None, label="", rows=None):
    if rows is not None:
        x, y = x[rows], y[rows]
    rep = o8.check_tolerance(y, o4.cpu_path(x, q, s, b), o4.oracle_fp64(x, q, s, b))
    _say(f"  {label}: {rep}")
    assert rep.ok, f"{label}: {rep}"


@pytest.mark.parametrize("n,k", [(16, 64), (48, 384), (4096, 4096), (1024, 12288)])
def test_device_pack_matches_host(n, k):
    q = np.random.default_rng(n + k).integers(-8, 8, (n, k)).astype(np.int8)
    host = rf.pack_weight_int4(torch.from_numpy(q))
    packed = rf.pack_weight_int4(_dev(q))
    assert torch.equal(host, packed.cpu())
    back = rf.ops.unpack_weight_int4_on_device(packed, n, k)   # state_dict()'s inverse
    assert back.device == packed.device and np.array_equal(back.cpu().numpy(), q)


@pytest.mark.parametrize("gs", [0, 32, 128])
@pytest.mark.parametrize("kernel,m", [("gemv", 1), ("gemv", 16), ("gemv", 64), ("gemm", 130)])
def test_unit_vectors_are_exact(gs, kernel, m):
    n, k = 64, 256
    q, s = make_w4(n, k, gs, 1)
    x = np.zeros((m, k), np.float16)
    cols = [(7 * i) % k for i in range(m)]
    x[np.arange(m), cols] = 1.0
    kern = rf.KERNEL_GEMV if kernel == "gemv" else rf.KERNEL_GEMM
    y = run(x, q, s, kernel=kern)
    want = o4.dequantize_int4(q, s)[:, cols].T
    assert np.array_equal(y.view(np.uint16), want.view(np.uint16)), f"{kernel} m={m} gs={gs}"


# (M, N, K, group_size): GEMV planner rules (strips, int4 tiles of 128 K),
# the K % 128 == 64 tail, split-K in both kernels, the BASELINE shapes.
CASES = [
    (1, 4096, 4096, 32), (1, 4096, 4096, 0), (1, 4096, 12288, 128), (1, 24576, 4096, 64),
    (1, 1024, 4096, 32), (2, 10240, 512, 32), (4, 512, 8192, 0), (1, 512, 1088, 32),
    (3, 16384, 512, 64), (8, 32768, 128, 32), (16, 16384, 256, 0), (12, 8192, 256, 32),
    (16, 4096, 4096, 32), (16, 1024, 8192, 128), (9, 1008, 1024, 32), (16, 2048, 1024, 0),
    (20, 16384, 128, 32), (32, 640, 8192, 64), (17, 1024, 576, 32), (40, 8192, 256, 0),
    (64, 1008, 640, 32), (65, 4096, 4096, 32), (130, 1040, 2112, 64), (200, 16400, 192, 0),
    (1024, 4096, 4096, 32), (1100, 1008, 640, 128), (300, 1024, 8192, 32), (256, 512, 4096, 0),
    # int4-only GEMV rules: M 3..4 many strips with x in LDS; M 5..16 long K, 2-way split
    (4, 12288, 4096, 32), (3, 10240, 1088, 0), (16, 4096, 12288, 32), (8, 2048, 8192, 128),
    # GEMM tiles with B loaded into registers: 128x256 (ragged M; per-channel), 128x128
    (520, 25600, 1024, 32), (2048, 12288, 1024, 0), (1024, 12288, 2048, 128),
    # GEMM interleaved schedule (one to two 128x128 tiles per CU), group-wise
    (520, 8192, 1024, 32), (1024, 6144, 1024, 128),
    # 160 tiles in a 3-way K split, run by the 128x128 tile with B in registers:
    # splits start at K blocks 0, 43 and 86 (an odd block: the second half of
    # an int4 tile), per-channel and group-wise
    (500, 5008, 8192, 0), (500, 5008, 8192, 32),
]


# One shape per int4 GEMV planner rule (planner_cases.GEMV_INT4_POLICY, whose
# plans the CPU suite checks), group-wise rows with 128-wide groups where K
# allows, else 32.
CASES += [(r[0], r[1], r[2], (128 if r[2] % 128 == 0 else 32) if r[3] else 0)
          for r in planner_cases.GEMV_INT4_POLICY]


@pytest.mark.parametrize("m,n,k,gs", CASES)
def test_w4a16_parity(m, n, k, gs):
    _say(f"w4a16 M={m} N={n} K={k} gs={gs}")
    q, s = make_w4(n, k, gs, 2)
    x = o8.make_activation(o8.derive_seed(2, "x4", m, k), m, k)
    b = (o8.normal(o8.derive_seed(2, "b4", n), (n,)) * 0.1).astype(np.float16) if m % 2 else None
    packed = rf.pack_weight_int4(_dev(q))
    y = run(x, q, s, b, packed=packed)
    rows = None if m <= 64 else np.unique(np.linspace(0, m - 1, 48).astype(int))
    check(y, x, q, s, b, label=f"w4 {m}x{n}x{k} gs={gs}", rows=rows)
    y2 = run(x, q, s, b, packed=packed)   # split-K counters were left zeroed; deterministic
    assert (y.view(np.uint16) == y2.view(np.uint16)).all()


@pytest.mark.parametrize("m", [1, 16, 64])
def test_gemm_forced_matches_gemv(m):
    q, s = make_w4(512, 1024, 32, 3)
    x = o8.make_activation(o8.derive_seed(3, "x", m), m, 1024)
    packed = rf.pack_weight_int4(_dev(q))
    yv = run(x, q, s, kernel=rf.KERNEL_GEMV, packed=packed)
    yg = run(x, q, s, kernel=rf.KERNEL_GEMM, packed=packed)
    check(yg, x, q, s, label=f"gemm forced m={m}")
    assert np.abs(yv.astype(np.float32) - yg.astype(np.float32)).max() <= \
        2e-2 * float(np.sqrt(np.mean(yv.astype(np.float32) ** 2)))


def test_w4a16_linear_module_and_errors():
    torch.manual_seed(0)
    lin = torch.nn.Linear(512, 256, bias=True)
    for gs in (None, 32):
        mod = rf.W4A16Linear.from_linear(lin, group_size=gs).to(DEV)
        x = torch.randn(3, 5, 512, dtype=torch.float16, device=DEV)
        y = mod(x)
        assert y.shape == (3, 5, 256) and y.dtype == torch.float16
        q = mod.rowmajor_weight().numpy()
        s = mod.weight_scale.cpu().numpy()
        b = mod.bias.cpu().numpy()
        check(y.reshape(15, 256).cpu().numpy(), x.reshape(15, 512).cpu().numpy(), q, s, b,
              label=f"module gs={gs}")
    w = rf.pack_weight_int4(torch.zeros(32, 128, dtype=torch.int8, device=DEV))
    x = torch.zeros(2, 128, dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError, match="32, 64 or 128"):
        rf.linear_w4a16(x, w, torch.ones(8, 32, dtype=torch.float16, device=DEV))
    with pytest.raises(RuntimeError, match="multiple of 16"):
        rf.linear_w4a16(x, w, torch.ones(24, dtype=torch.float16, device=DEV))
    with pytest.raises(RuntimeError, match="uint8"):
        rf.linear_w4a16(x, w.to(torch.int8), torch.ones(32, dtype=torch.float16, device=DEV))
    with pytest.raises(RuntimeError, match="packed int4 tiles"):
        rf.linear_w4a16(torch.zeros(2, 256, dtype=torch.float16, device=DEV), w,
                        torch.ones(32, dtype=torch.float16, device=DEV))


def test_w4a16_capi_direct_call():
    """The C ABI called through ctypes, as a non-torch host would bind it."""
    import ctypes
    lib = capi.load()
    m, n, k, gs = 4, 1024, 2048, 64
    q, s = make_w4(n, k, gs, 4)
    x = o8.make_activation(5, m, k)
    xd, sd = _dev(x), _dev(s)
    wp = rf.pack_weight_int4(_dev(q))
    y = torch.empty(m, n, dtype=torch.float16, device=DEV)
    wsb = lib.rf_w4a16_workspace_bytes(m, n, k)
    ws = torch.zeros(wsb, dtype=torch.uint8, device=DEV)
    st = lib.rf_w4a16_linear(xd.data_ptr(), k, wp.data_ptr(), sd.data_ptr(), gs, None,
                             y.data_ptr(), n, m, n, k, 0, ws.data_ptr(), wsb,
                             ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert st == capi.OK, capi.status_str(st)
    check(y.cpu().numpy(), x, q, s, label="capi direct")


@pytest.mark.parametrize("m,ldx,gs", [(64, (1 << 25) + 8, 32), (16, (1 << 25) + 8, 0),
                                      (130, (1 << 24) + 8, 32)])
def test_w4a16_rows_far_apart(m, ldx, gs):
    """Activation rows ldx halves apart, (M-1) * ldx * 2 > 2**32 bytes.  Through
    the C ABI the GEMV (M <= 64) addresses each 16-row m-tile from its own
    64-bit base and must equal the contiguous call bit for bit; the int4 GEMM
    has no 64-bit kernel and refuses (EKERNEL) before launch.  The torch op
    copies such a view to contiguous rows."""
    import ctypes
    n, k = 1024, 512
    _say(f"w4a16 rows far apart M={m} ldx={ldx} gs={gs}")
    q, s = make_w4(n, k, gs, 8)
    x = o8.make_activation(9, m, k)
    big = torch.empty((m - 1) * ldx + k, dtype=torch.float16, device=DEV)
    view = big.as_strided((m, k), (ldx, 1))
    view.copy_(_dev(x))
    sd, wp = _dev(s), rf.pack_weight_int4(_dev(q))
    ref = rf.linear_w4a16(_dev(x), wp, sd)
    lib = capi.load()
    wsb = lib.rf_w4a16_workspace_bytes(m, n, k)
    ws = torch.zeros(wsb, dtype=torch.uint8, device=DEV)
    y = torch.empty(m, n, dtype=torch.float16, device=DEV)
    st = lib.rf_w4a16_linear(view.data_ptr(), ldx, wp.data_ptr(), sd.data_ptr(), gs, None,
                             y.data_ptr(), n, m, n, k, capi.KERNEL_AUTO, ws.data_ptr(), wsb,
                             ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    if m <= 64:
        assert st == capi.OK, capi.status_str(st)
        assert torch.equal(y, ref)
        check(y.cpu().numpy(), x, q, s, label=f"w4 far rows M={m}")
    else:
        assert st == capi.EKERNEL, capi.status_str(st)
    assert torch.equal(rf.linear_w4a16(view, wp, sd), ref)
    del view, big


@pytest.mark.parametrize("m,n,k,gs", [(16, 1024, 8192, 32), (300, 1024, 8192, 0)])
def test_w4a16_graph_replays_match_eager(m, n, k, gs):
    """Inside a HIP graph: split-K GEMV (16 rows) and split-K GEMM (300 rows)
    replays, with eager calls between them, equal the eager result bit for bit."""
    q, s = make_w4(n, k, gs, 6)
    x = o8.make_activation(7, m, k)
    xd, sd, wp = _dev(x), _dev(s), rf.pack_weight_int4(_dev(q))
    eager = rf.linear_w4a16(xd, wp, sd)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        rf.linear_w4a16(xd, wp, sd)  # warm-up: workspace for this stream
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        out = rf.linear_w4a16(xd, wp, sd)
    for i in range(4):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        assert torch.equal(rf.linear_w4a16(xd, wp, sd), eager)
    check(out.cpu().numpy(), x, q, s, label=f"w4 graph {m}x{n}x{k} gs={gs}")


def _random_int4_launches(seed=4100, count=24):
    """Packed int4 over seeded random shapes: M 1..64 (GEMV) and a few GEMM
    rows, 16..2048 strips, K a multiple of 64 (K % 128 == 64 included),
    per-channel and group-wise scales."""
    rng = np.random.default_rng(seed)
    ms = [1, 2, 3, 4, 5, 8, 9, 12, 16, 24, 32, 48, 64, 96, 200]
    out = []
    for i in range(count):
        m = int(rng.choice(ms))
        n = int(rng.integers(1, 2049)) * 16
        k = int(rng.integers(1, 49)) * 64
        gs = int(rng.choice([0, 32, 64, 128]))
        if gs and k % gs:
            gs = 32
        out.append((i, m, n, k, gs))
    return out


@pytest.mark.parametrize("case", _random_int4_launches(),
                         ids=lambda c: f"r{c[0]}-{c[1]}x{c[2]}x{c[3]}-g{c[4]}")
def test_w4a16_random_shapes(case):
    i, m, n, k, gs = case
    _say(f"w4a16 random {i}: M={m} N={n} K={k} gs={gs}")
    q, s = make_w4(n, k, gs, 40 + i)
    x = o8.make_activation(o8.derive_seed(40, "x4r", i, m, k), m, k)
    y = run(x, q, s)
    rows = None if m <= 16 else np.r_[0:8, m - 8:m]
    check(y, x, q, s, label=f"w4 random {m}x{n}x{k} gs={gs}", rows=rows)



# Group-wise launches of >= 16 MiB of weights with 32- or 64-wide groups run
# with each XCD's workgroups on one contiguous strip range: a workgroup count
# with a remainder mod 8 (1025, 129, 188), a ragged last group (257 strips,
# two per workgroup), and K splits of 2 and 4.
XCD_GROUPED = [
    (1, 16400, 2048, 32), (16, 4112, 8192, 32), (12, 6000, 6144, 32),
    (16, 4096, 12288, 32), (16, 2048, 16384, 64), (5, 16384, 2048, 64),
]


@pytest.mark.parametrize("m,n,k,gs", XCD_GROUPED)
def test_w4a16_xcd_grouped_launches(m, n, k, gs):
    _say(f"w4a16 xcd-grouped M={m} N={n} K={k} gs={gs}")
    assert n * k // 2 >= 16 << 20
    q, s = make_w4(n, k, gs, 5)
    x = o8.make_activation(o8.derive_seed(5, "x4x", m, n, k), m, k)
    packed = rf.pack_weight_int4(_dev(q))
    y = run(x, q, s, packed=packed)
    check(y, x, q, s, label=f"w4 xcd {m}x{n}x{k} gs={gs}")
    y2 = run(x, q, s, packed=packed)
    assert (y.view(np.uint16) == y2.view(np.uint16)).all()


@pytest.mark.parametrize("gs", [0, 32])
def test_w4a16_workspace_grows_on_a_fresh_stream(gs):
    """A 5-way split int4 GEMM (256, 4096, 8192) needs 20 MB of workspace; on a
    fresh stream (16 MB default) the first call is refused, the buffer grown
    and the call repeated: bit-identical to the default stream's result, which
    is checked against the oracle on sampled rows."""
    m, n, k = 256, 4096, 8192
    fmt = 2 if gs else 1
    assert capi.plan(m, [n], k, fmt=fmt, cus=256)["workspace_bytes"] > (16 << 20)
    _say(f"w4a16 workspace growth M={m} N={n} K={k} gs={gs}")
    q, s = make_w4(n, k, gs, 6)
    x = o8.make_activation(o8.derive_seed(6, "x4w", m, k), m, k)
    packed, xd, sd = rf.pack_weight_int4(_dev(q)), _dev(x), _dev(s)
    ref = rf.linear_w4a16(xd, packed, sd)
    torch.cuda.synchronize()
    with fresh_hip_stream() as stream:
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            y = rf.linear_w4a16(xd, packed, sd)
        torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)
    check(ref.cpu().numpy(), x, q, s, label=f"w4 workspace growth gs={gs}", rows=np.r_[0:8, m - 8:m])


# Several packed-int4 projections in one launch (w4a16.linear_multi): the
# Qwen3-8B q/k/v and gate/up groups at decode and prefill sizes, per-channel
# and group-wise, a GEMV launch with a K split (long K, few strips) and one
# with a group-wise XCD strip range (>= 16 MiB), and biases on some
# projections.  Each output is checked against the oracle; the projections
# sharing x also run as single launches, which must agree within the bar.
MULTI = [
    (1, [4096, 1024, 1024], 4096, 0), (1, [4096, 1024, 1024], 4096, 32),
    (16, [4096, 1024, 1024], 4096, 128), (4, [12288, 12288], 4096, 0),
    (16, [12288, 12288], 4096, 32), (64, [2048, 512], 1024, 32),
    (3, [1024, 512], 16384, 0), (300, [1024, 512, 512], 2048, 32),
    (130, [2048, 1024], 1024, 0),
]


@pytest.mark.parametrize("m,ns,k,gs", MULTI)
def test_w4a16_linear_multi(m, ns, k, gs):
    fmt = 2 if gs else 1
    plan = capi.plan(m, ns, k, fmt=fmt)
    _say(f"w4a16 multi M={m} Ns={ns} K={k} gs={gs}: {plan['name']} splits {plan['splits']}")
    x = o8.make_activation(o8.derive_seed(9, "x4m", m, k), m, k)
    ws, packed, scales, biases = [], [], [], []
    for i, n in enumerate(ns):
        w = o8.make_weight(o8.derive_seed(9, "w4m", i, n, k), n, k)
        q, s = o4.quantize_int4_group_wise(w, gs) if gs else o4.quantize_int4_per_channel(w)
        b = (o8.make_activation(o8.derive_seed(9, "b4m", i, n), 1, n)[0] * 0.1
             if i == 1 else None)
        ws.append((q, s, b))
        packed.append(rf.pack_weight_int4(_dev(q)))
        scales.append(_dev(s))
        biases.append(None if b is None else _dev(b))
    xd = _dev(x)
    ys = rf.linear_multi_w4a16(xd, packed, scales, biases)
    torch.cuda.synchronize()
    for i, ((q, s, b), y) in enumerate(zip(ws, ys)):
        assert y.shape == (m, ns[i])
        got = y.cpu().numpy()
        check(got, x, q, s, b, label=f"multi proj {i} N={ns[i]}")
        single = rf.linear_w4a16(xd, packed[i], scales[i], biases[i]).cpu().numpy()
        check(single, x, q, s, b, label=f"single proj {i} N={ns[i]}")
    # deterministic: the split-K counters were left zero, same plan, same sums
    again = rf.linear_multi_w4a16(xd, packed, scales, biases)
    for a, b in zip(ys, again):
        assert torch.equal(a, b)
