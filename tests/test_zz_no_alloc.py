"""The no-allocation entry point against the one it varies (MI355X only).

rf_w8a16_linear_multi_noalloc runs the kernels of rf_w8a16_linear_multi with
the split-K counters and partials in the library's fixed scratch array
instead of a caller workspace.  Both are called through the C ABI (ctypes) on
the same inputs; the kernels and their reduction order are the same, so the
outputs must be equal bit for bit (stronger than the parity bar, which the
first call also meets against the oracle).  Two calls in a row, the second on
a smaller input; shapes chosen so that both kernels take their K-split paths
(the paths that use the scratch).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import rhinoforge_amd as rf
from rhinoforge_amd import capi
from oracle import w8a16 as o

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(*a):
    print(*a, flush=True)


def _case(m, ns, k, seed):
    x = o.make_activation(o.derive_seed(seed, "x", m, k), m, k)
    ws = []
    for i, n in enumerate(ns):
        q, s = o.quantize_linear_per_channel(o.make_weight(o.derive_seed(seed, "w", i, n, k), n, k))
        ws.append((q, s, rf.pack_weight(torch.from_numpy(q).to(DEV)), torch.from_numpy(s).to(DEV)))
    return x, ws


def _run(entry, x, ws, kernel):
    """Outputs of one call of `entry` ("workspace" or "noalloc"); returns (status, outputs)."""
    lib = capi.load()
    m, k = x.shape
    xd = torch.from_numpy(x).to(DEV)
    ns = [w[0].shape[0] for w in ws]
    outs = [torch.full((m, n), float("nan"), dtype=torch.float16, device=DEV) for n in ns]
    arr = (capi.Proj * len(ns))()
    for i, ((_, _, wp, sd), y) in enumerate(zip(ws, outs)):
        arr[i] = capi.Proj(wp.data_ptr(), sd.data_ptr(), None, y.data_ptr(), ns[i], ns[i])
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if entry == "noalloc":
        st = lib.rf_w8a16_linear_multi_noalloc(xd.data_ptr(), k, capi.LAYOUT_TILE16X64, arr,
                                               len(ns), m, k, kernel, stream)
    else:
        nsc = (ctypes.c_int64 * len(ns))(*ns)
        wsb = lib.rf_w8a16_workspace_bytes_multi(m, nsc, len(ns), k)
        wsd = torch.zeros(wsb, dtype=torch.uint8, device=DEV)
        st = lib.rf_w8a16_linear_multi(xd.data_ptr(), k, capi.LAYOUT_TILE16X64, arr, len(ns), m,
                                       k, kernel, wsd.data_ptr(), wsb, stream)
    torch.cuda.synchronize()
    return st, outs


# (first call, second smaller call): (M, output widths, K, kernel).  Every
# call's plan splits K, so every call uses the scratch (asserted below).
SEQUENCES = [
    # GEMV: M=16, K=12288 takes a 4-way K split; then M=4, one 1024-wide weight
    # with K=16384 (64 strips, 256 K blocks: 8-way split)
    ((16, [1024, 512, 256], 12288, capi.KERNEL_AUTO), (4, [1024], 16384, capi.KERNEL_AUTO)),
    # GEMM: M=512 k/v-like (64 tiles of 128x128: two K groups, 4-way K split)
    # then M=128, one weight (64x64 tiles, two K groups, 4-way split)
    ((512, [1024, 1024], 5120, capi.KERNEL_AUTO), (128, [1024], 4096, capi.KERNEL_GEMM)),
    # the mid-M GEMM tiles (M <= 64, K split to ~3 workgroups per CU), forced
    ((40, [2048, 1024], 4096, capi.KERNEL_GEMM), (24, [1024], 2048, capi.KERNEL_GEMM)),
]


@pytest.mark.parametrize("seq", range(len(SEQUENCES)))
def test_noalloc_matches_workspace_entry_point(seq):
    for call, (m, ns, k, kernel) in enumerate(SEQUENCES[seq]):
        _say(f"noalloc seq {seq} call {call}: M={m} Ns={ns} K={k} kernel={kernel}")
        plan = capi.plan(m, ns, k, kernel=kernel)
        assert plan["splits"] > 1 and plan["workspace_bytes"] > 0, plan  # uses the scratch
        x, ws = _case(m, ns, k, seed=100 * seq + call)
        st, ref = _run("workspace", x, ws, kernel)
        capi.check(st, "rf_w8a16_linear_multi")
        st, got = _run("noalloc", x, ws, kernel)
        capi.check(st, "rf_w8a16_linear_multi_noalloc")
        for (q, s, _, _), a, b in zip(ws, got, ref):
            assert torch.equal(a, b)
            rep = o.check_tolerance(a.cpu().numpy(), o.cpu_path(x, q, s), o.oracle_fp64(x, q, s))
            _say(f"  {rep}")
            assert rep.ok, str(rep)
    # the first sequence again: the scratch kept the last call's contents, the
    # counters were left zero, so a repeat is bit-identical
    m, ns, k, kernel = SEQUENCES[seq][0]
    x, ws = _case(m, ns, k, seed=100 * seq)
    _, ref = _run("workspace", x, ws, kernel)
    st, got = _run("noalloc", x, ws, kernel)
    capi.check(st, "rf_w8a16_linear_multi_noalloc repeat")
    for a, b in zip(got, ref):
        assert torch.equal(a, b)


def test_noalloc_refuses_shapes_beyond_its_scratch():
    """A prefill launch whose K split needs ~84 MB of partials (2048 x 5120 x 25600:
    640 tiles of 128x128 in two splits) is refused before launch with ESCRATCH;
    the workspace entry point runs it."""
    m, n, k = 2048, 5120, 25600
    lib = capi.load()
    xd = torch.zeros(m, k, dtype=torch.float16, device=DEV)
    wp = torch.zeros(rf.packed_shape(n, k), dtype=torch.int8, device=DEV)
    sd = torch.ones(n, dtype=torch.float16, device=DEV)
    y = torch.full((m, n), float("nan"), dtype=torch.float16, device=DEV)
    arr = (capi.Proj * 1)(capi.Proj(wp.data_ptr(), sd.data_ptr(), None, y.data_ptr(), n, n))
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    nsc = (ctypes.c_int64 * 1)(n)
    assert lib.rf_w8a16_workspace_bytes_multi(m, nsc, 1, k) > capi.NOALLOC_SCRATCH_BYTES
    st = lib.rf_w8a16_linear_multi_noalloc(xd.data_ptr(), k, capi.LAYOUT_TILE16X64, arr, 1, m, k,
                                           capi.KERNEL_AUTO, stream)
    torch.cuda.synchronize()
    assert st == capi.ESCRATCH, capi.status_str(st)
    assert torch.isnan(y).all()  # nothing ran
    assert "noalloc" in capi.status_str(st)


# Run in a fresh interpreter, so that the captured call below is the first
# no-allocation call of the process (the one that looks up the scratch array).
_CAPTURED_FIRST_CALL = r"""
import ctypes, sys
sys.path.insert(0, sys.argv[1])
import torch
import rhinoforge_amd as rf
from rhinoforge_amd import capi
from oracle import w8a16 as o

m, ns, k = 4, [1024], 16384                 # GEMV with an 8-way K split
assert capi.plan(m, ns, k)["splits"] > 1
lib = capi.load()
x = torch.from_numpy(o.make_activation(7, m, k)).cuda()
q, s = o.quantize_linear_per_channel(o.make_weight(8, ns[0], k))
wp, sd = rf.pack_weight(torch.from_numpy(q).cuda()), torch.from_numpy(s).cuda()
ref = rf.linear(x, wp, sd)                  # the workspace path (torch op)
y = torch.full((m, ns[0]), float("nan"), dtype=torch.float16, device="cuda")
arr = (capi.Proj * 1)(capi.Proj(wp.data_ptr(), sd.data_ptr(), None, y.data_ptr(), ns[0], ns[0]))
torch.cuda.synchronize()
side = torch.cuda.Stream()
g = torch.cuda.CUDAGraph()
dump = hasattr(g, "enable_debug_mode")
if dump:
    g.enable_debug_mode()
st = []
with torch.cuda.graph(g, stream=side):
    st.append(lib.rf_w8a16_linear_multi_noalloc(x.data_ptr(), k, capi.LAYOUT_TILE16X64, arr, 1,
                                                m, k, capi.KERNEL_AUTO,
                                                ctypes.c_void_p(side.cuda_stream)))
capi.check(st[0], "captured first rf_w8a16_linear_multi_noalloc")
torch.cuda.synchronize()
assert torch.isnan(y).all()                 # captured, not run
for rep in range(3):
    y.fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(y, ref), f"replay {rep}"
    # eager no-allocation calls between replays share the counters
    y2 = torch.full_like(y, float("nan"))
    arr2 = (capi.Proj * 1)(capi.Proj(wp.data_ptr(), sd.data_ptr(), None, y2.data_ptr(), ns[0], ns[0]))
    capi.check(lib.rf_w8a16_linear_multi_noalloc(x.data_ptr(), k, capi.LAYOUT_TILE16X64, arr2, 1,
                                                 m, k, capi.KERNEL_AUTO,
                                                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
               "eager rf_w8a16_linear_multi_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(y2, ref), f"eager call after replay {rep}"
kernels = None
if dump:
    import os, tempfile
    path = os.path.join(tempfile.mkdtemp(), "g.dot")
    try:
        g.debug_dump(path)
        kernels = open(path).read()
    except Exception as e:  # no graph dump on this build: the counter check above stands
        print("no graph dump:", e)
if kernels is not None:
    assert "gemv" in kernels and "zero_u4" not in kernels, "the first-call fill was captured"
print("captured first call ok", "(graph dump checked)" if kernels is not None else "")
"""


def test_noalloc_first_call_under_graph_capture():
    """The first no-allocation call of a process made under HIP graph capture:
    it records the GEMV (8-way K split) and no counter fill, so every replay,
    with eager no-allocation calls in between, matches the workspace entry
    point bit for bit."""
    import subprocess
    import sys
    from pathlib import Path
    root = str(Path(__file__).resolve().parents[1])
    _say("noalloc: first call under graph capture (fresh process)")
    res = subprocess.run([sys.executable, "-c", _CAPTURED_FIRST_CALL, root], capture_output=True,
                         text=True, timeout=110)
    _say(res.stdout[-2000:] + res.stderr[-2000:])
    assert res.returncode == 0, res.stderr[-3000:]
    assert "captured first call ok" in res.stdout
