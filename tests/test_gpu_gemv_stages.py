"""GPU parity of the decode GEMV's one-m-tile pipeline at every stage count it
treats differently (MI355X only).

A wavefront of a one-m-tile GEMV instance (M <= 16) streams its weight tiles
in stages of U tiles: one stage runs the plain loop; two or more run both
prologue stages and every refill unconditionally, a steady-state loop of two
full stages per iteration, then a peeled tail of two or three stages whose
last may be partial.  Within one workgroup the wavefronts can differ by one
tile, so one launch mixes stage counts.  Each case below names the plan it
must get (rf_w8a16_plan on a 256-CU part) and the stage counts its wavefronts
run; int8 and packed int4 (per-channel and group-wise) share the pipeline.
Same bar as the rest of the GPU suite: max|y - y_cpu| <= 1e-2 * rms(y_cpu),
cosine >= 0.9999 against the fp64 oracle, finite outputs, and a second call
bit-identical to the first.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import rhinoforge_amd as rf
from rhinoforge_amd import capi
from oracle import w4a16 as o4
from oracle import w8a16 as o

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(*a):
    print(*a, flush=True)


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


# (M, N, K, plan name, K splits, stages per wavefront (U tiles each)).
INT8_CASES = [
    # x in LDS, W=8 U=4, 131 K blocks: waves 0-2 run 17 tiles (5 stages, the
    # last of one tile), the rest 16 (4 full stages)
    (1, 512, 8384, "gemv 1x1 strips, 8 waves, x in LDS", 1, "5 / 4"),
    # x in LDS with a 2-way K split (65 + 64 blocks, the K tail, K % 64 = 8,
    # in the second), W=8 U=4: 9 / 8 tiles in the first split, 8 in the second
    (4, 512, 8200, "gemv 1x1 strips, 8 waves, x in LDS", 2, "3 / 2"),
    # two strips, W=8 U=2, 2-way K split of 197 blocks (99 + 98): 13 / 12 tiles
    (16, 4096, 12608, "gemv 1x2 strips, 8 waves", 2, "7 / 6"),
    # x in LDS, 80 blocks over 8 waves: 10 tiles = 4 + 4 + 2
    (1, 4096, 5120, "gemv 1x1 strips, 8 waves, x in LDS", 1, "3"),
    # two strips, W=8 U=2, 81 blocks: wave 0 11 tiles (6 stages, last partial), the rest 10 (5)
    (16, 5120, 5184, "gemv 1x2 strips, 8 waves", 1, "6 / 5"),
    # three strips, W=8 U=2, 64 blocks: 8 tiles, 4 stages
    (8, 24576, 4096, "gemv 1x3 strips, 8 waves", 1, "4"),
    # W=16 U=2, ragged N (256 strips, the last partial) and K tail, 66 blocks: 5 / 4 tiles
    (3, 4090, 4168, "gemv 1x1 strips, 16 waves", 1, "3 / 2"),
]


@pytest.mark.parametrize("case", INT8_CASES, ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}")
def test_int8_stage_counts(case):
    m, n, k, name, splits, stages = case
    p = capi.plan(m, [n], k, kernel=capi.KERNEL_GEMV, cus=256)
    assert (p["name"], p["splits"]) == (name, splits), p
    _say(f"int8 M={m} N={n} K={k}: {name}, {splits} split(s), stages {stages}")
    seed = o.derive_seed(31, "stages", m, n, k)
    q, s = o.quantize_linear_per_channel(o.make_weight(seed, n, k))
    x = o.make_activation(seed + 1, m, k)
    b = (o.normal(seed + 2, (n,)) * 0.1).astype(np.float16)
    wp = rf.pack_weight(_dev(q))
    ys = []
    for _ in range(2):
        y = rf.linear(_dev(x), wp, _dev(s), _dev(b), kernel=rf.KERNEL_GEMV)
        torch.cuda.synchronize()
        ys.append(y.cpu().numpy())
    rep = o.check_tolerance(ys[0], o.cpu_path(x, q, s, b), o.oracle_fp64(x, q, s, b))
    _say(f"  {rep}")
    assert rep.ok, str(rep)
    assert (ys[0].view(np.uint16) == ys[1].view(np.uint16)).all()


# (M, N, K, group size (0: per channel), plan name, K splits, stages per wavefront).
INT4_CASES = [
    # per-channel, x in LDS, W=8 U=2, 96 int4 tiles: 12 tiles, 6 stages
    (1, 4096, 12288, 0, "gemv 1x1 strips, 8 waves, x in LDS", 1, "6"),
    # per-channel, x in LDS, W=16 U=2 at M 3, 64 tiles: 4 tiles, 2 stages
    (3, 4096, 8192, 0, "gemv 1x1 strips, 16 waves, x in LDS", 1, "2"),
    # group-wise 32, W=8 U=1, 2-way split of 96 tiles: 6 tiles, 6 stages of one
    (8, 4096, 12288, 32, "gemv 1x2 strips, 8 waves", 2, "6"),
    # group-wise 32, four strips, W=8 U=1, 4-way split of 96 tiles: 3 tiles, 3 stages
    (16, 4096, 12288, 32, "gemv 1x4 strips, 8 waves", 4, "3"),
    # group-wise 128, x in LDS, W=16 U=1: 6 stages of one tile
    (2, 4096, 12288, 128, "gemv 1x1 strips, 16 waves, x in LDS", 1, "6"),
    # per-channel, W=8 U=1, 4-way split of 65 tiles (17/17/17/14), K % 128 = 64: 3 / 2 tiles
    (16, 1008, 8256, 0, "gemv 1x2 strips, 8 waves", 4, "3 / 2"),
]


@pytest.mark.parametrize("case", INT4_CASES, ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}g{c[3]}")
def test_int4_stage_counts(case):
    m, n, k, gs, name, splits, stages = case
    fmt = capi.FORMAT_INT4_GROUP if gs else capi.FORMAT_INT4
    p = capi.plan(m, [n], k, kernel=capi.KERNEL_GEMV, fmt=fmt, cus=256)
    assert (p["name"], p["splits"]) == (name, splits), p
    _say(f"int4 gs={gs} M={m} N={n} K={k}: {name}, {splits} split(s), stages {stages}")
    seed = o.derive_seed(37, "stages4", m, n, k)
    w = o.make_weight(seed, n, k)
    q, s = o4.quantize_int4_group_wise(w, gs) if gs else o4.quantize_int4_per_channel(w)
    x = o.make_activation(seed + 1, m, k)
    wp = rf.pack_weight_int4(_dev(q))
    ys = []
    for _ in range(2):
        y = rf.linear_w4a16(_dev(x), wp, _dev(s), None, kernel=rf.KERNEL_GEMV)
        torch.cuda.synchronize()
        ys.append(y.cpu().numpy())
    rep = o.check_tolerance(ys[0], o4.cpu_path(x, q, s, None), o4.oracle_fp64(x, q, s, None))
    _say(f"  {rep}")
    assert rep.ok, str(rep)
    assert (ys[0].view(np.uint16) == ys[1].view(np.uint16)).all()
