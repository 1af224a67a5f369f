"""CPU tests of the kernel planners through rf_w8a16_plan (the C ABI's analogue
of the reference's tile selection, src/ops/rpu_linear_tiling.h:544-595).

Each planner rule has one shape in planner_cases.py with the configuration,
tile and K splits it must get on a 256-CU part; the GPU suite runs the same
shapes for numerics.  A planner change that moves a shape to another
configuration fails here, not silently.
"""
from __future__ import annotations

import pytest

from rhinoforge_amd import capi
from planner_cases import GEMM_POLICY, GEMV_INT4_POLICY, GEMV_POLICY, STRIP_GROUP_LAUNCHES

CUS = 256  # MI355X


@pytest.mark.parametrize("row", GEMV_POLICY, ids=lambda r: f"{r[0]}x{r[1]}x{r[2]}")
def test_gemv_rule(row):
    m, n, k, name, tm, tn, splits = row
    p = capi.plan(m, n, k, kernel=capi.KERNEL_GEMV, cus=CUS)
    assert (p["name"], p["tile_m"], p["tile_n"], p["splits"]) == (name, tm, tn, splits), p
    assert (p["workspace_bytes"] > 0) == (splits > 1)


@pytest.mark.parametrize("row", GEMV_INT4_POLICY,
                         ids=lambda r: f"{r[0]}x{r[1]}x{r[2]}{'g' if r[3] else ''}")
def test_gemv_int4_rule(row):
    m, n, k, grouped, name, tm, tn, splits = row
    fmt = capi.FORMAT_INT4_GROUP if grouped else capi.FORMAT_INT4
    p = capi.plan(m, n, k, kernel=capi.KERNEL_GEMV, fmt=fmt, cus=CUS)
    assert (p["name"], p["tile_m"], p["tile_n"], p["splits"]) == (name, tm, tn, splits), p
    assert (p["workspace_bytes"] > 0) == (splits > 1)


@pytest.mark.parametrize("row", STRIP_GROUP_LAUNCHES, ids=lambda r: f"{r[0]}x{r[1]}x{r[2]}")
def test_gemv_strip_group_launches(row):
    m, ns, k, name = row
    p = capi.plan(m, ns, k, cus=CUS)
    assert (p["kernel"], p["name"], p["splits"]) == ("gemv", name, 1), p


@pytest.mark.parametrize("row", GEMM_POLICY, ids=lambda r: f"{r[0]}x{r[1]}x{r[2]}")
def test_gemm_rule(row):
    m, n, k, name, tm, tn, splits = row
    p = capi.plan(m, n, k, kernel=capi.KERNEL_GEMM, cus=CUS)
    assert (p["name"], p["tile_m"], p["tile_n"], p["splits"]) == (name, tm, tn, splits), p
    tiles = -(-m // tm) * -(-n // tn)
    assert p["workgroups"] == tiles * splits
    assert p["workspace_bytes"] == (splits * tiles * tm * tn * 4 if splits > 1 else 0)


# The BASELINE launches: which kernel AUTO runs (the GEMV <-> GEMM crossover).
BASELINE_LAUNCHES = [
    ((1, [3072], 1024), "gemv"),                   # cfg0
    ((1, [4096, 1024, 1024], 4096), "gemv"),       # cfg1 fused q/k/v, M 1 / 4 / 16
    ((16, [4096, 1024, 1024], 4096), "gemv"),
    ((16, [12288, 12288], 4096), "gemv"),          # cfg1 fused gate/up
    ((16, [4096], 12288), "gemv"),                 # cfg1 down
    ((8, [151936], 5120), "gemv"),                 # cfg2 lm_head
    ((2048, [12288, 12288], 4096), "gemm"),        # cfg3 fused gate/up
    ((2048, [4096], 12288), "gemm"),               # cfg3 down
    ((1, [25600, 25600], 5120), "gemv"),           # cfg4 at M 1 / 32 / 512
    ((32, [1024], 5120), "gemv"),                  # k/v at M 32: small weight, GEMV
    ((24, [4096, 1024, 1024], 4096), "gemv"),      # N*K < 2^25 up to M 24
    ((28, [4096, 1024, 1024], 4096), "gemm"),
    ((32, [2048], 6144), "gemv"),                  # N <= 2048, N*K <= 2^24 at M 32
    ((32, [4096], 4096), "gemm"),
    ((32, [8192], 5120), "gemm"),                  # q at M 32: mid-M GEMM tiles
    ((32, [5120], 25600), "gemm"),
    ((512, [8192, 1024, 1024], 5120), "gemm"),
]


@pytest.mark.parametrize("args,kernel", BASELINE_LAUNCHES, ids=lambda v: str(v))
def test_auto_kernel_choice_on_baseline_launches(args, kernel):
    m, ns, k = args
    assert capi.plan(m, ns, k, cus=CUS)["kernel"] == kernel


def test_cfg3_prefill_plans():
    """The two timed prefill launches: 1536 tiles of 128x256 (three rounds of
    the chip at two per CU) for fused gate/up; down: 256 tiles of 128x256, one
    eight-wavefront workgroup per CU (two K groups, B in registers)."""
    gu = capi.plan(2048, [12288, 12288], 4096, cus=CUS)
    assert (gu["name"], gu["workgroups"], gu["splits"]) == ("gemm 128x256 B-in-registers", 1536, 1)
    down = capi.plan(2048, [4096], 12288, cus=CUS)
    assert (down["name"], down["workgroups"], down["splits"], down["waves"]) == \
        ("gemm 128x256 two K groups, B-in-registers", 256, 1, 8)


def test_int4_plans_and_errors():
    p = capi.plan(16, [4096], 12288, fmt=capi.FORMAT_INT4_GROUP, cus=CUS)
    assert p["kernel"] == "gemv"
    p = capi.plan(1024, [6144], 1024, fmt=capi.FORMAT_INT4_GROUP, cus=CUS)
    assert p["name"] == "gemm 128x128 B-in-registers"  # group-wise at M >= 1024
    p = capi.plan(520, [8192], 1024, fmt=capi.FORMAT_INT4_GROUP, cus=CUS)
    assert p["name"] == "gemm 128x128 interleaved"
    # several int4 projections plan as one launch over their strips together
    p = capi.plan(1, [4096, 1024, 1024], 4096, fmt=capi.FORMAT_INT4, cus=CUS)
    assert p["kernel"] == "gemv" and p["workgroups"] == 384 // (p["tile_n"] // 16)  # 384 strips
    with pytest.raises(capi.W8A16Error):
        capi.plan(4, [64, 40], 128, fmt=capi.FORMAT_INT4, cus=CUS)  # N % 16 != 0
    with pytest.raises(capi.W8A16Error, match="cannot run"):
        capi.plan(65, [64], 128, kernel=capi.KERNEL_GEMV, cus=CUS)
