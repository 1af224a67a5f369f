"""CPU tests of bench.py's work accounting and its command-line contract.

The headline rates are algorithmic work over time, so the byte and FLOP
counts they divide are pinned here against values worked out by hand from
the per-launch definition B = N*K (int8 weight) + 2N (fp16 scale) + 2MK (fp16
activations) + 2MN (fp16 outputs), F = 2MNK, on the BASELINE configurations.
"""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402  (imports no GPU code at module level)


@pytest.mark.parametrize("m,n,k,mb", [
    (1, 3072, 1024, 3.160064),          # cfg0
    (1, 12288, 4096, 50.388992),        # cfg1 gate at M = 1
    (1, 151936, 5120, 778.530304),      # cfg2 lm_head, M = 1
    (8, 151936, 5120, 780.729088),      # cfg2 lm_head, M = 8
    (2048, 12288, 4096, 117.465088),    # cfg3 gate (or up)
    (32, 25600, 5120, 133.08928),       # cfg4 gate at M = 32
    (512, 25600, 5120, 162.58048),      # cfg4 gate at M = 512
])
def test_launch_bytes(m, n, k, mb):
    assert bench.nbytes(m, n, k) == round(mb * 1e6)


def test_bias_adds_its_vector():
    assert bench.nbytes(4, 4096, 4096, bias=True) - bench.nbytes(4, 4096, 4096) == 2 * 4096


@pytest.mark.parametrize("m,mb", [(1, 193.16736), (16, 195.44064)])
def test_cfg1_layer_bytes(m, mb):
    """The seven Qwen3-8B projections at one batch size."""
    assert sum(bench.nbytes(m, n, k) for _, n, k in bench.QWEN3_8B) == round(mb * 1e6)


def test_fused_launch_reads_the_shared_input_once():
    for m in bench.DECODE_M:
        for idxs in bench.DECODE_GROUPS:
            k = bench.QWEN3_8B[idxs[0]][2]
            separate = sum(bench.nbytes(m, bench.QWEN3_8B[i][1], k) for i in idxs)
            assert bench.group_bytes(m, idxs) == separate - (len(idxs) - 1) * 2 * m * k
    # the fused step covers every projection exactly once
    assert sorted(i for g in bench.DECODE_GROUPS for i in g) == list(range(len(bench.QWEN3_8B)))


def test_decode_step_bytes_per_launch():
    """The roofline's algorithmic bytes per launch: the fused step's bytes over
    its 12 launches (48,476,160 B on the BASELINE shapes)."""
    total = sum(bench.group_bytes(m, g) for m in bench.DECODE_M for g in bench.DECODE_GROUPS)
    launches = len(bench.DECODE_M) * len(bench.DECODE_GROUPS)
    assert launches == 12
    assert total / launches == 48_476_160


def test_prefill_step_flops():
    flops = sum(2 * bench.PREFILL_M * n * k for _, n, k in bench.PREFILL)
    assert flops == 2 * 2048 * (12288 * 4096 * 2 + 4096 * 12288)
    assert abs(flops - 6.185e11) / 6.185e11 < 1e-3


def test_w4_bytes_halve_the_weight():
    # per-channel: N*K/2 packed int4 weights + 2N scales; group-wise adds 2N*K/gs
    assert bench.nbytes_w4(1, 4096, 4096, 0) == 4096 * 4096 // 2 + 2 * 4096 + 2 * 4096 + 2 * 4096
    assert bench.nbytes_w4(1, 4096, 4096, 32) - bench.nbytes_w4(1, 4096, 4096, 0) == \
        2 * 4096 * (4096 // 32) - 2 * 4096


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
