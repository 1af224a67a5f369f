"""pytest configuration: the `gpu` marker and shared helpers.

`-m "not gpu"` runs the CPU suite (oracle, host logic, C-ABI exports, op
schemas and error paths); `-m gpu` runs the parity tests on an MI355X.
"""
from __future__ import annotations

import contextlib
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) HIP device")


def pytest_collection_modifyitems(config, items):
    gpu_items = [it for it in items if "gpu" in it.keywords]
    if not gpu_items:
        return
    import torch

    if not torch.cuda.is_available():
        skip = pytest.mark.skip(reason="no HIP device visible")
        for it in gpu_items:
            it.add_marker(skip)


@contextlib.contextmanager
def fresh_hip_stream():
    """A HIP stream made with hipStreamCreate (through the HIP runtime torch
    loaded) and wrapped for torch: unlike torch.cuda.Stream(), which hands
    out streams from a fixed pool, its handle is new to the W8A16 op's
    per-stream workspace cache.  Synchronized and destroyed on exit."""
    import ctypes
    import os

    import torch

    hip = ctypes.CDLL(os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so"))
    handle = ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(handle)) == 0
    try:
        yield torch.cuda.ExternalStream(handle.value)
    finally:
        assert hip.hipStreamSynchronize(handle) == 0
        assert hip.hipStreamDestroy(handle) == 0
