"""ctypes binding of the C ABI in include/w8a16.h.

This is the binding a Python host (such as the reference's runtime) would add
to call the library without the torch op.  It loads ``lib/librf_w8a16.so``;
import torch first in processes that use the GPU, so that the HIP runtime
torch ships is the one the library binds to.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "librf_w8a16.so"

OK = 0
EINVAL = 1
EALIGN = 2
ELAYOUT = 3
EWORKSPACE = 4
EHIP = 5
EDEVICE = 6
EKERNEL = 7
ESCRATCH = 8
NOALLOC_SCRATCH_BYTES = 32 << 20
LAYOUT_ROWMAJOR = 0
LAYOUT_TILE16X64 = 1
KERNEL_AUTO = 0
KERNEL_GEMV = 1
KERNEL_GEMM = 2
WS_COUNTER_BYTES = 65536
MAX_PROJ = 4


FORMAT_INT8 = 0
FORMAT_INT4 = 1
FORMAT_INT4_GROUP = 2


class Proj(ctypes.Structure):
    """struct rf_w8a16_proj (include/w8a16.h)."""
    _fields_ = [("w_packed", ctypes.c_void_p), ("scale", ctypes.c_void_p),
                ("bias", ctypes.c_void_p), ("y", ctypes.c_void_p),
                ("ldy", ctypes.c_int64), ("N", ctypes.c_int64)]


class PlanInfo(ctypes.Structure):
    """struct rf_w8a16_plan_info (include/w8a16.h)."""
    _fields_ = [("kernel", ctypes.c_int32), ("tile_m", ctypes.c_int32),
                ("tile_n", ctypes.c_int32), ("splits", ctypes.c_int32),
                ("waves", ctypes.c_int32), ("workgroups", ctypes.c_int32),
                ("workspace_bytes", ctypes.c_uint64), ("name", ctypes.c_char * 48)]

# name -> (restype, argtypes): every entry point declared in include/w8a16.h
_c = ctypes
SIGNATURES = {
    "rf_w8a16_status_str": (_c.c_char_p, [_c.c_int]),
    "rf_w8a16_abi_version": (_c.c_int, []),
    "rf_w8a16_packed_bytes": (_c.c_size_t, [_c.c_int64, _c.c_int64]),
    "rf_w8a16_pack_weight": (_c.c_int, [_c.c_void_p, _c.c_int64, _c.c_int64, _c.c_int64,
                                        _c.c_void_p, _c.c_size_t]),
    "rf_w8a16_unpack_weight": (_c.c_int, [_c.c_void_p, _c.c_int64, _c.c_int64, _c.c_void_p,
                                          _c.c_int64]),
    "rf_w8a16_pack_weight_device": (_c.c_int, [_c.c_void_p, _c.c_int64, _c.c_int64, _c.c_int64,
                                               _c.c_void_p, _c.c_size_t, _c.c_void_p]),
    "rf_w8a16_select_kernel": (_c.c_int, [_c.c_int64, _c.c_int64, _c.c_int64]),
    "rf_w8a16_plan": (_c.c_int, [_c.c_int64, _c.POINTER(_c.c_int64), _c.c_int32, _c.c_int64,
                                 _c.c_int32, _c.c_int32, _c.c_int32, _c.POINTER(PlanInfo)]),
    "rf_w8a16_workspace_bytes": (_c.c_size_t, [_c.c_int64, _c.c_int64, _c.c_int64]),
    "rf_w8a16_workspace_bytes_multi": (_c.c_size_t, [_c.c_int64, _c.POINTER(_c.c_int64), _c.c_int32,
                                                     _c.c_int64]),
    "rf_w8a16_linear_multi": (_c.c_int, [_c.c_void_p, _c.c_int64, _c.c_int32, _c.POINTER(Proj),
                                         _c.c_int32, _c.c_int64, _c.c_int64, _c.c_int32,
                                         _c.c_void_p, _c.c_size_t, _c.c_void_p]),
    "rf_w8a16_linear_multi_noalloc": (_c.c_int, [_c.c_void_p, _c.c_int64, _c.c_int32,
                                                 _c.POINTER(Proj), _c.c_int32, _c.c_int64,
                                                 _c.c_int64, _c.c_int32, _c.c_void_p]),
    "rf_w8a16_linear": (_c.c_int, [_c.c_void_p, _c.c_int64, _c.c_void_p, _c.c_int32,
                                   _c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_int64,
                                   _c.c_int64, _c.c_int64, _c.c_int64, _c.c_int32,
                                   _c.c_void_p, _c.c_size_t, _c.c_void_p]),
    "rf_w8a16_linear_argmax": (_c.c_int, [_c.c_void_p, _c.c_int64, _c.c_void_p, _c.c_int32,
                                          _c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_int64,
                                          _c.c_void_p, _c.c_int64, _c.c_int64, _c.c_int64,
                                          _c.c_void_p, _c.c_size_t, _c.c_void_p]),
    "rf_w8a16_workspace_bytes_argmax": (_c.c_size_t, [_c.c_int64, _c.c_int64, _c.c_int64]),
    "rf_w4a16_packed_bytes": (_c.c_size_t, [_c.c_int64, _c.c_int64]),
    "rf_w4a16_pack_weight": (_c.c_int, [_c.c_void_p, _c.c_int64, _c.c_int64, _c.c_int64,
                                        _c.c_void_p, _c.c_size_t]),
    "rf_w4a16_unpack_weight": (_c.c_int, [_c.c_void_p, _c.c_int64, _c.c_int64, _c.c_void_p,
                                          _c.c_int64]),
    "rf_w4a16_pack_weight_device": (_c.c_int, [_c.c_void_p, _c.c_int64, _c.c_int64, _c.c_int64,
                                               _c.c_void_p, _c.c_size_t, _c.c_void_p]),
    "rf_w4a16_workspace_bytes": (_c.c_size_t, [_c.c_int64, _c.c_int64, _c.c_int64]),
    "rf_w4a16_workspace_bytes_multi": (_c.c_size_t, [_c.c_int64, _c.POINTER(_c.c_int64), _c.c_int32,
                                                     _c.c_int64]),
    "rf_w4a16_linear_multi": (_c.c_int, [_c.c_void_p, _c.c_int64, _c.POINTER(Proj), _c.c_int32,
                                         _c.c_int32, _c.c_int64, _c.c_int64, _c.c_int32,
                                         _c.c_void_p, _c.c_size_t, _c.c_void_p]),
    "rf_w4a16_linear": (_c.c_int, [_c.c_void_p, _c.c_int64, _c.c_void_p, _c.c_void_p,
                                   _c.c_int32, _c.c_void_p, _c.c_void_p, _c.c_int64,
                                   _c.c_int64, _c.c_int64, _c.c_int64, _c.c_int32,
                                   _c.c_void_p, _c.c_size_t, _c.c_void_p]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load the C-ABI library (once) and declare every signature."""
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            raise OSError(f"{LIB_PATH} not built; run `python rhinoforge_amd/_build.py`")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


class W8A16Error(RuntimeError):
    def __init__(self, status: int, what: str) -> None:
        self.status = status
        super().__init__(f"{what}: {status_str(status)} (status {status})")


def status_str(status: int) -> str:
    return load().rf_w8a16_status_str(status).decode()


def check(status: int, what: str) -> None:
    if status != OK:
        raise W8A16Error(status, what)


def plan(m: int, ns, k: int, kernel: int = KERNEL_AUTO, fmt: int = FORMAT_INT8,
         cus: int = 0) -> dict:
    """The launch plan of a call (rf_w8a16_plan): kernel, tile, K splits,
    workgroups, workspace bytes and the configuration's name.  ``ns``: the
    output width, or the widths of projections sharing the input; ``cus``: the
    compute units to plan for (0: the current device's)."""
    ns = [int(n) for n in (ns if isinstance(ns, (list, tuple)) else [ns])]
    arr = (ctypes.c_int64 * len(ns))(*ns)
    info = PlanInfo()
    check(load().rf_w8a16_plan(m, arr, len(ns), k, kernel, fmt, cus, ctypes.byref(info)),
          "rf_w8a16_plan")
    return {"kernel": "gemv" if info.kernel == KERNEL_GEMV else "gemm", "tile_m": info.tile_m,
            "tile_n": info.tile_n, "splits": info.splits, "waves": info.waves,
            "workgroups": info.workgroups, "workspace_bytes": int(info.workspace_bytes),
            "name": info.name.decode()}
