"""Build the native pieces in-tree (no JIT cache, no pip install).

* ``lib/librf_w8a16.so``       -- gfx950 HIP kernels + the C ABI (hipcc)
* ``lib/librf_w8a16_torch.so`` -- the thin torch-library op (g++ against
  the installed PyTorch-ROCm headers), linked to the C-ABI library
* ``lib/librf_bench.so``       -- bench.py's streaming-read reference kernel
  (a measurement helper, not part of the C ABI)

Every HIP translation unit is compiled with packed-FP32 VALU ops disabled
(``-Xclang -target-feature -Xclang -packed-fp32-ops``); the host pass warns
that it does not know the feature, which is harmless.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "lib"
INCLUDE = ROOT / "include"

CAPI_SOURCES = ["w8a16_capi.hip", "w8a16_gemv.hip", "w8a16_gemm.hip"]
CAPI_LIB = LIBDIR / "librf_w8a16.so"
TORCH_LIB = LIBDIR / "librf_w8a16_torch.so"
BENCH_LIB = LIBDIR / "librf_bench.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
OFFLOAD_ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print("+", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def _atomic_link(tmp: Path, dst: Path) -> None:
    os.replace(tmp, dst)


def build_capi(verbose: bool = False) -> Path:
    """Compile the HIP kernels and the C ABI into lib/librf_w8a16.so."""
    LIBDIR.mkdir(exist_ok=True)
    objs = []
    for src in CAPI_SOURCES:
        obj = LIBDIR / (Path(src).stem + ".o")
        _run([HIPCC, *HIP_FLAGS, "-I", str(INCLUDE), "-c", str(CSRC / src), "-o", str(obj)], verbose)
        objs.append(str(obj))
    tmp = CAPI_LIB.with_name(CAPI_LIB.name + f".tmp{os.getpid()}")
    _run([HIPCC, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *objs,
          "-Wl,-soname,librf_w8a16.so", "-o", str(tmp)], verbose)
    _atomic_link(tmp, CAPI_LIB)
    for o in objs:
        os.unlink(o)
    return CAPI_LIB


def _torch_paths():
    import torch  # noqa: F401  (only for its install location)
    from torch.utils import cpp_extension

    inc = cpp_extension.include_paths()
    libdir = str(Path(torch.__file__).resolve().parent / "lib")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    return inc, libdir, abi


def build_torch_op(verbose: bool = False) -> Path:
    """Compile the torch-library op (host C++) into lib/librf_w8a16_torch.so."""
    LIBDIR.mkdir(exist_ok=True)
    inc, libdir, abi = _torch_paths()
    cxx = os.environ.get("CXX", "g++")
    tmp = TORCH_LIB.with_name(TORCH_LIB.name + f".tmp{os.getpid()}")
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-DTORCH_EXTENSION_NAME=rf_w8a16_torch",
           *[f"-I{p}" for p in inc], "-I/opt/rocm/include", f"-I{INCLUDE}",
           str(CSRC / "w8a16_torch.cpp"),
           f"-L{libdir}", "-ltorch", "-ltorch_cpu", "-lc10", "-lc10_hip", "-ltorch_hip",
           f"-L{LIBDIR}", "-lrf_w8a16", "-Wl,-rpath,$ORIGIN",
           "-Wl,-soname,librf_w8a16_torch.so",
           "-o", str(tmp)]
    _run(cmd, verbose)
    _atomic_link(tmp, TORCH_LIB)
    return TORCH_LIB


def build_bench(verbose: bool = False) -> Path:
    """Compile bench.py's streaming-read helper into lib/librf_bench.so."""
    LIBDIR.mkdir(exist_ok=True)
    tmp = BENCH_LIB.with_name(BENCH_LIB.name + f".tmp{os.getpid()}")
    _run([HIPCC, *HIP_FLAGS, "-shared", str(CSRC / "bench_read.hip"),
          "-Wl,-soname,librf_bench.so", "-o", str(tmp)], verbose)
    _atomic_link(tmp, BENCH_LIB)
    return BENCH_LIB


def build_all(verbose: bool = False) -> None:
    build_capi(verbose)
    build_torch_op(verbose)
    build_bench(verbose)


if __name__ == "__main__":
    build_all(verbose="-v" in sys.argv)
    print(f"built {CAPI_LIB} and {TORCH_LIB}")
