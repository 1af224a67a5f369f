"""Host code of the C ABI under AddressSanitizer and UndefinedBehaviorSanitizer.

tests/sanitize/capi_host_check.cpp drives every entry point that runs on the
host without a GPU -- the int8 and int4 packers and their inverses on exact
size buffers, rf_w8a16_plan over a grid of shapes, formats and CU counts, the
argument refusals the compute entry points take before any device query --
and is linked against the library sources built with -fsanitize=address and
-fsanitize=undefined on the host side only (the gfx950 code objects are built
as in the product).  A planted heap overrun built with the same flags shows
that the sanitizers are live.  CPU only: nothing here touches a GPU.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

from rhinoforge_amd import _build

HERE = Path(__file__).resolve().parent

# Host-side sanitizers only: each -fsanitize= is scoped to the host pass.
SAN_FLAGS = [
    "-Xarch_host", "-fsanitize=address",
    "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=all",
    "-Xarch_host", "-fno-omit-frame-pointer",
]
COMMON = [
    f"--offload-arch={_build.OFFLOAD_ARCH}", "-O1", "-g", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(_build.INCLUDE), "-I", str(_build.CSRC),
]
ENV = {**os.environ, "ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0",
       "UBSAN_OPTIONS": "print_stacktrace=1"}


def _hipcc_or_skip():
    if shutil.which(_build.HIPCC) is None and not Path(_build.HIPCC).exists():
        pytest.skip("hipcc not available")


def _compile_all(jobs, tmp_path):
    """Compile (source, object) pairs in parallel; fail with the log."""
    procs = [(src, subprocess.Popen([_build.HIPCC, *COMMON, *SAN_FLAGS, "-c", str(src), "-o", str(obj)],
                                    stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True))
             for src, obj in jobs]
    for src, p in procs:
        out, _ = p.communicate(timeout=900)
        assert p.returncode == 0, f"{src.name}:\n{out[-3000:]}"


def _link(objs, exe):
    res = subprocess.run([_build.HIPCC, f"--offload-arch={_build.OFFLOAD_ARCH}", *SAN_FLAGS,
                          *map(str, objs), "-o", str(exe)],
                         stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=300)
    assert res.returncode == 0, res.stdout[-3000:]


def test_capi_host_code_under_asan_ubsan(tmp_path):
    _hipcc_or_skip()
    srcs = [HERE / "sanitize" / "capi_host_check.cpp"] + [_build.CSRC / s for s in _build.CAPI_SOURCES]
    objs = [tmp_path / (s.stem + ".o") for s in srcs]
    _compile_all(list(zip(srcs, objs)), tmp_path)
    exe = tmp_path / "capi_host_check"
    _link(objs, exe)
    res = subprocess.run([str(exe)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                         timeout=300, env=ENV)
    assert res.returncode == 0, res.stdout[-4000:]
    assert "OK: 0 failure(s)" in res.stdout
    assert "runtime error" not in res.stdout  # UBSan report


def test_sanitizer_flags_catch_a_planted_overrun(tmp_path):
    """The same flags on a one-byte heap overrun: ASan must stop the program."""
    _hipcc_or_skip()
    src = tmp_path / "planted.cpp"
    src.write_text(
        "#include <cstdlib>\n#include <cstdio>\n"
        "int main(int argc, char**) {\n"
        "  char* p = static_cast<char*>(std::malloc(16));\n"
        "  p[15 + argc] = 1;  // one past the end (argc == 1)\n"
        "  std::printf(\"%d\\n\", p[0]);\n  std::free(p);\n  return 0;\n}\n")
    obj = tmp_path / "planted.o"
    _compile_all([(src, obj)], tmp_path)
    exe = tmp_path / "planted"
    _link([obj], exe)
    res = subprocess.run([str(exe)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                         timeout=60, env=ENV)
    assert res.returncode != 0
    assert "heap-buffer-overflow" in res.stdout
