"""CPU tests of the host side: C-ABI exports, the packer, op schemas, errors.

No compute call reaches a GPU here.  Error paths mirror the reference's
pre-launch checks (src/ops/rpu_linear.cpp:1119-1134, rpu_linear_gemv.cpp:105-123).
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import rhinoforge_amd as rf
from rhinoforge_amd import capi
from oracle import w8a16 as o

ROOT = Path(__file__).resolve().parents[1]


def declared_functions() -> list[str]:
    text = (ROOT / "include" / "w8a16.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rf_w[48]a16_\w+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    assert declared_functions() == sorted(capi.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(capi.LIB_PATH))
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert capi.load().rf_w8a16_abi_version() == 4


def test_status_strings():
    for st in range(0, 9):
        assert capi.status_str(st)
    assert "unknown" in capi.status_str(99)


def test_packed_bytes():
    lib = capi.load()
    assert lib.rf_w8a16_packed_bytes(3072, 1024) == 3072 * 1024
    assert lib.rf_w8a16_packed_bytes(151936, 5120) == 151936 * 5120
    assert lib.rf_w8a16_packed_bytes(17, 72) == 32 * 128
    assert lib.rf_w8a16_packed_bytes(0, 64) == 0
    assert lib.rf_w8a16_packed_bytes(16, -1) == 0


def _layout_index(n, k, kblocks):
    """Byte offset of q[n][k] in TILE16X64, from the definition in include/w8a16.h."""
    nb, nl = divmod(n, 16)
    kb, kk = divmod(k, 64)
    lane = nl + 16 * (kk // 16)
    return (nb * kblocks + kb) * 1024 + lane * 16 + (kk % 16)


@pytest.mark.parametrize("n,k", [(16, 64), (17, 72), (100, 8), (48, 320), (1, 1)])
def test_pack_matches_layout_definition_and_round_trips(n, k):
    rng = np.random.default_rng(n * 1000 + k)
    q = rng.integers(-128, 128, size=(n, k), dtype=np.int8)
    packed = rf.pack_weight(torch.from_numpy(q)).numpy().view(np.uint8).ravel()
    nb, kblocks, tile = rf.packed_shape(n, k)
    assert tile == 1024 and packed.size == nb * kblocks * 1024
    # every logical element lands where the header says, stored as q XOR 0x80
    idx = np.array([[_layout_index(i, j, kblocks) for j in range(k)] for i in range(n)])
    assert (packed[idx] == (q.view(np.uint8) ^ 0x80)).all()
    # padding holds q = 0
    mask = np.ones(packed.size, bool)
    mask[idx.ravel()] = False
    assert (packed[mask] == 0x80).all()
    # inverse
    packed_t = torch.from_numpy(packed.view(np.int8).reshape(nb, kblocks, 1024))
    assert (rf.unpack_weight(packed_t, n, k).numpy() == q).all()
    # the torch-op form of the inverse (used by state_dict on the weight's device)
    assert (rf.ops.unpack_weight_on_device(packed_t, n, k).numpy() == q).all()


def test_pack_is_a_permutation_on_aligned_shapes():
    q = np.arange(32 * 128, dtype=np.int64).astype(np.uint8).view(np.int8).reshape(32, 128)
    p = rf.pack_weight(torch.from_numpy(q)).numpy().view(np.uint8).ravel()
    assert sorted((p ^ 0x80).tolist()) == sorted(q.view(np.uint8).ravel().tolist())


def test_capi_pack_argument_errors():
    lib = capi.load()
    q = np.zeros((16, 64), np.int8)
    dst = np.zeros(16 * 64, np.uint8)
    qp, dp = q.ctypes.data, dst.ctypes.data
    assert lib.rf_w8a16_pack_weight(qp, 16, 64, 64, dp, 16 * 64) == capi.OK
    assert lib.rf_w8a16_pack_weight(qp, 16, 64, 63, dp, 16 * 64) == capi.EINVAL  # ldq < K
    assert lib.rf_w8a16_pack_weight(qp, 16, 64, 64, dp, 100) == capi.EINVAL      # dst too small
    assert lib.rf_w8a16_pack_weight(None, 16, 64, 64, dp, 16 * 64) == capi.EINVAL
    assert lib.rf_w8a16_unpack_weight(dp, 0, 64, qp, 64) == capi.EINVAL


def test_capi_linear_validation_without_gpu():
    """Argument checks run before any device query; nothing is dereferenced."""
    lib = capi.load()
    fake = 1 << 20  # 16-byte aligned, never dereferenced before validation fails
    args = dict(x=fake, ldx=1024, w=fake, layout=capi.LAYOUT_TILE16X64, s=fake, b=None,
                y=fake, ldy=3072, M=1, N=3072, K=1024, kernel=0, ws=None, wsb=0, stream=None)

    def call(**kw):
        a = {**args, **kw}
        return lib.rf_w8a16_linear(a["x"], a["ldx"], a["w"], a["layout"], a["s"], a["b"], a["y"],
                                   a["ldy"], a["M"], a["N"], a["K"], a["kernel"], a["ws"],
                                   a["wsb"], a["stream"])

    assert call(x=None) == capi.EINVAL
    assert call(M=0) == capi.EINVAL
    assert call(N=0) == capi.EINVAL
    assert call(ldx=1000) == capi.EINVAL
    assert call(ldy=3000) == capi.EINVAL
    assert call(layout=capi.LAYOUT_ROWMAJOR) == capi.ELAYOUT
    assert call(K=1020, ldx=1024) == capi.EALIGN
    assert call(x=fake + 2) == capi.EALIGN
    assert call(ldx=1028) == capi.EALIGN
    assert call(kernel=7) in (capi.EINVAL, capi.EHIP, capi.EDEVICE)
    # A valid call on a machine without a gfx950 device never reports success.
    assert call() in (capi.EHIP, capi.EDEVICE)


def test_capi_linear_multi_validation_without_gpu():
    lib = capi.load()
    fake = 1 << 20

    def projs(n_list, **kw):
        arr = (capi.Proj * len(n_list))()
        for i, n in enumerate(n_list):
            arr[i] = capi.Proj(kw.get("w", fake), kw.get("s", fake), None, kw.get("y", fake),
                               kw.get("ldy", n), n)
        return arr

    def call(arr, count, M=1, K=1024, ldx=1024, x=fake, layout=capi.LAYOUT_TILE16X64):
        return lib.rf_w8a16_linear_multi(x, ldx, layout, arr, count, M, K, 0, None, 0, None)

    ok = projs([4096, 1024, 1024])
    assert call(ok, 0) == capi.EINVAL
    assert call(ok, capi.MAX_PROJ + 1) == capi.EINVAL
    assert call(None, 1) == capi.EINVAL
    assert call(projs([4096, 0]), 2) == capi.EINVAL
    assert call(projs([64], ldy=32), 1) == capi.EINVAL
    assert call(projs([64], w=None), 1) == capi.EINVAL
    assert call(ok, 3, layout=capi.LAYOUT_ROWMAJOR) == capi.ELAYOUT
    assert call(projs([64], y=fake + 1), 1) == capi.EALIGN
    assert call(ok, 3, x=fake + 8) == capi.EALIGN
    assert call(ok, 3) in (capi.EHIP, capi.EDEVICE)


def test_capi_linear_argmax_validation_without_gpu():
    lib = capi.load()
    fake = 1 << 20

    def call(M=1, N=1024, K=1024, ldx=1024, x=fake, w=fake, s=fake, y=None, ldy=0, idx=fake,
             layout=capi.LAYOUT_TILE16X64):
        return lib.rf_w8a16_linear_argmax(x, ldx, w, layout, s, None, y, ldy, idx, M, N, K,
                                          None, 0, None)

    assert call(idx=None) == capi.EINVAL
    assert call(x=None) == capi.EINVAL
    assert call(M=0) == capi.EINVAL
    assert call(y=fake, ldy=100) == capi.EINVAL
    assert call(layout=capi.LAYOUT_ROWMAJOR) == capi.ELAYOUT
    assert call(idx=fake + 2) == capi.EALIGN
    assert call(x=fake + 8) == capi.EALIGN
    assert call(M=65) == capi.EKERNEL
    assert call() in (capi.EHIP, capi.EDEVICE)
    assert lib.rf_w8a16_workspace_bytes_argmax(64, 151936, 5120) >= capi.WS_COUNTER_BYTES
    assert lib.rf_w8a16_workspace_bytes_argmax(65, 151936, 5120) == 0
    assert lib.rf_w8a16_workspace_bytes_argmax(0, 16, 16) == 0


def test_workspace_bytes_multi_matches_single():
    lib = capi.load()
    for m, n, k in [(1, 1024, 4096), (16, 4096, 12288), (9, 1000, 1024), (2048, 4096, 4096)]:
        ns = (ctypes.c_int64 * 1)(n)
        assert lib.rf_w8a16_workspace_bytes_multi(m, ns, 1, k) == lib.rf_w8a16_workspace_bytes(m, n, k)
    ns = (ctypes.c_int64 * 3)(4096, 1024, 1024)
    assert lib.rf_w8a16_workspace_bytes_multi(16, ns, 3, 4096) >= capi.WS_COUNTER_BYTES
    assert lib.rf_w8a16_workspace_bytes_multi(16, ns, 0, 4096) == 0
    assert lib.rf_w8a16_workspace_bytes_multi(16, ns, 5, 4096) == 0


def test_select_kernel_policy():
    assert rf.select_kernel(1, 4096, 4096) == rf.KERNEL_GEMV
    assert rf.select_kernel(16, 151936, 5120) == rf.KERNEL_GEMV
    # M 17..28: the GEMV only for small weights (N*K <= 2^24)
    assert rf.select_kernel(17, 4096, 4096) == rf.KERNEL_GEMV
    assert rf.select_kernel(28, 4096, 4096) == rf.KERNEL_GEMV
    assert rf.select_kernel(17, 8192, 5120) == rf.KERNEL_GEMM
    assert rf.select_kernel(29, 4096, 4096) == rf.KERNEL_GEMM
    assert rf.select_kernel(32, 1024, 5120) == rf.KERNEL_GEMV   # N*K <= 2^23
    assert rf.select_kernel(33, 1024, 5120) == rf.KERNEL_GEMM
    assert rf.select_kernel(32, 5120, 25600) == rf.KERNEL_GEMM
    assert rf.select_kernel(64, 4096, 4096) == rf.KERNEL_GEMM
    assert rf.select_kernel(65, 4096, 4096) == rf.KERNEL_GEMM
    assert rf.select_kernel(2048, 12288, 4096) == rf.KERNEL_GEMM
    with pytest.raises(RuntimeError):
        rf.select_kernel(0, 16, 16)


def test_workspace_bytes_counter_region():
    lib = capi.load()
    for m, n, k in [(1, 1024, 4096), (16, 4096, 12288), (2048, 4096, 4096)]:
        assert lib.rf_w8a16_workspace_bytes(m, n, k) >= capi.WS_COUNTER_BYTES
    assert lib.rf_w8a16_workspace_bytes(0, 16, 16) == 0


# ---------------------------------------------------------------- torch op
def test_torch_op_schemas_registered():
    for name in ("linear", "linear_into", "linear_multi", "linear_argmax", "pack_weight",
                 "unpack_weight", "select_kernel"):
        assert hasattr(torch.ops.w8a16, name)


def test_torch_op_meta_shape():
    x = torch.empty(2, 3, 1024, dtype=torch.float16, device="meta")
    w = torch.empty(rf.packed_shape(3072, 1024), dtype=torch.int8, device="meta")
    s = torch.empty(3072, dtype=torch.float16, device="meta")
    assert rf.linear(x, w, s).shape == (2, 3, 3072)


def _cpu_args(n=48, k=128):
    q = torch.randint(-127, 128, (n, k), dtype=torch.int8)
    return (torch.zeros(2, k, dtype=torch.float16), rf.pack_weight(q),
            torch.ones(n, dtype=torch.float16))


def test_torch_op_refuses_cpu_tensors():
    x, w, s = _cpu_args()
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        rf.linear(x, w, s)
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        rf.linear_into(x, w, s, None, torch.empty(2, 48, dtype=torch.float16))
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        rf.linear_multi(x, [w, w], [s, s])
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        rf.linear_argmax(x, w, s)


@pytest.mark.parametrize("bad", ["x_dtype", "w_dtype", "s_dtype", "layout"])
def test_torch_op_argument_errors(bad):
    x, w, s = _cpu_args()
    kw = {}
    if bad == "x_dtype":
        x = x.float()
    elif bad == "w_dtype":
        w = w.to(torch.uint8)
    elif bad == "s_dtype":
        s = s.float()
    else:
        kw["layout"] = rf.LAYOUT_ROWMAJOR
    with pytest.raises(RuntimeError):
        torch.ops.w8a16.linear(x, w, s, None, kw.get("layout", 1), 0)


def test_pack_weight_rejects_bad_input():
    with pytest.raises(RuntimeError):
        rf.pack_weight(torch.zeros(4, 4, dtype=torch.float16))
    with pytest.raises(RuntimeError):
        rf.pack_weight(torch.zeros(4, dtype=torch.int8))
    with pytest.raises(RuntimeError):
        rf.unpack_weight(torch.zeros(10, dtype=torch.int8), 16, 64)


# ---------------------------------------------------------------- quant (torch)
@pytest.mark.parametrize("seed", [0, 1])
def test_package_quantizer_bit_exact_vs_oracle(seed):
    w = o.make_weight(seed, 130, 300)
    w[5] = 0
    q, s = rf.quantize_linear_per_channel(torch.from_numpy(w))
    q2, s2 = o.quantize_linear_per_channel(w)
    assert q.dtype == torch.int8 and s.dtype == torch.float16
    assert (q.numpy() == q2).all() and (s.numpy().view(np.uint16) == s2.view(np.uint16)).all()
    d = rf.dequantize_linear_per_channel(q, s).numpy()
    assert (d.view(np.uint16) == o.dequantize_linear_per_channel(q2, s2).view(np.uint16)).all()


def test_w8a16_linear_module_construction_on_cpu():
    lin = torch.nn.Linear(128, 40, bias=True)
    mod = rf.W8A16Linear.from_linear(lin)
    assert mod.weight.shape == rf.packed_shape(40, 128)
    q, s = rf.quantize_linear_per_channel(lin.weight.detach())
    assert torch.equal(mod.rowmajor_weight(), q) and torch.equal(mod.weight_scale, s)
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        mod(torch.zeros(1, 128, dtype=torch.float16))


def test_kernels_spill_nothing_to_scratch(tmp_path):
    """Every gfx950 kernel fits its register budget: a spill to scratch memory
    turns a bandwidth-bound kernel into one waiting on scratch traffic (the
    compiler's resource-usage remarks, same flags as the product build)."""
    import shutil
    import subprocess
    from rhinoforge_amd import _build

    if shutil.which(_build.HIPCC) is None and not Path(_build.HIPCC).exists():
        pytest.skip("hipcc not available")
    srcs = sorted((ROOT / "rhinoforge_amd" / "csrc").glob("*.hip"))
    procs = [(src, subprocess.Popen(
        [_build.HIPCC, *_build.HIP_FLAGS, "-c", str(src), "-o", str(tmp_path / (src.stem + ".o")),
         "-Rpass-analysis=kernel-resource-usage"],
        stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)) for src in srcs]
    kernels = 0
    for src, p in procs:
        out, _ = p.communicate(timeout=600)
        assert p.returncode == 0, out[-2000:]
        name = None
        for line in out.splitlines():
            m = re.search(r"Function Name: (\S+)", line)
            if m:
                name, kernels = m.group(1), kernels + 1
            m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
            if m:
                assert int(m.group(1)) == 0, f"{src.name}: {name} uses {m.group(1)} B/lane scratch"
    assert kernels >= 20
