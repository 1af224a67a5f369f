"""W4A16 on the CPU: the int4 oracle pinned, the packer, the C ABI's checks.

The reference has no int4 test vectors; the known answers below are derived
by hand from IEEE binary16 rounding (worked in the comments), so a restatement
that skipped the fp16 rounding of amax/7, used fp16 instead of fp32 weights
for the group-wise amax, or rounded half away from zero would fail them.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import rhinoforge_amd as rf
from rhinoforge_amd import capi
from oracle import w4a16 as o4
from oracle import w8a16 as o8


# ---------------------------------------------------------------- quantizers

def test_per_channel_int4_kat():
    # The reference's int8 KAT matrix (tests/test_quantization.py:15-18).
    # Row 0: amax 2 -> 2/7 = 0.2857143 -> fp16 step 2^-12 on [0.25, 0.5):
    #   0.2857143 / 2^-12 = 1170.29 -> 1170 * 2^-12 = 0.28564453125.
    #   q = round(-2/s = -7.0017) = -7, round(-0.5/s = -1.7504) = -2.
    # Row 1: amax 0.5 -> 0.5/7 = 0.0714286 -> step 2^-14: 1170.29 -> 0.0714111328125;
    #   -0.25/s = -3.5009 -> -4 (not a tie), 0.5/s = 7.0017 -> 7.
    w = np.array([[-2.0, -0.5, 0.5, 2.0], [-0.25, 0.0, 0.25, 0.5]], np.float32)
    q, s = o4.quantize_int4_per_channel(w)
    assert s.tolist() == [0.28564453125, 0.0714111328125]
    assert q.tolist() == [[-7, -2, 2, 7], [-4, 0, 4, 7]]
    qt, st = rf.quantize_int4_per_channel(torch.from_numpy(w))
    assert qt.tolist() == q.tolist() and st.numpy().tolist() == s.tolist()


def test_group_wise_int4_kat():
    # group_size 4, two groups per row.
    # Group (0,0): amax 1.0 -> 1/7 = 0.142857149 (fp32) -> step 2^-13 on [0.125, 0.25):
    #   1170.29 -> 1170 * 2^-13 = 0.142822265625; q = [-7, -4, 4, 7]
    #   (0.5 / s = 3.50085: above the tie, rounds to 4).
    # Group (0,1): amax 0.7 (fp32 0.69999999) -> /7 = 0.1 -> step 2^-14 on
    #   [0.0625, 0.125): 1638.4 -> 1638 * 2^-14 = 0.0999755859375;
    #   q = [7, -4, 0, 1]  (0.7/s = 7.0017, -0.35/s = -3.50085, 0.14/s = 1.40034).
    # Row 1, group 0 is all zero: s = 2^-14, q = 0.  Group 1: amax/7 = 4.3e-6 is
    #   below 2^-14, so s clamps to 2^-14 = 6.1e-5 and q = round(w / s):
    #   1e-5/s = 0.164 -> 0, 3e-5/s = 0.49 -> 0.
    w = np.array([[-1.0, -0.5, 0.5, 1.0, 0.7, -0.35, 0.0, 0.14],
                  [0.0, 0.0, 0.0, 0.0, 1e-5, -1e-5, 3e-5, 0.0]], np.float32)
    q, s = o4.quantize_int4_group_wise(w, 4)
    assert s.shape == (2, 2)  # [G, N]
    assert s[:, 0].tolist() == [0.142822265625, 0.0999755859375]
    assert s[:, 1].tolist() == [2.0 ** -14, 2.0 ** -14]
    assert q.tolist() == [[-7, -4, 4, 7, 7, -4, 0, 1], [0] * 8]
    qt, st, gs = rf.quantize_int4_group_wise(torch.from_numpy(w), 4)
    assert gs == 4 and qt.tolist() == q.tolist() and torch.equal(st, torch.from_numpy(s))


def test_group_wise_uses_fp32_weights_not_fp16():
    # amax 7 gives s = 1.  w = 2.5 + 2^-12 is an fp32 number but not an fp16
    # one (fp16 spacing on [2, 4) is 2^-9): from fp32 it rounds to 3, while an
    # fp16 cast first (as the per-channel quantizer does) gives the tie 2.5,
    # which rounds half-even to 2.
    w = np.array([[7.0, 2.5 + 2.0 ** -12, 0.0, 0.0]], np.float32)
    q, s = o4.quantize_int4_group_wise(w, 4)
    assert s.ravel().tolist() == [1.0] and q.tolist() == [[7, 3, 0, 0]]
    qt, _, _ = rf.quantize_int4_group_wise(torch.from_numpy(w), 4)
    assert qt.tolist() == [[7, 3, 0, 0]]


def test_round_half_even_in_group_wise():
    # s = 1 (amax 7): 2.5 -> 2, 3.5 -> 4, -2.5 -> -2, -0.5 -> 0.
    w = np.array([[7.0, 2.5, 3.5, -2.5, -0.5, 0.0, 0.0, 0.0]], np.float32)
    q, _ = o4.quantize_int4_group_wise(w, 8)
    assert q.tolist() == [[7, 2, 4, -2, 0, 0, 0, 0]]


@pytest.mark.parametrize("gs", [32, 64, 128])
def test_group_wise_invariants_and_torch_agreement(gs):
    w = o8.make_weight(o8.derive_seed(4, "w4", gs), 48, 256) * 3
    w[5, :gs] = 0.0                       # an all-zero group
    q, s = o4.quantize_int4_group_wise(w, gs)
    assert q.min() >= -8 and q.max() <= 7 and s.shape == (256 // gs, 48)
    per_group = np.abs(q.reshape(48, -1, gs)).max(axis=2)
    zero = (np.abs(w.reshape(48, -1, gs)).max(axis=2) == 0)
    assert (per_group[~zero] == 7).all() and (per_group[zero] == 0).all()
    assert (s.T[zero] == np.float16(2.0 ** -14)).all()
    qt, st, _ = rf.quantize_int4_group_wise(torch.from_numpy(w), gs)
    assert np.array_equal(qt.numpy(), q) and np.array_equal(st.numpy(), s)


def test_dequant_closed_form_exhaustive():
    qs = np.arange(-8, 8, dtype=np.int8)
    for sv in [2.0 ** -14, 0.0999755859375, 0.142822265625, 1.0, 3.14159, 1000.0]:
        q = np.tile(qs, (1, 1))
        s = np.array([[sv]], np.float16)
        got = o4.dequantize_int4(q, s)
        want = (np.float64(np.float16(sv)) * qs.astype(np.float64)).astype(np.float16)
        assert np.array_equal(got.ravel(), want)
        t = rf.dequantize_int4_group_wise(torch.from_numpy(q), torch.from_numpy(s))
        assert np.array_equal(t.numpy().ravel(), want)


# ---------------------------------------------------------------- oracle

def test_cpu_path_and_fp64_unit_vectors():
    q, s = o4.quantize_int4_group_wise(o8.make_weight(3, 32, 128), 32)
    w16 = o4.dequantize_int4(q, s)
    for k in (0, 31, 32, 127):
        x = np.zeros((1, 128), np.float16)
        x[0, k] = 1.0
        assert np.array_equal(o4.cpu_path(x, q, s)[0], w16[:, k])
        assert np.allclose(o4.oracle_fp64(x, q, s)[0],
                           np.repeat(s.T.astype(np.float64), 32, axis=1)[:, k] * q[:, k])


def test_fp64_oracle_brute_force_and_single_group():
    rng = np.random.default_rng(5)
    q = rng.integers(-8, 8, (3, 64)).astype(np.int8)
    s = rng.uniform(0.01, 0.1, (2, 3)).astype(np.float16)
    x = rng.standard_normal((2, 64)).astype(np.float16)
    y = o4.oracle_fp64(x, q, s)
    for m in range(2):
        for n in range(3):
            acc = 0.0
            for k in range(64):
                acc += float(x[m, k]) * float(s[k // 32, n]) * int(q[n, k])
            assert abs(y[m, n] - acc) <= 1e-12 * max(1.0, abs(acc))
    s1 = s[:1]
    assert np.array_equal(o4.oracle_fp64(x, q, s1), o4.oracle_fp64(x, q, s1[0]))


# ---------------------------------------------------------------- layout

@pytest.mark.parametrize("n,k", [(16, 128), (32, 256), (20, 64), (17, 200), (48, 384)])
def test_pack_matches_layout_definition(n, k):
    rng = np.random.default_rng(n * 1000 + k)
    q = rng.integers(-8, 8, (n, k)).astype(np.int8)
    packed = rf.pack_weight_int4(torch.from_numpy(q))
    assert tuple(packed.shape) == rf.packed_shape_int4(n, k)
    assert np.array_equal(packed.numpy().ravel(), o4.pack_reference(q))
    assert torch.equal(rf.unpack_weight_int4(packed, n, k), torch.from_numpy(q))


def test_pack_planted_nibble_swap_is_caught(monkeypatch):
    q = np.random.default_rng(1).integers(-8, 8, (16, 128)).astype(np.int8)
    good = rf.pack_weight_int4(torch.from_numpy(q)).numpy().ravel()

    def swapped(n, k, N, K):  # a plausible mistake: nibbles in plain position order
        kk = k % 8
        return ((n // 16) * ((K + 127) // 128) + k // 128) * 1024 + \
            (n % 16 + 16 * ((k % 128) // 32)) * 16 + 4 * ((k % 32) // 8) + kk // 2, 4 * (kk % 2)

    monkeypatch.setattr(o4, "pack_index", swapped)
    assert not np.array_equal(good, o4.pack_reference(q))


def test_pack_rejects_out_of_range_values():
    with pytest.raises(RuntimeError, match=r"\[-8, 7\]"):
        rf.pack_weight_int4(torch.full((16, 64), 8, dtype=torch.int8))
    with pytest.raises(RuntimeError):
        rf.pack_weight_int4(torch.zeros(16, 64, dtype=torch.float16))


# ---------------------------------------------------------------- C ABI / op checks

def test_capi_w4a16_sizes():
    lib = capi.load()
    assert lib.rf_w4a16_packed_bytes(16, 128) == 1024
    assert lib.rf_w4a16_packed_bytes(17, 129) == 32 * 256 // 2
    assert lib.rf_w4a16_packed_bytes(0, 128) == 0
    assert lib.rf_w4a16_workspace_bytes(1, 4096, 4096) >= capi.WS_COUNTER_BYTES
    assert lib.rf_w4a16_workspace_bytes(0, 16, 64) == 0


def test_capi_w4a16_validation_without_gpu():
    lib = capi.load()
    fake = 1 << 20
    args = dict(x=fake, ldx=4096, w=fake, s=fake, gs=32, b=None, y=fake, ldy=4096, M=1,
                N=4096, K=4096, kernel=0, ws=None, wsb=0, stream=None)

    def call(**kw):
        a = {**args, **kw}
        return lib.rf_w4a16_linear(a["x"], a["ldx"], a["w"], a["s"], a["gs"], a["b"], a["y"],
                                   a["ldy"], a["M"], a["N"], a["K"], a["kernel"], a["ws"],
                                   a["wsb"], a["stream"])

    assert call(x=None) == capi.EINVAL
    assert call(s=None) == capi.EINVAL
    assert call(gs=16) == capi.EINVAL
    assert call(N=4088, ldy=4096) == capi.EINVAL        # N % 16
    assert call(K=4032, ldx=4096, gs=128) == capi.EINVAL  # K % group_size
    assert call(K=4000, ldx=4096) == capi.EINVAL        # K % 64
    assert call(x=fake + 2) == capi.EALIGN
    assert call(s=fake + 2) == capi.EALIGN               # group-wise scale: 16 B
    assert call(s=fake + 2, gs=0) in (capi.EHIP, capi.EDEVICE)  # per-channel: 2 B is enough
    assert call() in (capi.EHIP, capi.EDEVICE)


def test_w4a16_op_schema_and_cpu_refusal():
    for name in ("linear", "pack_weight", "unpack_weight"):
        assert hasattr(torch.ops.w4a16, name)
    q = torch.randint(-8, 8, (32, 128), dtype=torch.int8)
    w = rf.pack_weight_int4(q)
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        rf.linear_w4a16(torch.zeros(2, 128, dtype=torch.float16), w,
                        torch.ones(4, 32, dtype=torch.float16))
    m = rf.W4A16Linear.from_quantized(q, torch.ones(4, 32, dtype=torch.float16))
    assert m.group_size == 32 and torch.equal(m.rowmajor_weight(), q)
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        m(torch.zeros(1, 128, dtype=torch.float16))
    x = torch.empty(3, 128, dtype=torch.float16, device="meta")
    out = torch.ops.w4a16.linear(x, torch.empty(rf.packed_shape_int4(32, 128), dtype=torch.uint8,
                                                device="meta"),
                                 torch.empty(32, dtype=torch.float16, device="meta"), None, 0)
    assert out.shape == (3, 32)


def test_w4a16_linear_module_checks():
    with pytest.raises(ValueError):
        rf.W4A16Linear(100, 32)
    with pytest.raises(ValueError):
        rf.W4A16Linear(128, 40)
    with pytest.raises(ValueError):
        rf.W4A16Linear(192, 32, group_size=128)
    lin = torch.nn.Linear(256, 64, bias=True)
    m = rf.W4A16Linear.from_linear(lin, group_size=64)
    q, s, _ = rf.quantize_int4_group_wise(lin.weight.detach(), 64)
    assert torch.equal(m.rowmajor_weight(), q) and torch.equal(m.weight_scale, s)
    assert m.bias.dtype == torch.float16
    pc = rf.W4A16Linear.from_linear(lin, group_size=None)
    assert pc.weight_scale.shape == (64,) and pc.group_size is None
