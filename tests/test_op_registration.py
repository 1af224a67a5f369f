"""CPU tests of the torch-library registration of every schema.

torch.library.opcheck runs each op's schema check, autograd-registration
check, FakeTensor check and AOT-dispatch check (dynamic shapes).  The compute
ops have no CPU kernel, so they are checked on meta tensors (their Meta
kernels); the packers run on the CPU.  The GPU suite repeats the compute ops
on device tensors.  The ops are not differentiable: like the reference's W8A16
schemas (src/core/rpu_dispatch_registrations.inc:1043-1068) autograd falls
through to the backend kernel.
"""
from __future__ import annotations

import pytest
import torch
from torch.library import opcheck

import rhinoforge_amd as rf

M, N, K = 4, 96, 136


def _meta(shape, dtype, requires_grad=False):
    return torch.empty(shape, dtype=dtype, device="meta", requires_grad=requires_grad)


def _cases():
    x = _meta((2, M, K), torch.float16)
    w = _meta(rf.packed_shape(N, K), torch.int8)
    s = _meta((N,), torch.float16)
    b = _meta((N,), torch.float16)
    out = _meta((2, M, N), torch.float16)
    q = torch.randint(-128, 128, (40, 70), dtype=torch.int8)
    q4 = torch.randint(-8, 8, (48, 128), dtype=torch.int8)
    w8 = torch.ops.w8a16
    w4 = torch.ops.w4a16
    return {
        "w8a16::linear": (w8.linear.default, (x, w, s, b)),
        "w8a16::linear no bias": (w8.linear.default, (x, w, s)),
        "w8a16::linear_into": (w8.linear_into.default, (x, w, s, b, out)),
        "w8a16::linear_multi": (w8.linear_multi.default, (x, [w, w], [s, s], [b, None])),
        "w8a16::linear_argmax logits": (w8.linear_argmax.default, (x, w, s, None, True)),
        "w8a16::linear_argmax ids": (w8.linear_argmax.default, (x, w, s, b, False)),
        "w8a16::pack_weight": (w8.pack_weight.default, (q,)),
        "w8a16::unpack_weight": (w8.unpack_weight.default, (w8.pack_weight(q), 40, 70)),
        "w4a16::linear group-wise": (w4.linear.default,
                                     (_meta((3, 128), torch.float16), _meta(rf.packed_shape_int4(48, 128), torch.uint8),
                                      _meta((4, 48), torch.float16))),
        "w4a16::linear per-channel": (w4.linear.default,
                                      (_meta((3, 128), torch.float16), _meta(rf.packed_shape_int4(48, 128), torch.uint8),
                                       _meta((48,), torch.float16))),
        "w4a16::linear_multi group-wise": (
            w4.linear_multi.default,
            (_meta((3, 128), torch.float16),
             [_meta(rf.packed_shape_int4(48, 128), torch.uint8),
              _meta(rf.packed_shape_int4(32, 128), torch.uint8)],
             [_meta((4, 48), torch.float16), _meta((4, 32), torch.float16)],
             [_meta((48,), torch.float16), None])),
        "w4a16::linear_multi per-channel": (
            w4.linear_multi.default,
            (_meta((3, 128), torch.float16), [_meta(rf.packed_shape_int4(48, 128), torch.uint8)],
             [_meta((48,), torch.float16)], [None])),
        "w4a16::pack_weight": (w4.pack_weight.default, (q4,)),
        "w4a16::unpack_weight": (w4.unpack_weight.default, (w4.pack_weight(q4), 48, 128)),
    }


@pytest.mark.parametrize("name", sorted(_cases()))
def test_opcheck_every_schema(name):
    op, args = _cases()[name]
    report = opcheck(op, args, raise_exception=False)
    failed = {k: v for k, v in report.items() if v != "SUCCESS"}
    assert not failed, f"{name}: {failed}"


def test_every_schema_is_covered():
    registered = {o for o in torch._C._dispatch_get_all_op_names()
                  if o.startswith(("w8a16::", "w4a16::"))}
    covered = {n.split(" ")[0] for n in _cases()}
    # select_kernel takes and returns plain ints (no tensors to check)
    assert registered - covered == {"w8a16::select_kernel"}
    assert torch.ops.w8a16.select_kernel(1, 4096, 4096) in (rf.KERNEL_GEMV, rf.KERNEL_GEMM)


def test_meta_kernels_check_shapes_like_the_device_kernels():
    x = _meta((M, K), torch.float16)
    s = _meta((N,), torch.float16)
    with pytest.raises(RuntimeError, match="packed int8 tiles"):
        torch.ops.w8a16.linear(x, _meta((N, K), torch.int8), s)  # unpacked (row-major) shape
    w = _meta(rf.packed_shape(N, K), torch.int8)
    with pytest.raises(RuntimeError, match="input must be float16"):
        torch.ops.w8a16.linear(x.float(), w, s)
    with pytest.raises(RuntimeError, match="at most 64 rows"):
        torch.ops.w8a16.linear_argmax(_meta((65, K), torch.float16), w, s)
    with pytest.raises(RuntimeError, match="out shape"):
        torch.ops.w8a16.linear_into(x, w, s, None, _meta((M, N + 1), torch.float16))
    with pytest.raises(RuntimeError, match="32, 64 or 128"):
        torch.ops.w4a16.linear(_meta((3, 128), torch.float16), _meta(rf.packed_shape_int4(48, 128), torch.uint8),
                               _meta((8, 48), torch.float16))


def test_outputs_do_not_require_grad():
    """Autograd falls through: an input that requires grad is accepted and the
    (non-differentiable) outputs carry no graph."""
    x = _meta((M, K), torch.float16, requires_grad=True)
    w = _meta(rf.packed_shape(N, K), torch.int8)
    s = _meta((N,), torch.float16)
    y = torch.ops.w8a16.linear(x, w, s)
    assert y.shape == (M, N) and not y.requires_grad
    ys = torch.ops.w8a16.linear_multi(x, [w], [s], [None])
    assert not ys[0].requires_grad


def test_a_row_major_weight_is_refused_by_every_op():
    """A row-major int8 [N, K] passed where the packed tiles belong raises in
    every op, also where N % 16 == 0 and K % 64 == 0 (every Qwen3 projection),
    on meta tensors and on CPU tensors alike: the packed form is 3-D
    [ceil(N/16), ceil(K/64), 1024], a rank no row-major weight has."""
    w8, w4 = torch.ops.w8a16, torch.ops.w4a16
    for dev in ("meta", "cpu"):
        x = torch.zeros(2, 4096, dtype=torch.float16, device=dev)
        q = torch.zeros(4096, 4096, dtype=torch.int8, device=dev)      # row-major [N, K]
        s = torch.ones(4096, dtype=torch.float16, device=dev)
        flat = torch.zeros(4096 * 4096, dtype=torch.int8, device=dev)  # right bytes, wrong shape
        out = torch.empty(2, 4096, dtype=torch.float16, device=dev)
        calls = {
            "linear": lambda w: w8.linear(x, w, s),
            "linear_into": lambda w: w8.linear_into(x, w, s, None, out),
            "linear_multi": lambda w: w8.linear_multi(x, [w, w], [s, s], [None, None]),
            "linear_argmax": lambda w: w8.linear_argmax(x, w, s, None, False),
        }
        for name, call in calls.items():
            for w in (q, flat):
                with pytest.raises(RuntimeError, match="packed int8 tiles"):
                    call(w)
        # the packed shape itself passes the checks (meta: shape inference;
        # cpu: then refused only for having no CPU implementation)
        wp = torch.zeros(rf.packed_shape(4096, 4096), dtype=torch.int8, device=dev)
        if dev == "meta":
            assert w8.linear(x, wp, s).shape == (2, 4096)
        else:
            with pytest.raises(RuntimeError, match="no CPU implementation"):
                w8.linear(x, wp, s)
        # int4: the reference's nibble-packed uint8 [N, K/2] is refused too
        q4 = torch.zeros(4096, 2048, dtype=torch.uint8, device=dev)
        with pytest.raises(RuntimeError, match="packed int4 tiles"):
            w4.linear(x, q4, s)
        with pytest.raises(RuntimeError, match="packed int4 tiles"):
            w4.linear_multi(x, [q4, q4], [s, s], [None, None])
    with pytest.raises(RuntimeError, match="packed must have shape"):
        rf.unpack_weight(torch.zeros(4096, 4096, dtype=torch.int8), 4096, 4096)


def test_w4a16_linear_multi_refuses_mixed_scale_forms():
    x = _meta((3, 128), torch.float16)
    w48, w32 = (_meta(rf.packed_shape_int4(n, 128), torch.uint8) for n in (48, 32))
    with pytest.raises(RuntimeError, match="same scale form"):
        torch.ops.w4a16.linear_multi(x, [w48, w32], [_meta((4, 48), torch.float16),
                                                     _meta((32,), torch.float16)], [])
    with pytest.raises(RuntimeError, match="same scale form"):
        torch.ops.w4a16.linear_multi(x, [w48, w32], [_meta((4, 48), torch.float16),
                                                     _meta((1, 32), torch.float16)], [])
    with pytest.raises(RuntimeError, match="between 1 and 4"):
        torch.ops.w4a16.linear_multi(x, [w48] * 5, [_meta((48,), torch.float16)] * 5, [])
