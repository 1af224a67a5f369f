"""Python face of the ``torch.ops.w8a16`` op (see csrc/w8a16_torch.cpp).

Call conventions follow the reference's eager ``linear_into``
(src/core/rpu_dispatch_registrations.inc:19-20; src/ops/rpu_linear.cpp:664-731)
with the fp16 scale next to the int8 weight, as in ``causal_decoder_set_lm_head``
(registrations :46).  The ``layout`` argument is the analogue of the
reference's recorded ``partition`` (python/rpu_backend/runtime/weights.py:386-408)
and ``kernel`` the analogue of ``force_gemm`` (src/ops/rpu_linear.cpp:1094-1103).
"""
from __future__ import annotations

import torch

LAYOUT_ROWMAJOR = 0
LAYOUT_TILE16X64 = 1
KERNEL_AUTO = 0
KERNEL_GEMV = 1
KERNEL_GEMM = 2


def packed_shape(n: int, k: int) -> tuple[int, int, int]:
    """Shape of the packed int8 weight for a logical [n, k] weight: one
    1024-byte tile per 16 output channels and 64 input channels,
    ``[ceil(n/16), ceil(k/64), 1024]``.  A row-major ``[N, K]`` matrix never
    has this rank, so the ops refuse one passed in its place."""
    return ((n + 15) // 16, (k + 63) // 64, 1024)


def pack_weight(q: torch.Tensor) -> torch.Tensor:
    """Row-major int8 [N, K] -> TILE16X64 packed int8 ``packed_shape(N, K)``.

    Replaces the reference's load-time swizzle ``transform_linear_weight``
    (runtime/weights.py:206-233).  Runs on the device for HIP tensors and on
    the host for CPU tensors; the on-disk checkpoint stays row-major.
    """
    return torch.ops.w8a16.pack_weight(q)


def unpack_weight(packed: torch.Tensor, n: int, k: int) -> torch.Tensor:
    """Inverse of :func:`pack_weight`; returns a CPU int8 [n, k] tensor."""
    return torch.ops.w8a16.unpack_weight(packed, n, k)


def unpack_weight_on_device(packed: torch.Tensor, n: int, k: int) -> torch.Tensor:
    """:func:`unpack_weight` on the packed tensor's own device (a tile
    permutation in torch ops, no host copy): the row-major int8 [n, k].

    Byte j of lane l in tile (nb, kb) holds q[16 nb + l % 16][64 kb + 16 (l / 16) + j]
    XOR 0x80, so the tiles viewed as [nb, kb, l / 16, l % 16, j] and permuted to
    [nb, l % 16, kb, l / 16, j] are the padded row-major matrix."""
    shape = packed_shape(n, k)
    if packed.dtype != torch.int8 or tuple(packed.shape) != shape:
        raise ValueError(f"packed must be int8 {list(shape)} for n={n}, k={k}, got "
                         f"{packed.dtype} {list(packed.shape)}")
    nb, kb, _ = shape
    t = packed.view(torch.uint8).view(nb, kb, 4, 16, 16).permute(0, 3, 1, 2, 4)
    t = t.reshape(nb * 16, kb * 64)[:n, :k] ^ 0x80
    return t.contiguous().view(torch.int8)


def linear(input: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
           bias: torch.Tensor | None = None, *, layout: int = LAYOUT_TILE16X64,
           kernel: int = KERNEL_AUTO) -> torch.Tensor:
    """y = input . (weight_scale (.) q)^T (+ bias), fp16 out, fp32 accumulation.

    input [..., K] fp16; weight = pack_weight(q) for q int8 [N, K];
    weight_scale fp16 [N]; bias fp16 [N] or None.  HIP tensors only.
    """
    return torch.ops.w8a16.linear(input, weight, weight_scale, bias, layout, kernel)


def linear_into(input: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
                bias: torch.Tensor | None, out: torch.Tensor, *,
                layout: int = LAYOUT_TILE16X64, kernel: int = KERNEL_AUTO) -> None:
    """In-place variant writing into a caller-owned contiguous ``out`` [..., N]."""
    torch.ops.w8a16.linear_into(input, weight, weight_scale, bias, out, layout, kernel)


def linear_multi(input: torch.Tensor, weights, weight_scales, biases=None, *,
                 layout: int = LAYOUT_TILE16X64, kernel: int = KERNEL_AUTO) -> list:
    """Several projections of one input (q/k/v, gate/up) in one decode launch.

    Returns [input . (s_i (.) q_i)^T (+ b_i)] for each (weight_i, weight_scale_i,
    bias_i).  All projections run in one launch of either kernel (the
    analogue of the reference's fused QKV W8A16 kernel,
    src/ops/rpu_linear.cpp:1546-1674).
    """
    weights = list(weights)
    if biases is None:
        biases = [None] * len(weights)
    return torch.ops.w8a16.linear_multi(input, weights, list(weight_scales), list(biases),
                                        layout, kernel)


def linear_argmax(input: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
                  bias=None, *, return_logits: bool = False, layout: int = LAYOUT_TILE16X64):
    """Greedy-decode lm_head: the index of the largest fp16 logit per row.

    Computes ``input . (s (.) q)^T (+ b)`` rounded to fp16 like ``linear`` and
    returns its argmax over the last dimension as int32 (the lowest index
    among equal maxima; NaN counts as the largest value, as torch.argmax
    does), with the reduction folded into the decode GEMV's epilogue (at most
    64 rows).  ``return_logits=True`` also returns the logits; otherwise
    ``(index, empty tensor)``.  Replaces the reference's decode lm_head GEMM
    followed by rpu_argmax (src/fused/rpu_qwen3_model.h:3653-3690,
    src/ops/rpu_argmax.cpp:485-640).
    """
    index, logits = torch.ops.w8a16.linear_argmax(input, weight, weight_scale, bias,
                                                  return_logits, layout)
    return (index, logits) if return_logits else index


def select_kernel(m: int, n: int, k: int) -> int:
    """Kernel the AUTO policy runs for (M, N, K): KERNEL_GEMV or KERNEL_GEMM."""
    return int(torch.ops.w8a16.select_kernel(m, n, k))


# ---- W4A16 (packed int4 weights) ---------------------------------------------

LAYOUT_TILE16X128_I4 = 2


def packed_shape_int4(n: int, k: int) -> tuple[int, int, int]:
    """Shape of the packed uint8 int4 weight for a logical [n, k] weight: one
    1024-byte tile per 16 output channels and 128 input channels,
    ``[ceil(n/16), ceil(k/128), 1024]`` (never the rank of the reference's
    row-major nibble-packed ``[N, K/2]``)."""
    return ((n + 15) // 16, (k + 127) // 128, 1024)


def pack_weight_int4(q: torch.Tensor) -> torch.Tensor:
    """int4 values in int8 containers [N, K] (range [-8, 7]) -> TILE16X128_I4
    packed uint8 ``packed_shape_int4(N, K)``.

    Replaces the reference's nibble packers (quant/int4_pack.py:45-58,
    quant/int4_pgrp_pack.py:158-162) with one layout for both scale modes.
    Runs on the device for HIP tensors and on the host (range-checked) for
    CPU tensors.
    """
    return torch.ops.w4a16.pack_weight(q)


def unpack_weight_int4(packed: torch.Tensor, n: int, k: int) -> torch.Tensor:
    """Inverse of :func:`pack_weight_int4`; returns a CPU int8 [n, k] tensor."""
    return torch.ops.w4a16.unpack_weight(packed, n, k)


def unpack_weight_int4_on_device(packed: torch.Tensor, n: int, k: int) -> torch.Tensor:
    """:func:`unpack_weight_int4` on the packed tensor's own device, in torch ops.

    Lane l of tile (nb, kt) holds channel 16 nb + l % 16, positions
    128 kt + 32 (l / 16) + 8 w + i in dword w; inside a dword, position i sits
    in nibble i / 2 (i even) or 4 + i / 2 (i odd), as q + 8.  Little-endian
    bytes 0, 1 therefore carry positions 0, 2 | 4, 6 (low nibble first) and
    bytes 2, 3 positions 1, 3 | 5, 7."""
    shape = packed_shape_int4(n, k)
    if packed.dtype != torch.uint8 or tuple(packed.shape) != shape:
        raise ValueError(f"packed must be uint8 {list(shape)} for n={n}, k={k}, got "
                         f"{packed.dtype} {list(packed.shape)}")
    nb, kt, _ = shape
    b = packed.view(nb, kt, 4, 16, 4, 4)           # [nb, kt, l/16, l%16, dword, byte]
    nib = torch.stack((b & 0xF, b >> 4), dim=-1)    # [..., byte, lo/hi]
    even = nib[..., 0:2, :].reshape(nb, kt, 4, 16, 4, 4)   # positions 0, 2, 4, 6
    odd = nib[..., 2:4, :].reshape(nb, kt, 4, 16, 4, 4)    # positions 1, 3, 5, 7
    pos = torch.stack((even, odd), dim=-1).reshape(nb, kt, 4, 16, 32)
    q = pos.permute(0, 3, 1, 2, 4).reshape(nb * 16, kt * 128)[:n, :k]
    return (q.to(torch.int16) - 8).to(torch.int8).contiguous()


def linear_w4a16(input: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
                 bias: torch.Tensor | None = None, *, kernel: int = KERNEL_AUTO) -> torch.Tensor:
    """y = input . W^T (+ bias) with a packed int4 weight, fp16 out, fp32 accumulation.

    weight_scale fp16 [N] selects per-channel scaling (W = s[n] q[n,k], scale
    applied to the fp32 sum); [K/group_size, N] selects group-wise scaling
    (W = RN_fp16(s[k/gs, n] q[n,k]), group_size 32, 64 or 128), the dispatch
    of the reference's launcher (src/ops/rpu_linear.cpp:1211-1489).  Needs
    N % 16 == 0 and K % 64 == 0.  HIP tensors only.
    """
    return torch.ops.w4a16.linear(input, weight, weight_scale, bias, kernel)


def linear_multi_w4a16(input: torch.Tensor, weights, weight_scales, biases=None, *,
                       kernel: int = KERNEL_AUTO) -> list:
    """Several packed-int4 projections of one input (q/k/v, gate/up) in one
    launch of either kernel, as :func:`linear_multi` does for int8.  Every
    scale has the same form: per-channel [N_i], or group-wise [K/gs, N_i]
    with one group size.  Returns [input . W_i^T (+ b_i)]."""
    weights = list(weights)
    if biases is None:
        biases = [None] * len(weights)
    return torch.ops.w4a16.linear_multi(input, weights, list(weight_scales), list(biases), kernel)
