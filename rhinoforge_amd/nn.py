"""``W8A16Linear``: an nn.Module holding a packed int8 weight and fp16 scale.

The reference keeps ``nn.Linear`` modules with an int8 ``weight`` Parameter and
an fp16 ``weight_scale`` buffer (python/rpu_backend/quant/load.py:267-284),
swizzles the weight in place at load time and records the layout on the
module (runtime/weights.py:386-408, 411-544).  Here the packed weight lives in
a ``weight`` buffer of shape ``packed_shape(N, K)`` and the layout tag in
``self.layout``; forward calls ``torch.ops.w8a16.linear``.

The packed bytes never leave the module under the checkpoint's name: its
state dict holds ``weight`` as the row-major int8 ``[N, K]`` checkpoint form
(quant/convert_qwen3.py:65-100), unpacked on save and packed on load, so a
``state_dict()`` / ``load_state_dict()`` round trip or an HF
``save_pretrained`` never mixes the two layouts (the hazard the reference
guards with its recorded layout, runtime/weights.py:28-49).  The packed
buffer itself is 3-D (``[ceil(N/16), ceil(K/64), 1024]`` tiles), a shape no
row-major weight has.  ``state_dict()`` unpacks on the weight's own device
(a tile permutation in torch ops): it costs one extra copy of the int8
weight in device memory while the dict is alive, and no host round trip.

State-dict versions (``_version``, recorded by torch in the dict's
metadata): 2 is the logical [N, K] form above.  A version-1 dict was written
by an earlier build of these modules, which stored either the logical form
or the packed bytes as a 2-D [ceil16(N), ceil64(K)] tensor; where the shape
tells which, it loads, and where both forms have the same shape (N % 16 == 0
and K % 64 == 0 for int8) it is refused rather than guessed.  A dict with no
version metadata (a checkpoint read from disk) holds the logical form.
"""
from __future__ import annotations

import torch
from torch import nn

from . import ops
from .quant import quantize_linear_per_channel


class _LogicalWeightStateDict:
    """State-dict hooks of the packed-weight modules: ``weight`` is saved as
    the logical int8 [N, K] tensor and packed again on load.  Subclasses give
    ``_unpack_here()`` (on the weight's device), ``_pack(q)``, the valid
    value range and ``_v1_packed_shape`` (the 2-D shape of the packed bytes
    version-1 dicts may hold, in the packed buffer's dtype)."""

    _version = 2
    _qmin, _qmax = -128, 127

    def _save_to_state_dict(self, destination, prefix, keep_vars):
        super()._save_to_state_dict(destination, prefix, keep_vars)
        if self.weight.is_meta:
            destination[prefix + "weight"] = torch.empty(
                (self.out_features, self.in_features), dtype=torch.int8, device="meta")
        else:
            destination[prefix + "weight"] = self._unpack_here()

    def _v1_weight(self, t, key, error_msgs):
        """The packed buffer for a version-1 dict's ``weight`` (logical or
        2-D packed bytes, told apart by shape), or None after an error."""
        shape = tuple(t.shape)
        logical = t.dtype == torch.int8 and shape == (self.out_features, self.in_features)
        packed = t.dtype == self.weight.dtype and shape == self._v1_packed_shape()
        if logical and packed:
            error_msgs.append(
                f"{key}: a version-1 state dict (an earlier build of {type(self).__name__}) "
                f"whose {list(shape)} weight may hold either the row-major checkpoint form or "
                f"packed bytes; re-export it from that build with rowmajor_weight(), or load "
                f"the row-major weight without the dict's version metadata")
            return None
        if packed:
            return t.to(self.weight.device).reshape(self.weight.shape).contiguous()
        return t  # the logical form (its checks follow)

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        key = prefix + "weight"
        logical = state_dict.get(key)
        if logical is not None:
            want = (self.out_features, self.in_features)
            version = local_metadata.get("version") if local_metadata else None
            if version is not None and version < 2 and isinstance(logical, torch.Tensor):
                got = self._v1_weight(logical, key, error_msgs)
                if got is None:
                    return
                if got is not logical:  # packed bytes: installed as they are
                    state_dict[key] = got
                    try:
                        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict,
                                                      missing_keys, unexpected_keys, error_msgs)
                    finally:
                        state_dict[key] = logical
                    return
            if logical.dtype != torch.int8 or tuple(logical.shape) != want:
                error_msgs.append(
                    f"{key}: expected the logical int8 {list(want)} weight (the checkpoint "
                    f"form; the module packs it), got {logical.dtype} {list(logical.shape)}")
                return
            if not logical.is_meta and (int(logical.min()) < self._qmin
                                        or int(logical.max()) > self._qmax):
                error_msgs.append(f"{key}: values outside [{self._qmin}, {self._qmax}]")
                return
            state_dict[key] = self._pack(logical.to(self.weight.device))
        try:
            super()._load_from_state_dict(state_dict, prefix, local_metadata, strict,
                                          missing_keys, unexpected_keys, error_msgs)
        finally:
            if logical is not None:
                state_dict[key] = logical


class W8A16Linear(_LogicalWeightStateDict, nn.Module):
    def __init__(self, in_features: int, out_features: int, bias: bool = False,
                 device=None) -> None:
        super().__init__()
        if in_features < 8 or in_features % 8:
            raise ValueError(f"in_features={in_features}: the kernels need K > 0 and K % 8 == 0")
        if out_features < 1:
            raise ValueError(f"out_features={out_features} must be >= 1")
        self.in_features = in_features
        self.out_features = out_features
        self.layout = ops.LAYOUT_TILE16X64
        self.register_buffer("weight", torch.full(ops.packed_shape(out_features, in_features),
                                                  -128, dtype=torch.int8, device=device))
        self.register_buffer("weight_scale", torch.ones(out_features, dtype=torch.float16,
                                                        device=device))
        if bias:
            self.register_buffer("bias", torch.zeros(out_features, dtype=torch.float16,
                                                     device=device))
        else:
            self.bias = None

    @classmethod
    def from_quantized(cls, q: torch.Tensor, weight_scale: torch.Tensor,
                       bias: torch.Tensor | None = None, *, device=None) -> "W8A16Linear":
        """From an on-disk pair: ``X.weight`` int8 [N, K] row-major and
        ``X.weight_scale`` fp16 [N] (quant/convert_qwen3.py:65-100 format).

        The weight is packed where it ends up: on ``device`` (default: q's
        device) by the pack kernel for a HIP device, on the host for the CPU.
        """
        if q.dtype != torch.int8 or q.dim() != 2:
            raise TypeError(f"weight must be int8 [N, K], got {q.dtype} {tuple(q.shape)}")
        n, k = q.shape
        if weight_scale.dtype != torch.float16 or tuple(weight_scale.shape) != (n,):
            raise TypeError(f"weight_scale must be fp16 [{n}], got {weight_scale.dtype} "
                            f"{tuple(weight_scale.shape)}")
        if bias is not None and tuple(bias.shape) != (n,):
            raise ValueError(f"bias must have shape ({n},), got {tuple(bias.shape)}")
        device = torch.device(device) if device is not None else q.device
        mod = cls(k, n, bias=bias is not None, device="meta")
        mod.weight = ops.pack_weight(q.to(device))
        mod.weight_scale = weight_scale.to(device).contiguous()
        if bias is not None:
            mod.bias = bias.to(device=device, dtype=torch.float16).contiguous()
        return mod

    @classmethod
    def from_linear(cls, linear: nn.Linear) -> "W8A16Linear":
        """Quantize a floating nn.Linear per channel, then pack."""
        q, s = quantize_linear_per_channel(linear.weight.detach())
        b = linear.bias.detach().to(torch.float16) if linear.bias is not None else None
        return cls.from_quantized(q, s, b)

    def rowmajor_weight(self) -> torch.Tensor:
        """The int8 [N, K] row-major weight (CPU), e.g. for checkpoint export."""
        return ops.unpack_weight(self.weight, self.out_features, self.in_features)

    def _unpack_here(self) -> torch.Tensor:
        return ops.unpack_weight_on_device(self.weight, self.out_features, self.in_features)

    def _v1_packed_shape(self) -> tuple[int, int]:
        return ((self.out_features + 15) // 16 * 16, (self.in_features + 63) // 64 * 64)

    def _pack(self, q: torch.Tensor) -> torch.Tensor:
        return ops.pack_weight(q)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return ops.linear(x, self.weight, self.weight_scale, self.bias, layout=self.layout)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, layout=TILE16X64")


class W4A16Linear(_LogicalWeightStateDict, nn.Module):
    """Linear layer with packed int4 weights and fp16 scales (W4A16).

    The reference replaces an fp16 ``nn.Linear``'s weight by a packed uint8
    ``[N, K/2]`` Parameter and registers the scale as a ``weight_scale``
    buffer: ``[N]`` per-channel, or the group-wise payload
    (quant/convert_qwen3_w4a16.py:79-121).  Here ``weight`` is the
    TILE16X128_I4 buffer, ``weight_scale`` is ``[N]`` or the logical
    ``[K/group_size, N]``, and forward calls ``torch.ops.w4a16.linear``.
    The state dict holds ``weight`` as the int4 values in an int8 [N, K]
    tensor (the reference writes no int4 checkpoint: its conversion is
    in-memory), packed again on load.
    """

    _qmin, _qmax = -8, 7

    def __init__(self, in_features: int, out_features: int, group_size: int | None = 32,
                 bias: bool = False, device=None) -> None:
        super().__init__()
        if in_features < 64 or in_features % 64:
            raise ValueError(f"in_features={in_features}: int4 tiles need K > 0 and K % 64 == 0")
        if out_features < 16 or out_features % 16:
            raise ValueError(f"out_features={out_features}: int4 tiles need N > 0 and N % 16 == 0")
        if group_size not in (None, 32, 64, 128) or (group_size and in_features % group_size):
            raise ValueError(f"group_size={group_size} must be None (per-channel) or 32/64/128 "
                             f"dividing in_features={in_features}")
        self.in_features = in_features
        self.out_features = out_features
        self.group_size = group_size
        self.layout = ops.LAYOUT_TILE16X128_I4
        self.register_buffer("weight", torch.full(ops.packed_shape_int4(out_features, in_features),
                                                  0x88, dtype=torch.uint8, device=device))
        sshape = (in_features // group_size, out_features) if group_size else (out_features,)
        self.register_buffer("weight_scale", torch.ones(sshape, dtype=torch.float16, device=device))
        if bias:
            self.register_buffer("bias", torch.zeros(out_features, dtype=torch.float16,
                                                     device=device))
        else:
            self.bias = None

    @classmethod
    def from_quantized(cls, q: torch.Tensor, weight_scale: torch.Tensor,
                       bias: torch.Tensor | None = None, *, device=None) -> "W4A16Linear":
        """From int4 values in int8 containers [N, K] and a scale [N] or
        [K/group_size, N] (quant/int4_pack.py:21-23, int4_pgrp_pack.py:33-60)."""
        if q.dtype != torch.int8 or q.dim() != 2:
            raise TypeError(f"q must be int8 [N, K] int4 values, got {q.dtype} {tuple(q.shape)}")
        n, k = q.shape
        if weight_scale.dtype != torch.float16 or weight_scale.dim() not in (1, 2):
            raise TypeError(f"weight_scale must be fp16 [N] or [G, N], got {weight_scale.dtype} "
                            f"{tuple(weight_scale.shape)}")
        if weight_scale.dim() == 1:
            group_size = None
            if tuple(weight_scale.shape) != (n,):
                raise ValueError(f"per-channel scale must be [{n}], got {tuple(weight_scale.shape)}")
        else:
            g = weight_scale.shape[0]
            if weight_scale.shape[1] != n or g < 1 or k % g:
                raise ValueError(f"group-wise scale must be [K/group_size, {n}], got "
                                 f"{tuple(weight_scale.shape)}")
            group_size = k // g
        device = torch.device(device) if device is not None else q.device
        mod = cls(k, n, group_size=group_size, bias=bias is not None, device="meta")
        mod.weight = ops.pack_weight_int4(q.to(device))
        mod.weight_scale = weight_scale.to(device).contiguous()
        if bias is not None:
            mod.bias = bias.to(device=device, dtype=torch.float16).contiguous()
        return mod

    @classmethod
    def from_linear(cls, linear: nn.Linear, group_size: int | None = 32) -> "W4A16Linear":
        """Quantize a floating nn.Linear (group-wise by default, as the
        reference's W4A16 converter, convert_qwen3_w4a16.py:40-42), then pack."""
        from .quant.int4 import quantize_int4_group_wise, quantize_int4_per_channel
        w = linear.weight.detach()
        if group_size:
            q, s, _ = quantize_int4_group_wise(w, group_size)
        else:
            q, s = quantize_int4_per_channel(w)
        b = linear.bias.detach().to(torch.float16) if linear.bias is not None else None
        return cls.from_quantized(q, s, b)

    def rowmajor_weight(self) -> torch.Tensor:
        """The int4 values as an int8 [N, K] tensor (CPU)."""
        return ops.unpack_weight_int4(self.weight, self.out_features, self.in_features)

    def _unpack_here(self) -> torch.Tensor:
        return ops.unpack_weight_int4_on_device(self.weight, self.out_features,
                                                self.in_features)

    def _v1_packed_shape(self) -> tuple[int, int]:
        return (self.out_features, (self.in_features + 127) // 128 * 64)

    def _pack(self, q: torch.Tensor) -> torch.Tensor:
        return ops.pack_weight_int4(q)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return ops.linear_w4a16(x, self.weight, self.weight_scale, self.bias)

    def extra_repr(self) -> str:
        mode = f"group_size={self.group_size}" if self.group_size else "per-channel"
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, {mode}, layout=TILE16X128_I4")


class W8A16Embedding(nn.Module):
    """Token embedding with an int8 row-major table and one fp16 scale per row.

    The checkpoint form of ``quantized_embed_tokens`` (quant/load.py:303-316,
    343-356): ``weight`` int8 [V, H], ``weight_scale`` fp16 [V].  A lookup
    gathers rows and dequantizes them as ``fp16(f32(q) * f32(s))``
    (adapters/qwen3.py:654-680); the table is gathered, never multiplied, so
    it stays row-major.
    """

    def __init__(self, weight: torch.Tensor, weight_scale: torch.Tensor,
                 padding_idx: int | None = None) -> None:
        super().__init__()
        if weight.dtype != torch.int8 or weight.dim() != 2:
            raise TypeError(f"weight must be int8 [V, H], got {weight.dtype} "
                            f"{tuple(weight.shape)}")
        if weight_scale.dtype != torch.float16 or tuple(weight_scale.shape) != (weight.size(0),):
            raise TypeError(f"weight_scale must be fp16 [{weight.size(0)}], got "
                            f"{weight_scale.dtype} {tuple(weight_scale.shape)}")
        self.num_embeddings, self.embedding_dim = weight.shape
        self.padding_idx = padding_idx
        self.register_buffer("weight", weight.contiguous())
        self.register_buffer("weight_scale", weight_scale.contiguous())

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        rows = self.weight[input_ids].to(torch.float32)
        return (rows * self.weight_scale[input_ids].to(torch.float32).unsqueeze(-1)
                ).to(torch.float16)

    def extra_repr(self) -> str:
        return f"{self.num_embeddings}, {self.embedding_dim}, int8 rows"
