"""CPU tests: the packed-weight modules keep the checkpoint form in their state dict.

A W8A16Linear's ``weight`` buffer holds TILE16X64 tiles, shaped
[ceil(N/16), ceil(K/64), 1024]; the checkpoint tensor is the row-major int8
[N, K] (quant/convert_qwen3.py:65-100).  The module's state dict always
carries the row-major weight (unpacked on save, packed on load), so round
trips and checkpoint loads cannot mix the layouts.  Earlier builds of the
module (state-dict version 1) stored either form as a 2-D tensor; such a
dict loads where its shape tells the form and is refused where it cannot.
"""
from __future__ import annotations

import pytest
import torch

import rhinoforge_amd as rf


@pytest.mark.parametrize("n,k", [(64, 128), (40, 72)])
def test_w8a16_state_dict_round_trip_is_row_major(n, k):
    g = torch.Generator().manual_seed(n + k)
    q = torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8)
    s = (torch.rand(n, generator=g) * 0.01 + 1e-3).half()
    b = torch.randn(n, generator=g).half()
    mod = rf.W8A16Linear.from_quantized(q, s, b)  # packed on the host
    sd = mod.state_dict()
    assert sd["weight"].dtype == torch.int8 and tuple(sd["weight"].shape) == (n, k)
    assert torch.equal(sd["weight"], q)            # the checkpoint form, not the packed bytes
    assert torch.equal(sd["weight_scale"], s) and torch.equal(sd["bias"], b)
    fresh = rf.W8A16Linear(k, n, bias=True)
    fresh.load_state_dict(sd)
    assert torch.equal(fresh.weight, mod.weight)   # packed again on load
    assert torch.equal(fresh.weight, rf.pack_weight(q))
    assert torch.equal(sd["weight"], q)            # the caller's dict is left as it was


def test_w8a16_loads_a_converted_checkpoint_pair():
    """The raw row-major pair of a converted checkpoint (what HF from_pretrained
    or a plain load_state_dict hands over) is packed, never copied verbatim."""
    n, k = 128, 256  # packed and row-major shapes coincide
    q = torch.randint(-128, 128, (n, k), dtype=torch.int8)
    mod = rf.W8A16Linear(k, n)
    mod.load_state_dict({"weight": q, "weight_scale": torch.ones(n, dtype=torch.float16)})
    assert not torch.equal(mod.weight, q)
    assert torch.equal(mod.rowmajor_weight(), q)


def test_w8a16_refuses_a_weight_of_the_wrong_form():
    mod = rf.W8A16Linear(72, 40)
    packed = rf.pack_weight(torch.zeros(40, 72, dtype=torch.int8))  # [3, 2, 1024]: packed tiles
    with pytest.raises(RuntimeError, match="logical int8"):
        mod.load_state_dict({"weight": packed, "weight_scale": torch.ones(40, dtype=torch.float16)})
    with pytest.raises(RuntimeError, match="logical int8"):
        mod.load_state_dict({"weight": torch.zeros(40, 72, dtype=torch.float16),
                             "weight_scale": torch.ones(40, dtype=torch.float16)})


@pytest.mark.parametrize("group_size", [None, 32])
def test_w4a16_state_dict_round_trip(group_size):
    n, k = 48, 128
    q = torch.randint(-8, 8, (n, k), dtype=torch.int8)
    s = torch.rand((k // group_size, n) if group_size else (n,)).half() + 0.01
    mod = rf.W4A16Linear.from_quantized(q, s)
    sd = mod.state_dict()
    assert sd["weight"].dtype == torch.int8 and torch.equal(sd["weight"], q)
    fresh = rf.W4A16Linear(k, n, group_size=group_size)
    fresh.load_state_dict(sd)
    assert torch.equal(fresh.weight, mod.weight)
    bad = dict(sd)
    bad["weight"] = q.clone()
    bad["weight"][0, 0] = 9
    with pytest.raises(RuntimeError, match="outside"):
        fresh.load_state_dict(bad)


def _v1_dict(weight, n):
    """A state dict as an earlier (version-1) build of the module saved it."""
    from collections import OrderedDict
    sd = OrderedDict(weight=weight, weight_scale=torch.ones(n, dtype=torch.float16))
    sd._metadata = OrderedDict({"": {"version": 1}})
    return sd


def test_state_dict_records_version_2():
    mod = rf.W8A16Linear(128, 64)
    assert rf.W8A16Linear._version == 2 and rf.W4A16Linear._version == 2
    assert mod.state_dict()._metadata[""]["version"] == 2


def test_w8a16_version1_dicts_load_where_the_shape_tells_the_form():
    n, k = 40, 72                               # packed 2-D [48, 128] != logical [40, 72]
    q = torch.randint(-128, 128, (n, k), dtype=torch.int8)
    want = rf.pack_weight(q)
    mod = rf.W8A16Linear(k, n)
    mod.load_state_dict(_v1_dict(q, n))         # row-major form: packed on load
    assert torch.equal(mod.weight, want)
    mod = rf.W8A16Linear(k, n)
    mod.load_state_dict(_v1_dict(want.reshape(48, 128), n))  # 2-D packed bytes: installed
    assert torch.equal(mod.weight, want) and torch.equal(mod.rowmajor_weight(), q)


def test_w8a16_version1_dict_of_ambiguous_shape_is_refused():
    """N=128, K=256: the earlier build's packed bytes and the row-major weight
    are both int8 [128, 256]; loading either guess could be silently wrong."""
    n, k = 128, 256
    q = torch.randint(-128, 128, (n, k), dtype=torch.int8)
    mod = rf.W8A16Linear(k, n)
    before = mod.weight.clone()
    with pytest.raises(RuntimeError, match="version-1 state dict"):
        mod.load_state_dict(_v1_dict(q, n))
    assert torch.equal(mod.weight, before)
    # the same tensor without version metadata is the checkpoint form
    mod.load_state_dict({"weight": q, "weight_scale": torch.ones(n, dtype=torch.float16)})
    assert torch.equal(mod.rowmajor_weight(), q)


def test_w4a16_version1_packed_bytes_load():
    n, k = 48, 128
    q = torch.randint(-8, 8, (n, k), dtype=torch.int8)
    want = rf.pack_weight_int4(q)
    mod = rf.W4A16Linear(k, n, group_size=None)
    mod.load_state_dict(_v1_dict(want.reshape(n, k // 2), n))  # uint8 [48, 64]
    assert torch.equal(mod.weight, want)
    mod = rf.W4A16Linear(k, n, group_size=None)
    mod.load_state_dict(_v1_dict(q, n))                          # int8 [48, 128]
    assert torch.equal(mod.weight, want)


@pytest.mark.parametrize("n,k", [(48, 128), (40, 256), (16, 384)])
def test_w4a16_device_unpack_matches_host_unpack(n, k):
    q = torch.randint(-8, 8, (n, k), dtype=torch.int8)
    p = rf.pack_weight_int4(q)
    assert torch.equal(rf.ops.unpack_weight_int4_on_device(p, n, k), q)
    assert torch.equal(rf.unpack_weight_int4(p, n, k), q)
