"""Pi0.5 and Wall-OSS W8A16 checkpoints (``rpu_quant_config.json``) on the CPU:
conversion, the record's checks, and swap-in of ``W8A16Linear`` /
``W4A16Linear`` / ``W8A16Embedding`` into a meta skeleton.

What is pinned here: every swapped module holds exactly the checkpoint's int8
rows and fp16 scales (packing round-trips through ``rowmajor_weight``), every
other tensor equals the source, and each refusal the reference's Pi0.5 loader
makes (adapters/pi05/loader.py:45-143: record fields, partial decoders, scales
without weights, misshaped scales) raises before a tensor is read.  Forward
numerics run in the GPU suite (test_gpu_rpu_loader.py).
"""
from __future__ import annotations

import json
import shutil
from pathlib import Path

import pytest
import torch
from safetensors.torch import load_file, save_file

transformers = pytest.importorskip("transformers")

import rhinoforge_amd as rf  # noqa: E402
from rhinoforge_amd.quant import convert, load  # noqa: E402
from ckpt_util import Pi05Tree, WallTree, read_all, write_pi05_source, write_wall_source  # noqa: E402

QUIET = dict(log=lambda *a: None)


@pytest.fixture(scope="module")
def pi05(tmp_path_factory):
    root = tmp_path_factory.mktemp("pi05")
    write_pi05_source(root / "src", seed=1)
    convert.convert_pi05_checkpoint(root / "src", root / "w8", **QUIET)
    convert.convert_pi05_checkpoint(root / "src", root / "w4fake", bits=4, **QUIET)
    convert.convert_pi05_checkpoint(root / "src", root / "w4real", bits=4, real_w4=True, **QUIET)
    return root


@pytest.fixture(scope="module")
def wall(tmp_path_factory):
    root = tmp_path_factory.mktemp("wall")
    write_wall_source(root / "src", seed=2)
    convert.convert_wall_oss_checkpoint(root / "src", root / "w8", **QUIET)
    return root


def _skeleton(cls=Pi05Tree, **kw):
    with torch.device("meta"):
        return cls(**kw)


def _copy(src: Path, dst: Path) -> Path:
    shutil.copytree(src, dst)
    return dst


def _edit_tensors(ckpt: Path, fn) -> None:
    path = ckpt / "model.safetensors"
    t = load_file(str(path))
    fn(t)
    save_file(t, str(path))


def _edit_record(ckpt: Path, fn) -> None:
    path = ckpt / "rpu_quant_config.json"
    rec = json.loads(path.read_text())
    fn(rec)
    path.write_text(json.dumps(rec))


# ---------------------------------------------------------------- conversion

def test_pi05_conversion_quantizes_both_decoders_only(pi05):
    src, ck = read_all(pi05 / "src"), read_all(pi05 / "w8")
    n = 0
    for name, t in src.items():
        if convert.pi05_decoder_of(name):
            q, s = rf.quantize_linear_per_channel(t)
            assert torch.equal(ck[name], q) and torch.equal(ck[convert.scale_name(name)], s)
            n += 1
        else:
            assert torch.equal(ck[name], t.to(torch.float16)), name
    assert n == 2 * 2 * 7
    rec = load.read_rpu_quant_config(pi05 / "w8")
    assert (rec["method"], rec["value_bits"], rec["target"]) == \
        ("w8a16", 8, "pi05_gemma_vlm_and_expert")


def test_pi05_four_bit_records_and_ranges(pi05):
    fake = read_all(pi05 / "w4fake")
    real = read_all(pi05 / "w4real")
    rf_fake = load.read_rpu_quant_config(pi05 / "w4fake")
    rf_real = load.read_rpu_quant_config(pi05 / "w4real")
    assert (rf_fake["method"], rf_fake["kernel"]) == ("w4a16_fake_int8", "w8a16")
    assert (rf_real["method"], rf_real["kernel"]) == ("w4a16", "wint4a16")
    assert set(rf_real["mixed_int8_suffixes"]) == {"k_proj.weight", "v_proj.weight"}
    for name, t in fake.items():
        if t.dtype == torch.int8:
            assert t.abs().max() <= 7, name
    for name, t in real.items():
        if t.dtype == torch.int8:
            bound = 127 if name.endswith(("k_proj.weight", "v_proj.weight")) else 7
            assert t.abs().max() <= bound, name


def test_wall_oss_conversion_lists_every_quantized_weight(wall):
    rec = load.read_rpu_quant_config(wall / "w8")
    ck = read_all(wall / "w8")
    int8 = sorted(n for n, t in ck.items() if t.dtype == torch.int8)
    assert rec["quantized_weights"] == int8 and rec["quantized_weight_count"] == len(int8)
    assert "embed_tokens.weight" not in int8 and "head.weight" in int8
    assert len(int8) == 2 * 4 + 1


# ---------------------------------------------------------------- loading

@pytest.mark.parametrize("variant,w4", [("w8", False), ("w4fake", False), ("w4real", True)])
def test_pi05_load_swaps_every_decoder_projection(pi05, variant, w4):
    ck = read_all(pi05 / variant)
    model = _skeleton()
    swapped = load.load_rpu_quant_checkpoint(model, pi05 / variant, device="cpu")
    assert len(swapped) == 28
    for name in swapped:
        mod = model.get_submodule(name)
        kv = name.endswith(("k_proj", "v_proj"))
        want = rf.W4A16Linear if (w4 and not kv) else rf.W8A16Linear
        assert type(mod) is want, name
        assert torch.equal(mod.rowmajor_weight(), ck[name + ".weight"]), name
        assert torch.equal(mod.weight_scale, ck[name + ".weight_scale"]), name
    for name, p in model.named_parameters():
        assert not p.is_meta and p.dtype == torch.float16
        assert torch.equal(p, ck[name]), name
    vlm = model.vlm()
    assert vlm.embed_tokens.embed_scale.item() == pytest.approx(128 ** 0.5)
    assert not vlm.rotary_emb.inv_freq.is_meta
    assert not any(b.is_meta for b in model.buffers())


def test_pi05_load_into_a_materialized_model(pi05):
    """A policy built on the CPU (not meta) is filled the same way; buffers the
    checkpoint lacks stay as the model computed them."""
    torch.manual_seed(5)
    model = Pi05Tree()
    inv = model.expert().rotary_emb.inv_freq.clone()
    assert len(load.load_rpu_quant_checkpoint(model, pi05 / "w8", device="cpu")) == 28
    assert torch.equal(model.expert().rotary_emb.inv_freq, inv)


def test_pi05_scale_lists_and_kv_replication_after_load(pi05):
    model = _skeleton()
    load.load_rpu_quant_checkpoint(model, pi05 / "w8", device="cpu")
    exp = model.expert()
    assert load.detect_and_validate_decoder_w8a16(exp, label="expert")
    lists = load.decoder_scale_lists(exp, label="expert")
    assert len(lists) == 7 and all(len(l) == 2 for l in lists)
    k0 = exp.layers[0].self_attn.k_proj.rowmajor_weight()
    assert load.replicate_kv_heads(exp, 4, label="expert") == 4
    k1 = exp.layers[0].self_attn.k_proj
    assert k1.out_features == 4 * 32
    assert torch.equal(k1.rowmajor_weight(), k0.repeat(4, 1))  # one KV head: 4 copies


def test_pi05_floating_decoder_stays_linear(pi05, tmp_path):
    """A checkpoint with one decoder quantized and the other floating (the
    all-or-none rule is per decoder): the floating one loads as nn.Linear."""
    ck = _copy(pi05 / "w8", tmp_path / "ck")
    src = read_all(pi05 / "src")

    def floatify(t):
        for name in list(t):
            if convert.pi05_decoder_of(name) == "expert":
                t[name] = src[name].to(torch.float16)
                del t[convert.scale_name(name)]
    _edit_tensors(ck, floatify)
    model = _skeleton()
    swapped = load.load_rpu_quant_checkpoint(model, ck, device="cpu")
    assert len(swapped) == 14 and all("paligemma." in n for n in swapped)
    assert type(model.expert().layers[0].mlp.up_proj) is torch.nn.Linear
    assert not load.detect_and_validate_decoder_w8a16(model.expert())


def test_wall_oss_load(wall):
    ck = read_all(wall / "w8")
    model = _skeleton(WallTree)
    swapped = load.load_rpu_quant_checkpoint(model, wall / "w8", device="cpu")
    assert len(swapped) == 9
    qkv = model.layers[0].self_attn.qkv_proj
    assert isinstance(qkv, rf.W8A16Linear) and qkv.bias is not None
    assert torch.equal(qkv.bias, ck["layers.0.self_attn.qkv_proj.bias"])
    assert type(model.embed_tokens) is torch.nn.Embedding
    assert torch.equal(model.layers[1].norm.weight, ck["layers.1.norm.weight"])


def test_wall_oss_quantized_embedding(tmp_path):
    write_wall_source(tmp_path / "src", seed=4)
    convert.convert_wall_oss_checkpoint(tmp_path / "src", tmp_path / "w8", skip_modules=(),
                                        **QUIET)
    model = _skeleton(WallTree)
    swapped = load.load_rpu_quant_checkpoint(model, tmp_path / "w8", device="cpu")
    assert "embed_tokens" in swapped and isinstance(model.embed_tokens, rf.W8A16Embedding)
    ck = read_all(tmp_path / "w8")
    ids = torch.tensor([[0, 7, 255]])
    want = (ck["embed_tokens.weight"].float() * ck["embed_tokens.weight_scale"].float()[:, None])
    assert torch.equal(model.embed_tokens(ids)[0], want[ids[0]].to(torch.float16))


def test_wall_oss_refuses_k_not_multiple_of_8(tmp_path):
    write_wall_source(tmp_path / "src", odd_k=True)
    convert.convert_wall_oss_checkpoint(tmp_path / "src", tmp_path / "w8", **QUIET)
    with pytest.raises(ValueError, match="multiple of 8"):
        load.load_rpu_quant_checkpoint(_skeleton(WallTree, odd_k=True), tmp_path / "w8",
                                       device="cpu")


# ---------------------------------------------------------------- refusals

def _drop_one_expert_int8(t):
    name = "model.paligemma_with_expert.gemma_expert.model.layers.1.mlp.down_proj.weight"
    t[name] = t[name].float().to(torch.float16)
    del t[convert.scale_name(name)]


def _scale_fp32(t):
    name = "model.paligemma_with_expert.paligemma.model.language_model.layers.0.self_attn.q_proj"
    t[name + ".weight_scale"] = t[name + ".weight_scale"].float()


def _orphan_scale(t):
    t["model.action_in_proj.weight_scale"] = torch.ones(64, dtype=torch.float16)


def _int8_extra(t):
    t["model.action_out_proj.weight"] = torch.zeros(32, 64, dtype=torch.int8)


def _extra_tensor(t):
    t["model.not_a_module.weight"] = torch.zeros(4, dtype=torch.float16)


def _missing_tensor(t):
    del t["model.action_out_proj.bias"]


def _bad_shape(t):
    t["model.action_in_proj.bias"] = torch.zeros(63, dtype=torch.float16)


@pytest.mark.parametrize("edit,exc,match", [
    (_drop_one_expert_int8, ValueError, "partly quantized"),
    (_scale_fp32, TypeError, "fp16"),
    (_orphan_scale, KeyError, "no int8 weight"),
    (_int8_extra, KeyError, "does not list"),
    (_extra_tensor, KeyError, "no parameter or buffer"),
    (_missing_tensor, KeyError, "absent from the checkpoint"),
    (_bad_shape, ValueError, "checkpoint shape"),
])
def test_pi05_refusals(pi05, tmp_path, edit, exc, match):
    ck = _copy(pi05 / "w8", tmp_path / "ck")
    _edit_tensors(ck, edit)
    with pytest.raises(exc, match=match):
        load.load_rpu_quant_checkpoint(_skeleton(), ck, device="cpu")


@pytest.mark.parametrize("field,value,match", [
    ("method", "nvfp4", "none of"),
    ("storage", "int4", "stores"),
    ("value_bits", 8, "stores"),
    ("mode", "group_wise_symmetric", "per-output-channel"),
    ("target", "something_else", "no known layout"),
    ("mixed_int8_suffixes", ["qkv_proj.weight"], "unknown projection"),
])
def test_record_refusals(pi05, tmp_path, field, value, match):
    ck = _copy(pi05 / "w4fake", tmp_path / "ck")
    _edit_record(ck, lambda r: r.__setitem__(field, value))
    with pytest.raises(ValueError, match=match):
        load.load_rpu_quant_checkpoint(_skeleton(), ck, device="cpu")


def test_missing_or_malformed_record(pi05, tmp_path):
    ck = _copy(pi05 / "w8", tmp_path / "ck")
    (ck / "rpu_quant_config.json").write_text("[1, 2]")
    with pytest.raises(ValueError, match="JSON object"):
        load.read_rpu_quant_config(ck)
    (ck / "rpu_quant_config.json").unlink()
    with pytest.raises(FileNotFoundError, match="rpu_quant_config.json"):
        load.load_rpu_quant_checkpoint(_skeleton(), ck, device="cpu")


def test_wall_oss_list_must_match_the_model(wall, tmp_path):
    ck = _copy(wall / "w8", tmp_path / "ck")
    _edit_record(ck, lambda r: r.update(quantized_weights=r["quantized_weights"] + ["nope.weight"],
                                        quantized_weight_count=r["quantized_weight_count"] + 1))
    with pytest.raises(TypeError, match="not the weight of an nn.Linear"):
        load.load_rpu_quant_checkpoint(_skeleton(WallTree), ck, device="cpu")
    ck2 = _copy(wall / "w8", tmp_path / "ck2")
    _edit_record(ck2, lambda r: r.update(quantized_weight_count=3))
    with pytest.raises(ValueError, match="counts"):
        load.load_rpu_quant_checkpoint(_skeleton(WallTree), ck2, device="cpu")
    ck3 = _copy(wall / "w8", tmp_path / "ck3")
    _edit_record(ck3, lambda r: r.update(quantized_weights=r["quantized_weights"][1:],
                                         quantized_weight_count=r["quantized_weight_count"] - 1))
    with pytest.raises(KeyError, match="does not list"):
        load.load_rpu_quant_checkpoint(_skeleton(WallTree), ck3, device="cpu")


def test_tied_head_is_loaded_once_and_stays_tied(tmp_path):
    """A head sharing the embedding table: the checkpoint holds the table once
    (embed_tokens.weight, kept floating by the default skip list) and the
    loaded model keeps one tensor under both names."""
    write_wall_source(tmp_path / "src", seed=9, tied_head=True)
    convert.convert_wall_oss_checkpoint(tmp_path / "src", tmp_path / "w8", **QUIET)
    ck = read_all(tmp_path / "w8")
    assert "head.weight" not in ck
    model = _skeleton(WallTree, tied_head=True)
    swapped = load.load_rpu_quant_checkpoint(model, tmp_path / "w8", device="cpu")
    assert len(swapped) == 8
    assert model.head.weight is model.embed_tokens.weight
    assert torch.equal(model.head.weight, ck["embed_tokens.weight"])
