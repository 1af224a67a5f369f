"""Checkpoint converter, loader and swap-in on the CPU (no kernel calls).

A tiny random Qwen3 checkpoint is written with ``save_pretrained``, converted
to the W8A16 on-disk format and loaded back.  What is checked:

* the converter writes exactly ``quantize_linear_per_channel`` of the fp16
  source for every projection (and the derived lm_head), fp16 for the rest,
  the reference's ``quant_config`` record, and a consistent shard index;
* the loader installs ``W8A16Linear`` modules whose packed weight unpacks to
  the checkpoint's int8 rows, and refuses every inventory, dtype and shape
  mismatch before any weight is read;
* KV-head replication in packed form equals replication of the row-major
  weight followed by packing.
"""
from __future__ import annotations

import json
import shutil
from pathlib import Path

import pytest
import torch
from safetensors import safe_open
from safetensors.torch import load_file, save_file

transformers = pytest.importorskip("transformers")

import rhinoforge_amd as rf  # noqa: E402
from rhinoforge_amd.quant import convert, load  # noqa: E402
from rhinoforge_amd.quant._common import quantize_linear_per_channel  # noqa: E402
from ckpt_util import read_all, tiny_config, write_source  # noqa: E402


@pytest.fixture(scope="module")
def ckpts(tmp_path_factory):
    root = tmp_path_factory.mktemp("w8a16_ckpt")
    write_source(root / "src")
    convert.convert_checkpoint(root / "src", root / "dst", quant_lm_head=True, log=lambda *a: None)
    convert.convert_checkpoint(root / "src", root / "dst_plain", log=lambda *a: None)
    return root


def _copy(src: Path, dst: Path) -> Path:
    shutil.copytree(src, dst)
    return dst


# ---------------------------------------------------------------- converter

def test_converter_quantizes_projections_exactly(ckpts):
    src, dst = read_all(ckpts / "src"), read_all(ckpts / "dst")
    n_proj = 0
    for name, w in src.items():
        if name.endswith(convert.QUANT_PROJ_SUFFIXES):
            q, s = quantize_linear_per_channel(w)
            assert dst[name].dtype == torch.int8 and torch.equal(dst[name], q), name
            assert torch.equal(dst[convert.scale_name(name)], s), name
            n_proj += 1
        else:
            assert dst[name].dtype == torch.float16
            assert torch.equal(dst[name], w.to(torch.float16)), name
    assert n_proj == 2 * 7
    # Tied source: lm_head derived from the embedding and quantized.
    assert "lm_head.weight" not in src
    q, s = quantize_linear_per_channel(src["model.embed_tokens.weight"])
    assert torch.equal(dst["lm_head.weight"], q)
    assert torch.equal(dst["lm_head.weight_scale"], s)


def test_converter_config_record(ckpts):
    cfg = json.loads((ckpts / "dst" / "config.json").read_text())
    assert cfg["quant_config"] == {
        "method": "w8a16", "mode": "per_channel_symmetric", "qaxis": 0, "skip_modules": [],
        "quantized_lm_head": True, "quantized_embed_tokens": False, "lm_head_untied": True,
        "embed_tokens_untied": False}
    assert cfg["tie_word_embeddings"] is False and cfg["torch_dtype"] == "float16"
    plain = json.loads((ckpts / "dst_plain" / "config.json").read_text())
    assert plain["quant_config"]["skip_modules"] == ["lm_head"]
    assert plain["tie_word_embeddings"] is True
    assert "lm_head.weight" not in read_all(ckpts / "dst_plain")
    assert (ckpts / "dst" / "generation_config.json").is_file()


def test_converter_refuses_overwrite_and_copies_int8(ckpts, tmp_path):
    with pytest.raises(FileExistsError):
        convert.convert_checkpoint(ckpts / "src", ckpts / "dst", log=lambda *a: None)
    stats = convert.convert_checkpoint(ckpts / "dst", tmp_path / "again", skip_modules=[],
                                       log=lambda *a: None)
    assert stats["quantized"] == 0
    a, b = read_all(ckpts / "dst"), read_all(tmp_path / "again")
    assert a.keys() == b.keys() and all(torch.equal(a[k], b[k]) for k in a)


def test_converter_sharded_index(tmp_path):
    write_source(tmp_path / "src", shard="150KB")
    shards, index = convert.checkpoint_shards(tmp_path / "src")
    assert index is not None and len(shards) > 1
    convert.convert_checkpoint(tmp_path / "src", tmp_path / "dst", quant_lm_head=True,
                               quant_embed_tokens=True, log=lambda *a: None)
    new_shards, new_index = convert.checkpoint_shards(tmp_path / "dst")
    assert new_shards == shards
    wm = new_index["weight_map"]
    for shard in new_shards:
        with safe_open(str(tmp_path / "dst" / shard), framework="pt") as f:
            for name in f.keys():
                assert wm[name] == shard, name
    assert set(wm) == set(read_all(tmp_path / "dst"))
    dst = read_all(tmp_path / "dst")
    # Quantized embedding and the lm_head derived from it are the same pair.
    assert torch.equal(dst["lm_head.weight"], dst["model.embed_tokens.weight"])
    assert torch.equal(dst["lm_head.weight_scale"], dst["model.embed_tokens.weight_scale"])
    assert new_index["metadata"]["total_size"] == sum(
        t.numel() * t.element_size() for t in dst.values())


def test_verify_checkpoint_passes_and_catches_a_bad_scale(ckpts, tmp_path):
    worst = convert.verify_checkpoint(ckpts / "src", ckpts / "dst")
    assert worst["n"] == 15 and worst["cosine"] > 0.9999
    bad = _copy(ckpts / "dst", tmp_path / "bad")
    t = load_file(str(bad / "model.safetensors"))
    name = "model.layers.1.mlp.up_proj.weight_scale"
    t[name] = t[name].clone()
    t[name][::2] = -t[name][::2]          # flip half the rows' sign
    save_file(t, str(bad / "model.safetensors"), metadata={"format": "pt"})
    with pytest.raises(ValueError, match="up_proj"):
        convert.verify_checkpoint(ckpts / "src", bad)


# ---------------------------------------------------------------- loader

def test_is_w8a16_config():
    from types import SimpleNamespace
    assert load.is_w8a16_config(SimpleNamespace(quant_config={"method": "w8a16"}))
    assert not load.is_w8a16_config(SimpleNamespace(quant_config={"method": "other"}))
    assert not load.is_w8a16_config(SimpleNamespace())


def test_loader_installs_packed_projections(ckpts):
    ck = read_all(ckpts / "dst")
    model = load.load_w8a16_model(None, ckpts / "dst", device="cpu")
    n = 0
    for name, mod in model.named_modules():
        if isinstance(mod, rf.W8A16Linear):
            assert torch.equal(mod.rowmajor_weight(), ck[name + ".weight"]), name
            assert torch.equal(mod.weight_scale, ck[name + ".weight_scale"]), name
            assert mod.weight.shape == rf.packed_shape(mod.out_features, mod.in_features)
            n += 1
    assert n == 15 and isinstance(model.lm_head, rf.W8A16Linear)
    assert torch.equal(model.model.norm.weight, ck["model.norm.weight"])
    assert model.model.embed_tokens.weight.dtype == torch.float16
    fresh = transformers.Qwen3ForCausalLM(tiny_config()).model.rotary_emb
    assert torch.equal(model.model.rotary_emb.inv_freq, fresh.inv_freq)
    assert load.detect_and_validate_decoder_w8a16(model.model)
    lists = load.decoder_scale_lists(model.model)
    assert len(lists) == 7 and all(len(x) == 2 for x in lists)
    assert lists[1][0] is model.model.layers[0].self_attn.k_proj.weight_scale


def test_loader_tied_lm_head_and_int8_embedding(ckpts, tmp_path):
    plain = load.load_w8a16_model(None, ckpts / "dst_plain", device="cpu")
    assert isinstance(plain.lm_head, torch.nn.Linear)
    assert plain.lm_head.weight is plain.model.embed_tokens.weight
    convert.convert_checkpoint(ckpts / "src", tmp_path / "emb", quant_lm_head=True,
                               quant_embed_tokens=True, log=lambda *a: None)
    m = load.load_w8a16_model(None, tmp_path / "emb", device="cpu")
    emb = m.model.embed_tokens
    assert isinstance(emb, rf.W8A16Embedding)
    ids = torch.tensor([[0, 5, 383, 5]])
    out = emb(ids)
    want = (emb.weight[ids].float() * emb.weight_scale[ids].float()[..., None]).half()
    assert out.dtype == torch.float16 and torch.equal(out, want)
    # the closed form fp16(f32(q)*f32(s)) == RN_fp16(s*q): exact product, one rounding
    direct = (emb.weight[ids].double() * emb.weight_scale[ids].double()[..., None]).half()
    assert torch.equal(out, direct)


def test_loaded_model_refuses_cpu_forward(ckpts):
    model = load.load_w8a16_model(None, ckpts / "dst", device="cpu")
    with pytest.raises(RuntimeError, match="CPU"):
        model(torch.tensor([[1, 2, 3]]))


def _rewrite(path: Path, fn) -> None:
    t = load_file(str(path / "model.safetensors"))
    fn(t)
    save_file(t, str(path / "model.safetensors"), metadata={"format": "pt"})


@pytest.mark.parametrize("case,exc,match", [
    ("drop_scale", KeyError, "with no fp16 scale"),
    ("fp32_scale", TypeError, "scales are fp16"),
    ("short_scale", ValueError, "one entry per weight row"),
    ("extra_tensor", KeyError, "has no parameter of that name"),
    ("drop_norm", KeyError, "absent from the checkpoint"),
    ("orphan_scale", KeyError, "no int8 weight beside it"),
    ("float_projection", KeyError, "differ from what quant_config implies"),
    ("int32_tensor", TypeError, "floating tensors only"),
    ("wrong_shape", ValueError, "checkpoint shape"),
])
def test_loader_refuses_bad_checkpoints(ckpts, tmp_path, case, exc, match):
    d = _copy(ckpts / "dst", tmp_path / case)
    p = "model.layers.0.self_attn.v_proj"

    def edit(t):
        if case == "drop_scale":
            del t[p + ".weight_scale"]
        elif case == "fp32_scale":
            t[p + ".weight_scale"] = t[p + ".weight_scale"].float()
        elif case == "short_scale":
            t[p + ".weight_scale"] = t[p + ".weight_scale"][:-1].clone()
        elif case == "extra_tensor":
            t["model.layers.0.bogus.weight"] = torch.zeros(4, dtype=torch.float16)
        elif case == "drop_norm":
            del t["model.norm.weight"]
        elif case == "orphan_scale":
            t["model.norm.weight_scale"] = torch.ones(128, dtype=torch.float16)
        elif case == "float_projection":
            t[p + ".weight"] = t[p + ".weight"].to(torch.float16)
            del t[p + ".weight_scale"]
        elif case == "int32_tensor":
            t["model.norm.weight"] = t["model.norm.weight"].to(torch.int32)
        elif case == "wrong_shape":
            t[p + ".weight"] = t[p + ".weight"][:, :64].clone()
    _rewrite(d, edit)
    with pytest.raises(exc, match=match):
        load.load_w8a16_model(None, d, device="cpu")


def test_loader_refuses_non_local_and_unmarked(ckpts, tmp_path):
    with pytest.raises(FileNotFoundError, match="local directory"):
        load.load_w8a16_model(None, "Qwen/Qwen3-8B", device="cpu")
    with pytest.raises(ValueError, match="w8a16"):
        load.load_w8a16_model(None, ckpts / "src", device="cpu")


def test_loader_refuses_index_mismatch(tmp_path):
    write_source(tmp_path / "src", shard="150KB")
    convert.convert_checkpoint(tmp_path / "src", tmp_path / "dst", log=lambda *a: None)
    idx_path = tmp_path / "dst" / "model.safetensors.index.json"
    idx = json.loads(idx_path.read_text())
    good = load.load_w8a16_model(None, tmp_path / "dst", device="cpu")
    assert load.detect_and_validate_decoder_w8a16(good.model)
    name = "model.norm.weight"
    other = [s for s in sorted(set(idx["weight_map"].values())) if s != idx["weight_map"][name]]
    idx["weight_map"][name] = other[0]
    idx_path.write_text(json.dumps(idx))
    with pytest.raises(KeyError, match="index puts"):
        load.load_w8a16_model(None, tmp_path / "dst", device="cpu")


# ---------------------------------------------------------------- swap-in

def _reference_loader_form(ckpts) -> torch.nn.Module:
    """The reference loader's output: nn.Linear with an int8 Parameter and a
    fp16 weight_scale buffer (quant/load.py:258-284)."""
    ck = read_all(ckpts / "dst")
    cfg = transformers.AutoConfig.from_pretrained(str(ckpts / "dst"), local_files_only=True)
    model = transformers.Qwen3ForCausalLM(cfg).to(torch.float16).eval()
    for name, mod in model.named_modules():
        if name + ".weight_scale" in ck:
            mod.weight = torch.nn.Parameter(ck[name + ".weight"], requires_grad=False)
            mod.register_buffer("weight_scale", ck[name + ".weight_scale"])
    return model


def test_swap_w8a16_linears(ckpts):
    model = _reference_loader_form(ckpts)
    swapped = load.swap_w8a16_linears(model)
    assert len(swapped) == 15 and "lm_head" in swapped
    ck = read_all(ckpts / "dst")
    for name in swapped:
        mod = model.get_submodule(name)
        assert isinstance(mod, rf.W8A16Linear)
        assert torch.equal(mod.rowmajor_weight(), ck[name + ".weight"])
    assert load.swap_w8a16_linears(model) == []
    with pytest.raises(TypeError, match="parent"):
        load.swap_w8a16_linears(torch.nn.Linear(8, 8))
    bad = torch.nn.Sequential(torch.nn.Linear(8, 8))
    bad[0].weight = torch.nn.Parameter(torch.zeros(8, 8, dtype=torch.int8), requires_grad=False)
    with pytest.raises(KeyError, match="weight_scale"):
        load.swap_w8a16_linears(bad)


def test_partial_decoder_is_refused(ckpts):
    model = load.load_w8a16_model(None, ckpts / "dst", device="cpu")
    model.model.layers[1].mlp.up_proj = torch.nn.Linear(128, 320, bias=False)
    with pytest.raises(ValueError, match="partially W8A16"):
        load.decoder_scale_lists(model.model)
    fp = transformers.Qwen3ForCausalLM(tiny_config())
    assert load.decoder_scale_lists(fp.model) == ([], [], [], [], [], [], [])


# ---------------------------------------------------------------- KV replication

@pytest.mark.parametrize("head_dim", [32, 24])
def test_replicate_kv_heads_packed_matches_rowmajor(tmp_path, head_dim):
    kw = dict(head_dim=head_dim, attention_bias=True)
    write_source(tmp_path / "src", seed=3, **kw)
    convert.convert_checkpoint(tmp_path / "src", tmp_path / "dst", log=lambda *a: None)
    model = load.load_w8a16_model(None, tmp_path / "dst", device="cpu")
    dec = model.model
    before = {i: (l.self_attn.k_proj.rowmajor_weight(), l.self_attn.k_proj.weight_scale.clone(),
                  l.self_attn.k_proj.bias.clone()) for i, l in enumerate(dec.layers)}
    assert load.replicate_kv_heads(dec, 4) == 4
    for i, layer in enumerate(dec.layers):
        k = layer.self_attn.k_proj
        q0, s0, b0 = before[i]
        want_q = q0.view(2, head_dim, 128).repeat_interleave(2, 0).reshape(4 * head_dim, 128)
        assert k.out_features == 4 * head_dim
        assert torch.equal(k.rowmajor_weight(), want_q)
        assert torch.equal(k.weight, rf.pack_weight(want_q))
        assert torch.equal(k.weight_scale, s0.view(2, head_dim).repeat_interleave(2, 0).flatten())
        assert torch.equal(k.bias, b0.view(2, head_dim).repeat_interleave(2, 0).flatten())
        assert layer.self_attn.num_key_value_groups == 1
    assert load.replicate_kv_heads(dec, 4) == 4            # idempotent
    with pytest.raises(ValueError, match="already replicated"):
        load.replicate_kv_heads(dec, 2)
    fresh = load.load_w8a16_model(None, tmp_path / "dst", device="cpu").model
    with pytest.raises(ValueError, match="multiple"):
        load.replicate_kv_heads(fresh, 3)
    with pytest.raises(ValueError, match="divisible"):
        load.replicate_kv_heads(fresh, 8)


def test_qwen3_vl_checkpoint_loads_with_text_projections_swapped(tmp_path):
    """The VL family (AutoModelForImageTextToText): the text decoder's seven
    projections per layer become W8A16Linear; the vision tower stays floating
    (its attn.qkv / mlp.linear_fc* names are not quantized projections,
    quant/convert_qwen3.py:25-33)."""
    if not hasattr(transformers, "Qwen3VLConfig"):
        pytest.skip("transformers without Qwen3-VL")
    torch.manual_seed(0)
    cfg = transformers.Qwen3VLConfig(
        text_config=dict(vocab_size=512, hidden_size=128, intermediate_size=256,
                         num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                         head_dim=32, max_position_embeddings=256,
                         rope_scaling={"rope_type": "default", "mrope_section": [4, 6, 6]}),
        vision_config=dict(depth=2, hidden_size=64, intermediate_size=128, num_heads=2,
                           out_hidden_size=128, deepstack_visual_indexes=[1], patch_size=16,
                           temporal_patch_size=2, spatial_merge_size=2))
    transformers.Qwen3VLForConditionalGeneration(cfg).save_pretrained(
        tmp_path / "src", safe_serialization=True)
    stats = convert.convert_checkpoint(tmp_path / "src", tmp_path / "dst", log=lambda *a: None)
    assert stats["quantized"] == 2 * 7
    model = load.load_w8a16_model(None, tmp_path / "dst", device="cpu")
    assert type(model).__name__ == "Qwen3VLForConditionalGeneration"
    assert load.detect_and_validate_decoder_w8a16(model.model.language_model)
    assert not any(isinstance(m, rf.W8A16Linear) for m in model.model.visual.modules())
    ck = read_all(tmp_path / "dst")
    for name, mod in model.named_modules():
        if isinstance(mod, rf.W8A16Linear):
            assert torch.equal(mod.rowmajor_weight(), ck[name + ".weight"]), name
