"""Pi0.5, Wall-OSS and Qwen3-VL W8A16 checkpoints loaded with swap-in, on the GPU.

* every swapped Pi0.5 projection (``W8A16Linear``, and ``W4A16Linear`` for a
  real-W4 record) against the fp64 oracle on the checkpoint's own int8 rows;
* both Pi0.5 Gemma decoders (the VLM and the action expert), the Wall-OSS
  stand-in and a Qwen3-VL text stack end to end against the same modules
  computed on the CPU in fp32 with the dequantized weights ``f32(s) *
  f32(q)`` (the verifier form, quant/verify_qwen3_w8a16.py:185-197);
* KV-head replication of the expert's int8 k/v projections leaves its output
  unchanged.

Tolerances: projections use the op's bar (max|err| <= 1e-2 rms(y_cpu), cos >=
0.9999 against the fp64 oracle).  Whole stacks in fp16 on the GPU against fp32
on the CPU: per-row cos >= 0.9999 and max|err| <= 2e-2 rms.
"""
from __future__ import annotations

import pytest
import torch

transformers = pytest.importorskip("transformers")

import rhinoforge_amd as rf  # noqa: E402
from rhinoforge_amd.quant import convert, load  # noqa: E402
from oracle import w8a16 as o8, w4a16 as o4  # noqa: E402
from ckpt_util import (Pi05Tree, WallTree, read_all, write_pi05_source,  # noqa: E402
                       write_wall_source)

pytestmark = pytest.mark.gpu
DEV = "cuda"
QUIET = dict(log=lambda *a: None)
PI05 = dict(vlm=(256, 512), expert=(128, 256))


def _say(*a):
    print(*a, flush=True)


def _fill_dequantized(ref: torch.nn.Module, ck: dict, prefix: str = "") -> torch.nn.Module:
    """fp32 copy of a checkpoint: int8 weights as f32(s)*f32(q), the rest as stored."""
    with torch.no_grad():
        for name, p in ref.named_parameters():
            t = ck[prefix + name]
            if t.dtype == torch.int8:
                s = ck[prefix + name[: -len(".weight")] + ".weight_scale"]
                p.copy_(s.float()[:, None] * t.float())
            else:
                p.copy_(t.float())
    return ref.float().eval()


def _row_stats(y, ref):
    y, ref = y.double().reshape(-1, y.shape[-1]), ref.double().reshape(-1, ref.shape[-1])
    cos = torch.nn.functional.cosine_similarity(y, ref, dim=1).min().item()
    rel = ((y - ref).abs().max() / ref.pow(2).mean().sqrt()).item()
    return cos, rel


def _embeds(batch, seq, hidden, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(batch, seq, hidden, generator=g)


@pytest.fixture(scope="module")
def pi05(tmp_path_factory):
    root = tmp_path_factory.mktemp("pi05_gpu")
    write_pi05_source(root / "src", seed=11, **PI05)
    convert.convert_pi05_checkpoint(root / "src", root / "w8", **QUIET)
    convert.convert_pi05_checkpoint(root / "src", root / "w4fake", bits=4, **QUIET)
    convert.convert_pi05_checkpoint(root / "src", root / "w4real", bits=4, real_w4=True, **QUIET)
    return root


def _load_pi05(ckpt):
    with torch.device("meta"):
        model = Pi05Tree(**PI05)
    swapped = load.load_rpu_quant_checkpoint(model, ckpt, device=DEV)
    assert len(swapped) == 28
    return model.eval()


@pytest.mark.parametrize("variant", ["w8", "w4real"])
@pytest.mark.parametrize("m", [1, 7, 96])
def test_pi05_projections_match_oracle(pi05, variant, m):
    model = _load_pi05(pi05 / variant)
    ck = read_all(pi05 / variant)
    n8 = n4 = 0
    for name, mod in model.named_modules():
        if not isinstance(mod, (rf.W8A16Linear, rf.W4A16Linear)):
            continue
        q = ck[name + ".weight"].numpy()
        s = ck[name + ".weight_scale"].numpy()
        x = o8.make_activation(o8.derive_seed(17, name, m), m, mod.in_features)
        y = mod(torch.from_numpy(x).to(DEV))
        torch.cuda.synchronize()
        o = o4 if isinstance(mod, rf.W4A16Linear) else o8
        rep = o8.check_tolerance(y.cpu().numpy(), o.cpu_path(x, q, s), o.oracle_fp64(x, q, s))
        assert rep.ok, f"{variant} {name} m={m}: {rep}"
        n4 += isinstance(mod, rf.W4A16Linear)
        n8 += isinstance(mod, rf.W8A16Linear)
    _say(f"  {variant} m={m}: {n8} W8A16 + {n4} W4A16 projections within tolerance")
    assert (n8, n4) == ((28, 0) if variant == "w8" else (8, 20))


@pytest.mark.parametrize("variant", ["w8", "w4fake", "w4real"])
@pytest.mark.parametrize("batch,seq", [(2, 5), (2, 48)])
def test_pi05_decoders_match_fp32_cpu(pi05, variant, batch, seq):
    model = _load_pi05(pi05 / variant)
    ck = read_all(pi05 / variant)
    torch.manual_seed(0)
    ref = Pi05Tree(**PI05)
    _fill_dequantized(ref, ck)
    for which, hidden in (("vlm", PI05["vlm"][0]), ("expert", PI05["expert"][0])):
        x = _embeds(batch, seq, hidden, seed=batch * 1000 + seq + hidden)
        with torch.no_grad():
            y = getattr(model, which)()(inputs_embeds=x.to(DEV, torch.float16))
            want = getattr(ref, which)()(inputs_embeds=x)
        y = y.last_hidden_state.float().cpu()
        cos, rel = _row_stats(y, want.last_hidden_state)
        _say(f"  {variant} {which} batch={batch} seq={seq}: cos_min={cos:.7f} err/rms={rel:.4f}")
        assert torch.isfinite(y).all()
        assert cos >= 0.9999 and rel <= 2e-2, (variant, which)


def test_pi05_expert_kv_replication_keeps_output(pi05):
    model = _load_pi05(pi05 / "w8")
    exp = model.expert()
    x = _embeds(2, 24, PI05["expert"][0], seed=4).to(DEV, torch.float16)
    with torch.no_grad():
        y0 = exp(inputs_embeds=x).last_hidden_state.float().cpu()
    assert load.replicate_kv_heads(exp, 4, label="expert") == 4
    assert exp.layers[0].self_attn.k_proj.out_features == 4 * 32
    with torch.no_grad():
        y1 = exp(inputs_embeds=x).last_hidden_state.float().cpu()
    cos, rel = _row_stats(y1, y0)
    _say(f"  expert KV 1->4 heads: cos_min={cos:.8f} err/rms={rel:.5f}")
    assert cos >= 0.99999 and rel <= 1e-2


@pytest.mark.parametrize("quant_embed", [False, True])
def test_wall_oss_matches_fp32_cpu(tmp_path, quant_embed):
    write_wall_source(tmp_path / "src", seed=6, hidden=128, inter=384)
    skip = () if quant_embed else ("embed_tokens",)
    convert.convert_wall_oss_checkpoint(tmp_path / "src", tmp_path / "w8", skip_modules=skip,
                                        **QUIET)
    with torch.device("meta"):
        model = WallTree(hidden=128, inter=384)
    swapped = load.load_rpu_quant_checkpoint(model, tmp_path / "w8", device=DEV)
    assert len(swapped) == 9 + quant_embed
    ck = read_all(tmp_path / "w8")
    ref = WallTree(hidden=128, inter=384)
    if quant_embed:   # the table is gathered and dequantized; give the CPU model the same rows
        ck = dict(ck)
        ck["embed_tokens.weight"] = (ck["embed_tokens.weight"].float()
                                     * ck.pop("embed_tokens.weight_scale").float()[:, None]
                                     ).to(torch.float16)
    _fill_dequantized(ref, ck)
    g = torch.Generator().manual_seed(8)
    for batch, seq in ((1, 1), (3, 40)):
        ids = torch.randint(0, 256, (batch, seq), generator=g)
        with torch.no_grad():
            y = model(ids.to(DEV)).float().cpu()
            want = ref(ids)
        cos, rel = _row_stats(y, want)
        _say(f"  wall-oss embed={'int8' if quant_embed else 'fp16'} batch={batch} seq={seq}: "
             f"cos_min={cos:.7f} err/rms={rel:.4f}")
        assert cos >= 0.9999 and rel <= 2e-2


def test_qwen3_vl_text_stack_matches_fp32_cpu(tmp_path):
    if not hasattr(transformers, "Qwen3VLConfig"):
        pytest.skip("transformers without Qwen3-VL")
    torch.manual_seed(0)
    cfg = transformers.Qwen3VLConfig(
        text_config=dict(vocab_size=512, hidden_size=256, intermediate_size=512,
                         num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                         head_dim=64, max_position_embeddings=256,
                         rope_scaling={"rope_type": "default", "mrope_section": [8, 12, 12]}),
        vision_config=dict(depth=1, hidden_size=64, intermediate_size=128, num_heads=2,
                           out_hidden_size=256, deepstack_visual_indexes=[0], patch_size=16,
                           temporal_patch_size=2, spatial_merge_size=2))
    transformers.Qwen3VLForConditionalGeneration(cfg).save_pretrained(
        tmp_path / "src", safe_serialization=True)
    convert.convert_checkpoint(tmp_path / "src", tmp_path / "dst", **QUIET)
    model = load.load_w8a16_model(None, tmp_path / "dst", device=DEV).eval()
    text = model.model.language_model
    assert load.detect_and_validate_decoder_w8a16(text)
    ck = read_all(tmp_path / "dst")
    ref_cfg = transformers.AutoConfig.from_pretrained(str(tmp_path / "dst"), local_files_only=True)
    ref = _fill_dequantized(transformers.Qwen3VLForConditionalGeneration(ref_cfg), ck)
    g = torch.Generator().manual_seed(12)
    for batch, seq in ((1, 6), (2, 72)):
        ids = torch.randint(0, 512, (batch, seq), generator=g)
        with torch.no_grad():
            y = model(input_ids=ids.to(DEV)).logits.float().cpu()
            want = ref(input_ids=ids).logits
        cos, rel = _row_stats(y, want)
        _say(f"  qwen3-vl text batch={batch} seq={seq}: cos_min={cos:.7f} err/rms={rel:.4f}")
        assert cos >= 0.9999 and rel <= 2e-2
    n = 0
    for name, mod in text.named_modules():
        if isinstance(mod, rf.W8A16Linear):
            full = "model.language_model." + name
            q, s = ck[full + ".weight"].numpy(), ck[full + ".weight_scale"].numpy()
            x = o8.make_activation(o8.derive_seed(23, name), 9, mod.in_features)
            y = mod(torch.from_numpy(x).to(DEV))
            torch.cuda.synchronize()
            rep = o8.check_tolerance(y.cpu().numpy(), o8.cpu_path(x, q, s),
                                     o8.oracle_fp64(x, q, s))
            assert rep.ok, f"{name}: {rep}"
            n += 1
    assert n == 2 * 7
