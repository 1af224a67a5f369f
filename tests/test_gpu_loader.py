"""A converted HF Qwen3 checkpoint, loaded with ``W8A16Linear`` swap-in, on the GPU.

* every loaded projection (decoder and lm_head) against the fp64 oracle on the
  checkpoint's own int8 rows, through the GEMV (M <= 64) and GEMM paths;
* end-to-end logits against the same model computed on the CPU in fp32 with
  the dequantized weights ``f32(s) * f32(q)`` (the verifier form,
  quant/verify_qwen3_w8a16.py:185-197), and against an fp16 HF model on the
  GPU whose Linear weights are ``RN_fp16(s * q)`` (the reference's dequant,
  quant/_common.py:39-41);
* greedy decode through HF ``generate`` (KV cache, M=1 GEMV launches);
* KV-head replication leaves the logits unchanged;
* the fused lm_head argmax on the loaded head.

Tolerances: projections use the op's bar (max|err| <= 1e-2 rms(y_cpu), cos >=
0.9999).  Whole-model fp16 logits: per-row cos >= 0.9999 and max|err| <= 2e-2
rms against the fp32 CPU model and against the fp16 GPU model.  A greedy token must equal the CPU model's argmax wherever that
argmax leads the runner-up by more than 4x the row's max logit error.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

transformers = pytest.importorskip("transformers")

import rhinoforge_amd as rf  # noqa: E402
from rhinoforge_amd.quant import convert, load  # noqa: E402
from oracle import w8a16 as o  # noqa: E402
from ckpt_util import read_all, write_source  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda"
SHAPE = dict(vocab_size=1000, hidden_size=256, intermediate_size=704, num_attention_heads=8,
             num_key_value_heads=2, head_dim=32, max_position_embeddings=256)


def _say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    root = tmp_path_factory.mktemp("w8a16_gpu_ckpt")
    write_source(root / "src", seed=7, **SHAPE)
    convert.convert_checkpoint(root / "src", root / "dst", quant_lm_head=True, log=lambda *a: None)
    return root / "dst"


@pytest.fixture(scope="module")
def model(ckpt):
    return load.load_w8a16_model(None, ckpt, device=DEV)


def _ids(batch, seq, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, SHAPE["vocab_size"], (batch, seq), generator=g)


def _cpu_reference(ckpt) -> torch.nn.Module:
    """fp32 CPU model: quantized weights as f32(s)*f32(q), the rest as stored."""
    ck = read_all(ckpt)
    cfg = transformers.AutoConfig.from_pretrained(str(ckpt), local_files_only=True)
    ref = transformers.Qwen3ForCausalLM(cfg).float().eval()
    with torch.no_grad():
        for name, p in ref.named_parameters():
            t = ck[name]
            if t.dtype == torch.int8:
                s = ck[name[: -len(".weight")] + ".weight_scale"]
                p.copy_(s.float()[:, None] * t.float())
            else:
                p.copy_(t.float())
    return ref


def _gpu_fp16_reference(ckpt) -> torch.nn.Module:
    ck = read_all(ckpt)
    cfg = transformers.AutoConfig.from_pretrained(str(ckpt), local_files_only=True)
    ref = transformers.Qwen3ForCausalLM(cfg).to(torch.float16).eval()
    with torch.no_grad():
        for name, p in ref.named_parameters():
            t = ck[name]
            if t.dtype == torch.int8:
                s = ck[name[: -len(".weight")] + ".weight_scale"]
                p.copy_(rf.dequantize_linear_per_channel(t, s))
            else:
                p.copy_(t)
    return ref.to(DEV)


def _row_stats(y, ref):
    y, ref = y.double().reshape(-1, y.shape[-1]), ref.double().reshape(-1, ref.shape[-1])
    cos = torch.nn.functional.cosine_similarity(y, ref, dim=1)
    err = (y - ref).abs().max().item()
    rms = ref.pow(2).mean().sqrt().item()
    return cos.min().item(), err / rms, (y - ref).abs().amax(dim=1)


@pytest.mark.parametrize("m", [1, 5, 96])
def test_loaded_projections_match_oracle(model, ckpt, m):
    ck = read_all(ckpt)
    n = 0
    for name, mod in model.named_modules():
        if not isinstance(mod, rf.W8A16Linear):
            continue
        q = ck[name + ".weight"].numpy()
        s = ck[name + ".weight_scale"].numpy()
        x = o.make_activation(o.derive_seed(5, name, m), m, mod.in_features)
        y = mod(torch.from_numpy(x).to(DEV))
        torch.cuda.synchronize()
        rep = o.check_tolerance(y.cpu().numpy(), o.cpu_path(x, q, s), o.oracle_fp64(x, q, s))
        assert rep.ok, f"{name} m={m}: {rep}"
        n += 1
    _say(f"  m={m}: {n} projections within tolerance")
    assert n == 2 * 7 + 1


@pytest.mark.parametrize("batch,seq", [(1, 5), (2, 48)])
def test_end_to_end_logits(model, ckpt, batch, seq):
    ids = _ids(batch, seq, seed=batch * 100 + seq)
    with torch.no_grad():
        y = model(ids.to(DEV)).logits.float().cpu()
        ref32 = _cpu_reference(ckpt)(ids).logits
        ref16 = _gpu_fp16_reference(ckpt)(ids.to(DEV)).logits.float().cpu()
    cos32, rel32, _ = _row_stats(y, ref32)
    cos16, rel16, _ = _row_stats(y, ref16)
    _say(f"  batch={batch} seq={seq}: vs fp32 CPU cos_min={cos32:.7f} err/rms={rel32:.4f}; "
         f"vs fp16 GPU cos_min={cos16:.7f} err/rms={rel16:.4f}")
    assert torch.isfinite(y).all()
    assert cos32 >= 0.9999 and rel32 <= 2e-2
    assert cos16 >= 0.9999 and rel16 <= 2e-2


def test_greedy_generate_agrees_with_cpu_model(model, ckpt):
    ids = _ids(2, 12, seed=3)
    with torch.no_grad():
        out = model.generate(ids.to(DEV), attention_mask=torch.ones_like(ids).to(DEV),
                             max_new_tokens=8, do_sample=False, pad_token_id=0).cpu()
        ref = _cpu_reference(ckpt)(out).logits
        mine = model(out.to(DEV)).logits.float().cpu()
    assert out.shape == (2, 20)
    checked = 0
    for b in range(2):
        for pos in range(11, 19):
            row = ref[b, pos]
            top2 = row.topk(2).values
            err = (mine[b, pos] - row).abs().max().item()
            if (top2[0] - top2[1]).item() > 4 * err:
                assert out[b, pos + 1].item() == int(row.argmax()), (b, pos)
                checked += 1
    _say(f"  greedy tokens checked against the CPU model: {checked}/16")
    assert checked >= 8


def test_kv_replication_keeps_logits(ckpt):
    ids = _ids(2, 24, seed=9)
    base = load.load_w8a16_model(None, ckpt, device=DEV)
    with torch.no_grad():
        y0 = base(ids.to(DEV)).logits.float().cpu()
    assert load.replicate_kv_heads(base.model, 8) == 8
    assert base.model.layers[0].self_attn.k_proj.out_features == 8 * 32
    with torch.no_grad():
        y1 = base(ids.to(DEV)).logits.float().cpu()
    cos, rel, _ = _row_stats(y1, y0)
    _say(f"  replicated 2->8 KV heads: cos_min={cos:.8f} err/rms={rel:.5f}")
    assert cos >= 0.99999 and rel <= 1e-2


def test_fused_argmax_on_loaded_lm_head(model):
    ids = _ids(3, 16, seed=21)
    with torch.no_grad():
        h = model.model(ids.to(DEV)).last_hidden_state[:, -1].contiguous()
        head = model.lm_head
        idx, logits = rf.linear_argmax(h, head.weight, head.weight_scale, return_logits=True)
        plain = head(h)
    torch.cuda.synchronize()
    lg = logits.float().cpu()
    cos, rel, _ = _row_stats(lg, plain.float().cpu())
    assert cos >= 0.9999 and rel <= 1e-2
    first = torch.tensor([int(np.flatnonzero(r == r.max())[0]) for r in lg.numpy()])
    assert torch.equal(idx.cpu().long(), first)
