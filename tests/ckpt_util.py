"""Tiny HF Qwen3 checkpoints for the loader tests (not collected by pytest)."""
from __future__ import annotations

from pathlib import Path

import torch
import transformers
from safetensors.torch import load_file

from rhinoforge_amd.quant import convert


def tiny_config(**kw):
    base = dict(vocab_size=384, hidden_size=128, intermediate_size=320, num_hidden_layers=2,
                num_attention_heads=4, num_key_value_heads=2, head_dim=32,
                max_position_embeddings=128, tie_word_embeddings=True)
    base.update(kw)
    return transformers.Qwen3Config(**base)


def write_source(path: Path, seed: int = 0, shard: str | None = None, **kw) -> torch.nn.Module:
    torch.manual_seed(seed)
    model = transformers.Qwen3ForCausalLM(tiny_config(**kw)).eval()
    kwargs = {"max_shard_size": shard} if shard else {}
    model.save_pretrained(path, safe_serialization=True, **kwargs)
    return model


def read_all(path: Path) -> dict[str, torch.Tensor]:
    out = {}
    for shard in convert.checkpoint_shards(path)[0]:
        out.update(load_file(str(path / shard)))
    return out


# ---- Pi0.5 and Wall-OSS module trees (rpu_quant_config.json checkpoints) -----
def gemma_config(hidden: int, inter: int, layers: int = 2, **kw):
    base = dict(vocab_size=256, hidden_size=hidden, intermediate_size=inter,
                num_hidden_layers=layers, num_attention_heads=4, num_key_value_heads=1,
                head_dim=32, max_position_embeddings=128)
    base.update(kw)
    return transformers.GemmaConfig(**base)


class Pi05Tree(torch.nn.Module):
    """The module names of a Pi0.5 policy around its two Gemma decoders
    (``model.paligemma_with_expert.paligemma.model.language_model`` and
    ``model.paligemma_with_expert.gemma_expert.model``), plus two floating
    action projections that no conversion touches."""

    def __init__(self, vlm=(128, 256), expert=(64, 128), action_dim: int = 32):
        super().__init__()
        nn = torch.nn
        self.model = nn.Module()
        pwe = self.model.paligemma_with_expert = nn.Module()
        pwe.paligemma = nn.Module()
        pwe.paligemma.model = nn.Module()
        pwe.paligemma.model.language_model = transformers.GemmaModel(gemma_config(*vlm))
        pwe.gemma_expert = nn.Module()
        pwe.gemma_expert.model = transformers.GemmaModel(gemma_config(*expert))
        self.model.action_in_proj = nn.Linear(action_dim, expert[0])
        self.model.action_out_proj = nn.Linear(expert[0], action_dim)

    def vlm(self):
        return self.model.paligemma_with_expert.paligemma.model.language_model

    def expert(self):
        return self.model.paligemma_with_expert.gemma_expert.model


class WallTree(torch.nn.Module):
    """A small stand-in with Wall-OSS-style names: an embedding, biased
    attention projections, an MoE-style expert MLP and norms."""

    def __init__(self, vocab: int = 256, hidden: int = 64, inter: int = 192, odd_k: bool = False,
                 tied_head: bool = False):
        super().__init__()
        nn = torch.nn
        self.embed_tokens = nn.Embedding(vocab, hidden)
        self.layers = nn.ModuleList()
        for _ in range(2):
            blk = nn.Module()
            blk.self_attn = nn.Module()
            blk.self_attn.qkv_proj = nn.Linear(hidden, 3 * hidden, bias=True)
            blk.self_attn.o_proj = nn.Linear(hidden, hidden, bias=False)
            blk.mlp = nn.Module()
            blk.mlp.gate_up_proj = nn.Linear(hidden, 2 * inter, bias=False)
            blk.mlp.down_proj = nn.Linear(inter, hidden, bias=False)
            blk.norm = nn.LayerNorm(hidden)
            self.layers.append(blk)
        if tied_head:   # an output head sharing the embedding table
            self.head = nn.Linear(hidden, vocab, bias=False)
            self.head.weight = self.embed_tokens.weight
        else:
            self.head = nn.Linear(30 if odd_k else hidden, 48, bias=True)

    def forward(self, ids):
        h = self.embed_tokens(ids)
        for blk in self.layers:
            q, k, v = blk.self_attn.qkv_proj(h).chunk(3, dim=-1)
            h = h + blk.self_attn.o_proj(torch.tanh(q) * k + v)
            g, u = blk.mlp.gate_up_proj(blk.norm(h)).chunk(2, dim=-1)
            h = h + blk.mlp.down_proj(torch.nn.functional.silu(g) * u)
        return self.head(h)


def write_tree(path: Path, model: torch.nn.Module, config: dict) -> None:
    """Save ``model``'s state dict as one safetensors shard plus config.json."""
    from safetensors.torch import save_file
    import json
    path.mkdir(parents=True, exist_ok=True)
    sd, seen = {}, set()
    for k, v in model.state_dict(keep_vars=True).items():
        if id(v) in seen:
            continue  # a tied tensor is stored once, under its first name
        seen.add(id(v))
        sd[k] = v.detach().contiguous()
    save_file(sd, str(path / "model.safetensors"))
    (path / "config.json").write_text(json.dumps(config))


def write_pi05_source(path: Path, seed: int = 0, **kw) -> Pi05Tree:
    torch.manual_seed(seed)
    model = Pi05Tree(**kw).eval()
    write_tree(path, model, {"type": "pi05", "tiny": True})
    return model


def write_wall_source(path: Path, seed: int = 0, **kw) -> WallTree:
    torch.manual_seed(seed)
    model = WallTree(**kw).eval()
    write_tree(path, model, {"model_type": "wall_oss", "tiny": True})
    return model
