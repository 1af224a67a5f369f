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
