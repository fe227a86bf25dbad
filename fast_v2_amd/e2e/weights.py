"""Local-path checkpoint loading for the block-diffusion model (no network).

A Fast-dLLM v2 / Qwen2.5 checkpoint directory holds ``config.json`` and one or more
``*.safetensors`` files whose tensor names are those of the Hugging Face Qwen2 layout
(``model.embed_tokens.weight``, ``model.layers.{i}.self_attn.q_proj.weight`` ...,
``model.norm.weight``, ``lm_head.weight``). BlockDiffusionLM uses the same module
names, so tensors load by name; ``lm_head.weight`` falls back to the embedding when
the checkpoint ties them (``tie_word_embeddings``). Only safetensors files are read
(no pickle).
"""
from __future__ import annotations

import json
from pathlib import Path
from typing import Dict, Iterable, Optional, Union

import torch

from .model import BlockDiffusionConfig, BlockDiffusionLM

_CONFIG_KEYS = ("vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers", "num_attention_heads",
                "num_key_value_heads", "rms_norm_eps", "rope_theta", "bd_size")


def config_from_json(path: Union[str, Path]) -> BlockDiffusionConfig:
    """BlockDiffusionConfig from a checkpoint's config.json (keys it does not hold keep
    the 7B defaults)."""
    data = json.loads(Path(path).read_text())
    return BlockDiffusionConfig(**{k: data[k] for k in _CONFIG_KEYS if k in data})


def _safetensors_files(path: Path) -> Iterable[Path]:
    if path.is_file():
        return [path]
    index = path / "model.safetensors.index.json"
    if index.exists():
        names = sorted(set(json.loads(index.read_text())["weight_map"].values()))
        return [path / n for n in names]
    files = sorted(path.glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"no *.safetensors under {path}")
    return files


@torch.no_grad()
def load_safetensors(model: BlockDiffusionLM, path: Union[str, Path], strict: bool = True) -> Dict[str, list]:
    """Copy the checkpoint's tensors into ``model`` (cast to each parameter's dtype, on
    its device). Returns {"missing": [...], "unexpected": [...]}; with ``strict`` a
    missing parameter (other than a tied lm_head) raises KeyError."""
    from safetensors import safe_open

    params = dict(model.named_parameters())
    loaded = set()
    unexpected = []
    for f in _safetensors_files(Path(path)):
        with safe_open(str(f), framework="pt", device="cpu") as sf:
            for name in sf.keys():
                p = params.get(name)
                if p is None:
                    unexpected.append(name)
                    continue
                t = sf.get_tensor(name)
                if tuple(t.shape) != tuple(p.shape):
                    raise ValueError(f"{name}: checkpoint shape {tuple(t.shape)} != model {tuple(p.shape)}")
                p.copy_(t.to(device=p.device, dtype=p.dtype))
                loaded.add(name)
    missing = [n for n in params if n not in loaded]
    if "lm_head.weight" in missing and "model.embed_tokens.weight" in loaded:
        params["lm_head.weight"].copy_(params["model.embed_tokens.weight"])
        missing.remove("lm_head.weight")
    if strict and missing:
        raise KeyError(f"checkpoint lacks {len(missing)} parameters, e.g. {missing[:4]}")
    return {"missing": missing, "unexpected": unexpected}


def load_model(path: Union[str, Path], device, dtype=torch.bfloat16,
               config: Optional[BlockDiffusionConfig] = None) -> BlockDiffusionLM:
    """Build the model from ``path``/config.json (or ``config``) and load its weights."""
    from .model import build_model

    path = Path(path)
    cfg = config or config_from_json(path / "config.json" if path.is_dir() else path.parent / "config.json")
    model = build_model(cfg, device, dtype)
    load_safetensors(model, path)
    return model


__all__ = ["config_from_json", "load_safetensors", "load_model"]
