"""Local safetensors loading into the block-diffusion model (CPU; no GPU, no network)."""
import json

import pytest
import torch
from safetensors.torch import save_file

from fast_v2_amd.e2e import model as em
from fast_v2_amd.e2e import weights as ew


def _tiny_cfg():
    return em.BlockDiffusionConfig(vocab_size=64, hidden_size=32, intermediate_size=48, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2)


def _checkpoint(tmp_path, cfg, tie=False, shards=2):
    src = em.build_model(cfg, "cpu", torch.float32, seed=7)
    sd = {k: v.clone() for k, v in src.state_dict().items() if k != "model.inv_freq"}
    if tie:
        sd.pop("lm_head.weight")
    names = sorted(sd)
    weight_map = {}
    for i in range(shards):
        part = {n: sd[n].contiguous() for n in names[i::shards]}
        fname = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
        save_file(part, str(tmp_path / fname))
        weight_map.update({n: fname for n in part})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
    conf = {k: getattr(cfg, k) for k in ("vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers",
                                         "num_attention_heads", "num_key_value_heads", "rms_norm_eps",
                                         "rope_theta", "bd_size")}
    (tmp_path / "config.json").write_text(json.dumps(conf))
    return src


def test_load_sharded_checkpoint_exactly(tmp_path):
    cfg = _tiny_cfg()
    src = _checkpoint(tmp_path, cfg)
    model = ew.load_model(tmp_path, "cpu", torch.float32)
    assert model.config == cfg
    for (n, a), (_, b) in zip(src.named_parameters(), model.named_parameters()):
        assert torch.equal(a, b), n


def test_tied_lm_head_and_bf16_cast(tmp_path):
    cfg = _tiny_cfg()
    src = _checkpoint(tmp_path, cfg, tie=True, shards=1)
    model = ew.load_model(tmp_path, "cpu", torch.bfloat16)
    assert model.lm_head.weight.dtype == torch.bfloat16
    assert torch.equal(model.lm_head.weight, src.model.embed_tokens.weight.to(torch.bfloat16))
    assert torch.equal(model.model.layers[1].mlp.down_proj.weight, src.model.layers[1].mlp.down_proj.weight.bfloat16())


def test_missing_and_mismatched_tensors_are_reported(tmp_path):
    cfg = _tiny_cfg()
    src = em.build_model(cfg, "cpu", torch.float32)
    save_file({"model.norm.weight": src.model.norm.weight.detach().clone()}, str(tmp_path / "only.safetensors"))
    model = em.build_model(cfg, "cpu", torch.float32)
    with pytest.raises(KeyError):
        ew.load_safetensors(model, tmp_path / "only.safetensors")
    rep = ew.load_safetensors(model, tmp_path / "only.safetensors", strict=False)
    assert "lm_head.weight" in rep["missing"] and not rep["unexpected"]
    save_file({"model.norm.weight": torch.zeros(7)}, str(tmp_path / "bad.safetensors"))
    with pytest.raises(ValueError):
        ew.load_safetensors(model, tmp_path / "bad.safetensors", strict=False)
