"""Local checkpoint loading (mirror_sd/loader.py:20-116): config.json parsing with
overrides, the three weight-file layouts, the dtype cast, strict names.  CPU only;
tests/test_gpu_loader.py loads a checkpoint into the GPU model."""

import json

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from mirror_sd_amd import loader
from mirror_sd_amd.config import DFlashConfig, build_target_layer_ids


def _write_cfg(d, **extra):
    cfg = {"hidden_size": 256, "num_hidden_layers": 2, "intermediate_size": 512,
           "num_attention_heads": 2, "num_key_value_heads": 1, "head_dim": 128,
           "rms_norm_eps": 1e-6, "rope_theta": 1e6, "vocab_size": 1024,
           "dflash_config": {"block_size": 8, "mask_token_id": 1023,
                             "target_layer_ids": [1, 9, 17, 25, 33]}}
    cfg.update(extra)
    (d / "config.json").write_text(json.dumps(cfg))
    return cfg


def test_config_from_json_with_overrides(tmp_path):
    _write_cfg(tmp_path)
    cfg = loader.load_config(tmp_path, {"rope_theta": 5e5})
    assert (cfg.hidden_size, cfg.num_hidden_layers, cfg.vocab_size) == (256, 2, 1024)
    assert (cfg.block_size, cfg.mask_token_id) == (8, 1023)
    assert cfg.target_layer_ids == [1, 9, 17, 25, 33]
    assert cfg.rope_theta == 5e5 and cfg.num_target_features == 5


def test_config_defaults_follow_from_dict(tmp_path):
    """A bare config.json gets from_dict's defaults (dflash.py:77-105), not the class ones."""
    (tmp_path / "config.json").write_text(json.dumps({"num_hidden_layers": 5}))
    cfg = loader.load_config(tmp_path)
    assert cfg.rope_theta == 10000.0 and cfg.mask_token_id == 151667
    assert cfg.intermediate_size == 10944 and cfg.num_key_value_heads == 2
    assert cfg.target_layer_ids == build_target_layer_ids(36, 5) == [1, 9, 17, 25, 33]


def test_config_rope_scaling(tmp_path):
    """llama3 (LLaMA-3.1 checkpoints) and linear scaling load; a type the library does not
    implement is refused at load."""
    _write_cfg(tmp_path, rope_scaling={"rope_type": "yarn", "factor": 4.0})
    with pytest.raises(NotImplementedError):
        loader.load_config(tmp_path)
    _write_cfg(tmp_path, rope_scaling={"rope_type": "llama3", "factor": 8.0})
    assert loader.load_config(tmp_path).rope_scaling["rope_type"] == "llama3"
    _write_cfg(tmp_path, rope_scaling={"rope_type": "default"})
    assert loader.load_config(tmp_path).rope_scaling == {"rope_type": "default"}
    with pytest.raises(FileNotFoundError):
        loader.load_config(tmp_path / "nothing")


def _tensors(seed=0):
    g = torch.Generator().manual_seed(seed)
    return {"a.weight": torch.randn(4, 8, generator=g) * 0.02,
            "b.weight": torch.randn(3, generator=g).half(),
            "c.count": torch.arange(5, dtype=torch.int32)}


def test_weight_file_layouts(tmp_path):
    t = _tensors()
    # sharded with an index: each file once, sorted, whatever the index order
    d1 = tmp_path / "sharded"
    d1.mkdir()
    save_file({"b.weight": t["b.weight"]}, str(d1 / "model-00002-of-00002.safetensors"))
    save_file({"a.weight": t["a.weight"], "c.count": t["c.count"]},
              str(d1 / "model-00001-of-00002.safetensors"))
    save_file({"zzz": torch.zeros(1)}, str(d1 / "stray.safetensors"))   # not in the index
    (d1 / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {
        "b.weight": "model-00002-of-00002.safetensors",
        "a.weight": "model-00001-of-00002.safetensors",
        "c.count": "model-00001-of-00002.safetensors"}}))
    assert [p.name for p in loader.weight_files(d1)] == [
        "model-00001-of-00002.safetensors", "model-00002-of-00002.safetensors"]
    # a single model.safetensors wins over other files
    d2 = tmp_path / "single"
    d2.mkdir()
    save_file(t, str(d2 / "model.safetensors"))
    save_file({"zzz": torch.zeros(1)}, str(d2 / "extra.safetensors"))
    assert [p.name for p in loader.weight_files(d2)] == ["model.safetensors"]
    # otherwise every *.safetensors, sorted
    d3 = tmp_path / "glob"
    d3.mkdir()
    save_file({"b.weight": t["b.weight"]}, str(d3 / "w2.safetensors"))
    save_file({"a.weight": t["a.weight"]}, str(d3 / "w1.safetensors"))
    assert [p.name for p in loader.weight_files(d3)] == ["w1.safetensors", "w2.safetensors"]
    for d in (d1, d2):
        got = loader.load_safetensors(d)
        assert set(got) == set(t)
        assert got["a.weight"].dtype == torch.bfloat16
        assert torch.equal(got["a.weight"], t["a.weight"].to(torch.bfloat16))
        assert torch.equal(got["b.weight"], t["b.weight"].to(torch.bfloat16))
        assert got["c.count"].dtype == torch.int32 and torch.equal(got["c.count"], t["c.count"])
    got = loader.load_safetensors(d3, dtype="float32")
    assert got["b.weight"].dtype == torch.float32
    assert torch.equal(got["b.weight"], t["b.weight"].float())
    with pytest.raises(FileNotFoundError):
        loader.load_safetensors(tmp_path)
    with pytest.raises(ValueError):
        loader.load_safetensors(d1, dtype="int8")


def test_names_are_checked_strictly():
    cfg = DFlashConfig(hidden_size=256, num_hidden_layers=2, intermediate_size=512,
                       num_attention_heads=2, num_key_value_heads=1, vocab_size=1024)
    names = loader.expected_names(cfg)
    assert len(names) == 2 * 11 + 3 and len(set(names)) == len(names)
    assert "layers.1.mlp.down_proj.weight" in names and "layers.0.self_attn.k_norm.weight" in names
    loader.check_names(cfg, names)
    with pytest.raises(ValueError, match="missing"):
        loader.check_names(cfg, names[1:])
    with pytest.raises(ValueError, match="unexpected"):
        loader.check_names(cfg, names + ["layers.0.self_attn.q_proj.bias"])
    loader.check_names(cfg, names + ["layers.0.self_attn.q_proj.bias"], strict=False)


def test_model_loader_rejects_remote_ids_and_other_quantisation(tmp_path):
    with pytest.raises(FileNotFoundError):
        loader.load_dflash_model("z-lab/Qwen3-8B-DFlash-b16")
    _write_cfg(tmp_path)
    with pytest.raises(NotImplementedError):
        loader.load_dflash_model(tmp_path, quantize=4)
