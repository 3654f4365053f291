"""Load a DFlash draft checkpoint from a local directory (mirror_sd/loader.py:20-116).

Directory layout, as the reference reads it:

* ``config.json``: parsed by ``DFlashConfig.from_dict`` (loader.py:59-72,
  dflash.py:77-105), after ``config_overrides`` are merged in;
* weights: the shards named by ``model.safetensors.index.json`` (each file once,
  sorted), else ``model.safetensors``, else every ``*.safetensors`` in sorted order
  (loader.py:75-116).  Later files override earlier ones on a repeated name.

Every tensor is first rounded to ``dtype`` (bfloat16 by default, the reference's
``dtype=mx.bfloat16`` cast, loader.py:23, 95-113).  The names are the reference module's
attributes (``layers.{i}.self_attn.q_proj.weight`` ..., ``fc.weight``,
``hidden_norm.weight``, ``norm.weight``; dflash.py:246-252, 325-339, 365-379), loaded
strictly as MLX ``load_weights`` does: a missing or unexpected name is an error
(``sanitize`` is the identity, dflash.py:408-409).  The seven projections of each layer
are then quantised to W8A16 on the GPU with the per-output-row quantiser of
ane_model.py:265-279 (the ANE container format); fc and the norm gains are kept in fp16.

The embedding and lm_head come from the target model (target.py:188-197) and are passed
in; without them the model runs ``__call__`` / ``read_output`` but not ``draft``.

Differences from the reference, all loud: there is no hub download (the path must be a
local directory); ``quantize`` only accepts None or 8 because the projections always run
W8A16 (MLX's group-wise ``nn.quantize`` is a different format); RoPE scaling other than
none / "default" is rejected, since the kernels apply plain neox RoPE.
"""

from __future__ import annotations

import json
from pathlib import Path
from typing import Dict, Iterable, List, Optional, Tuple

from .config import DFlashConfig, require_supported_rope
from .synth import PROJ_NAMES, proj_key

__all__ = ["load_dflash_model", "load_config", "load_safetensors", "expected_names",
           "check_names", "weight_files"]

_DTYPES = ("bfloat16", "float16", "float32")


def load_config(model_path, overrides: Optional[Dict] = None) -> DFlashConfig:
    """loader.py:59-72: config.json (+ overrides) -> DFlashConfig.from_dict."""
    path = Path(model_path) / "config.json"
    if not path.exists():
        raise FileNotFoundError(f"No config.json found at {path}")
    with open(path) as f:
        d = json.load(f)
    if overrides:
        d.update(overrides)
    cfg = DFlashConfig.from_dict(d)
    require_supported_rope(cfg)
    return cfg


def weight_files(model_path) -> List[Path]:
    """The safetensors files of a checkpoint directory, in the reference's order."""
    p = Path(model_path)
    index = p / "model.safetensors.index.json"
    if index.exists():
        with open(index) as f:
            wm = json.load(f)["weight_map"]
        return [p / name for name in sorted(set(wm.values()))]
    single = p / "model.safetensors"
    if single.exists():
        return [single]
    return sorted(p.glob("*.safetensors"))


def load_safetensors(model_path, dtype: str = "bfloat16", device="cpu") -> Dict[str, "object"]:
    """loader.py:75-116: name -> torch tensor rounded to ``dtype``, on ``device``.

    Files are read tensor by tensor (safetensors ``safe_open``), so host memory holds one
    tensor at a time when ``device`` is a GPU."""
    import torch
    from safetensors import safe_open
    if dtype not in _DTYPES:
        raise ValueError(f"dtype must be one of {_DTYPES}")
    tdt = getattr(torch, dtype)
    files = weight_files(model_path)
    if not files:
        raise FileNotFoundError(f"no safetensors files in {model_path}")
    out: Dict[str, torch.Tensor] = {}
    for fpath in files:
        with safe_open(str(fpath), framework="pt", device="cpu") as f:
            for k in f.keys():
                t = f.get_tensor(k)
                if t.is_floating_point() and t.dtype != tdt:
                    t = t.to(device).to(tdt)
                else:
                    t = t.to(device)
                out[k] = t
    return out


def expected_names(cfg: DFlashConfig) -> List[str]:
    """Parameter names of the reference DFlashDraftModel for ``cfg``."""
    names = []
    for i in range(cfg.num_hidden_layers):
        names += [proj_key(i, p) for p in PROJ_NAMES]
        names += [f"layers.{i}.input_layernorm.weight", f"layers.{i}.post_attention_layernorm.weight",
                  f"layers.{i}.self_attn.q_norm.weight", f"layers.{i}.self_attn.k_norm.weight"]
    names += ["fc.weight", "hidden_norm.weight", "norm.weight"]
    return names


def check_names(cfg: DFlashConfig, names: Iterable[str], strict: bool = True) -> None:
    """Missing names always raise; unexpected names raise when ``strict`` (MLX default)."""
    have = set(names)
    want = expected_names(cfg)
    missing = [n for n in want if n not in have]
    if missing:
        raise ValueError(f"checkpoint is missing {len(missing)} tensors, e.g. {missing[:4]}")
    if strict:
        extra = sorted(have - set(want))
        if extra:
            raise ValueError(f"checkpoint has {len(extra)} unexpected tensors, e.g. {extra[:4]}")


def load_dflash_model(model_path, config_overrides: Optional[Dict] = None,
                      dtype: str = "bfloat16", quantize: Optional[int] = None, *,
                      embed_tokens=None, lm_head=None, max_ctx: int = 8192,
                      max_block: Optional[int] = None, device=None, max_seqs: int = 1,
                      strict: bool = True) -> Tuple["object", DFlashConfig]:
    """loader.py:20-56 for a local directory: returns (DFlashDraftModel, DFlashConfig).

    ``embed_tokens`` / ``lm_head``: the target's [V, H] tensors (any float dtype; stored
    fp16).  ``quantize``: None or 8 (both give the W8A16 projections)."""
    import torch
    from .dflash import DFlashDraftModel
    p = Path(model_path)
    if not p.is_dir():
        raise FileNotFoundError(f"{p} is not a local checkpoint directory (no hub download)")
    if quantize not in (None, 8):
        raise NotImplementedError("the projections run W8A16 only (quantize=None or 8)")
    cfg = load_config(p, config_overrides)
    dev = torch.device(device if device is not None else "cuda")
    weights = load_safetensors(p, dtype, device=dev)
    check_names(cfg, weights.keys(), strict=strict)
    model = DFlashDraftModel(cfg, max_ctx=max_ctx, max_block=max_block, device=dev,
                             max_seqs=max_seqs)
    if embed_tokens is not None:
        weights["embed_tokens.weight"] = embed_tokens
    if lm_head is not None:
        weights["lm_head.weight"] = lm_head
    model.load_weights(weights)
    del weights
    return model, cfg
