"""Draft-model configuration: the schema of the reference's ``DFlashConfig``.

Field names, defaults and the two construction paths (class defaults versus
``from_dict`` defaults) follow mirror_sd/dflash.py:34-105 exactly, including the
places where the two disagree (rope_theta 1e6 vs 1e4, mask id 151669 vs 151667,
intermediate 12288 vs 10944, kv heads 8 vs 2), because checkpoints loaded through
``from_dict`` rely on the latter.  ``build_target_layer_ids`` follows
dflash.py:108-119 and ``extract_context_feature`` dflash.py:122-130.

The named workloads at the bottom are the benchmark shapes this library is
measured and tested on (hidden/heads/FFN/block/context/vocab per workload).
"""

from __future__ import annotations

import copy
from dataclasses import dataclass, field, asdict
from typing import List, Optional, Sequence


@dataclass
class DFlashConfig:
    """Mirror of ``DFlashConfig`` (mirror_sd/dflash.py:34-50)."""

    hidden_size: int = 4096
    num_hidden_layers: int = 5
    intermediate_size: int = 12288
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    head_dim: int = 128
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1000000.0
    max_position_embeddings: int = 40960
    vocab_size: int = 151936
    block_size: int = 16
    mask_token_id: int = 151669
    target_layer_ids: List[int] = field(default_factory=lambda: [4, 12, 19, 26, 33])
    num_target_layers: int = 36
    rope_scaling: Optional[dict] = None

    # dflash.py:52-58
    @classmethod
    def qwen3_8b(cls, num_target_layers: int = 36) -> "DFlashConfig":
        cfg = cls(num_target_layers=num_target_layers)
        cfg.target_layer_ids = build_target_layer_ids(num_target_layers, cfg.num_hidden_layers)
        return cfg

    # dflash.py:60-75
    @classmethod
    def qwen3_4b(cls, num_target_layers: int = 36) -> "DFlashConfig":
        cfg = cls(hidden_size=2560, num_hidden_layers=5, intermediate_size=6912,
                  num_attention_heads=20, num_key_value_heads=4, head_dim=128,
                  vocab_size=151936)
        cfg.num_target_layers = num_target_layers
        cfg.target_layer_ids = build_target_layer_ids(num_target_layers, cfg.num_hidden_layers)
        return cfg

    # dflash.py:77-105
    @classmethod
    def from_dict(cls, d: dict) -> "DFlashConfig":
        dcfg = d.get("dflash_config", {})
        num_hidden_layers = d.get("num_hidden_layers", dcfg.get("num_hidden_layers", 5))
        num_target_layers = dcfg.get("num_target_layers", d.get("num_target_layers", 36))
        cfg = cls(
            hidden_size=d.get("hidden_size", 4096),
            num_hidden_layers=num_hidden_layers,
            intermediate_size=d.get("intermediate_size", 10944),
            num_attention_heads=d.get("num_attention_heads", 32),
            num_key_value_heads=d.get("num_key_value_heads", 2),
            head_dim=d.get("head_dim", 128),
            rms_norm_eps=d.get("rms_norm_eps", 1e-6),
            rope_theta=d.get("rope_theta", 10000.0),
            max_position_embeddings=d.get("max_position_embeddings", 4096),
            vocab_size=d.get("vocab_size", 151936),
            block_size=dcfg.get("block_size", d.get("block_size", 16)),
            mask_token_id=dcfg.get("mask_token_id", d.get("mask_token_id", 151667)),
            num_target_layers=num_target_layers,
        )
        if "target_layer_ids" in dcfg:
            cfg.target_layer_ids = list(dcfg["target_layer_ids"])
        else:
            cfg.target_layer_ids = build_target_layer_ids(cfg.num_target_layers,
                                                           cfg.num_hidden_layers)
        if "rope_scaling" in d:
            cfg.rope_scaling = d["rope_scaling"]
        return cfg

    @property
    def num_target_features(self) -> int:
        """Number of tapped target layers concatenated into target_hidden (dflash.py:373-377)."""
        return len(self.target_layer_ids)

    def to_dict(self) -> dict:
        return asdict(self)

    def copy(self) -> "DFlashConfig":
        return copy.deepcopy(self)


def build_target_layer_ids(num_target_layers: int, num_draft_layers: int) -> List[int]:
    """dflash.py:108-119: evenly spaced taps over target layers [1, L-3]."""
    if num_draft_layers == 1:
        return [num_target_layers // 2]
    start = 1
    end = num_target_layers - 3
    span = end - start
    return [int(round(start + (i * span) / (num_draft_layers - 1)))
            for i in range(num_draft_layers)]


def select_context_features(hidden_states: Sequence, layer_ids: Sequence[int]) -> list:
    """The tensors extract_context_feature concatenates (dflash.py:124-129): all of them
    when there is one per layer id, else (every layer output, embedding at index 0)
    layer ``lid`` read at ``lid + 1``."""
    if len(hidden_states) == len(layer_ids):
        return list(hidden_states)
    return [hidden_states[lid + 1] for lid in layer_ids]


def extract_context_feature(hidden_states: Sequence, layer_ids: Sequence[int]):
    """dflash.py:122-130: concatenate tapped layer outputs along the feature axis.

    Works on torch tensors or numpy arrays; GPU tensors are concatenated by the library's
    copy kernel.  ``DFlashDraftModel`` also takes the list itself as ``target_hidden`` and
    then reads the tensors where they lie (no concatenated copy).
    """
    sel = select_context_features(hidden_states, layer_ids)
    first = sel[0]
    if hasattr(first, "detach"):  # torch
        if first.is_cuda:
            from .dflash import concat_features
            return concat_features(sel)
        import torch
        return torch.cat(sel, dim=-1)
    import numpy as np
    return np.concatenate(sel, axis=-1)


# ---------------------------------------------------------------------------
# Named benchmark / test workloads.
# ---------------------------------------------------------------------------

@dataclass
class Workload:
    """One benchmark shape: a draft config plus block/context sizes."""

    name: str
    cfg: DFlashConfig
    block: int
    ctx: int
    description: str = ""
    with_lm_head: bool = True
    n_feat: int = 5
    seq_ctx: tuple = ()   # batched workloads: context rows of each sequence


def _draft_cfg(hidden, heads, kv_heads, ffn, layers, vocab=151936, theta=1e6,
               block=16, mask_id=151669, n_feat=5):
    if mask_id >= vocab:     # a reduced test vocabulary: use its last id as the mask
        mask_id = vocab - 1
    cfg = DFlashConfig(hidden_size=hidden, num_hidden_layers=layers,
                       intermediate_size=ffn, num_attention_heads=heads,
                       num_key_value_heads=kv_heads, head_dim=128, rms_norm_eps=1e-6,
                       rope_theta=theta, vocab_size=vocab, block_size=block,
                       mask_token_id=mask_id)
    # n_feat tapped layers -> fc input is n_feat*hidden.
    cfg.target_layer_ids = build_target_layer_ids(36, n_feat)
    return cfg


def workload(name: str) -> Workload:
    """Return a named workload.

    qwen3_4b_layer  : 1 layer, H2560, 32/8 heads, FFN 9728, block 16, ctx 64 (no lm_head).
    qwen3_8b_draft  : 5 layers, H4096, 32/8, FFN 12288, block 16, ctx 2048, V151936.
    dflash_27b      : 5 layers, H5120, 40/8, FFN 17408, block 32, ctx 4096, V151936.
    dflash_27b_ctxN : dflash_27b at context N (64, 2048, 4096, 16384, 32768).
    llama8b_batch   : 5 layers, H4096, 32/8, FFN 14336, V128256, theta 5e5; 8 sequences x
                      block 32 with contexts U[512, 8192] from seed 1 (mask id V-1).
    """
    if name == "qwen3_4b_layer":
        cfg = _draft_cfg(2560, 32, 8, 9728, 1, block=16)
        return Workload(name, cfg, block=16, ctx=64, with_lm_head=False,
                        description="1 layer, H2560, 32/8 heads, FFN 9728, block 16, ctx 64")
    if name == "qwen3_8b_draft":
        cfg = _draft_cfg(4096, 32, 8, 12288, 5, block=16)
        return Workload(name, cfg, block=16, ctx=2048,
                        description="5 layers, H4096, 32/8 heads, FFN 12288, block 16, ctx 2048, V151936")
    if name == "dflash_27b" or name.startswith("dflash_27b_ctx"):
        ctx = 4096 if name == "dflash_27b" else int(name[len("dflash_27b_ctx"):])
        cfg = _draft_cfg(5120, 40, 8, 17408, 5, block=32)
        return Workload(name, cfg, block=32, ctx=ctx,
                        description=f"5 layers, H5120, 40/8 heads, FFN 17408, block 32, ctx {ctx}, V151936")
    if name == "llama8b_batch":
        # 8 independent sequences x block 32; ragged contexts drawn U[512, 8192] from seed 1
        import numpy as np
        ctxs = tuple(int(c) for c in np.random.default_rng(1).integers(512, 8193, 8))
        cfg = _draft_cfg(4096, 32, 8, 14336, 5, vocab=128256, theta=5e5, block=32)
        return Workload(name, cfg, block=32, ctx=max(ctxs), seq_ctx=ctxs,
                        description="5 layers, H4096, 32/8 heads, FFN 14336, V128256, theta 5e5, "
                                    f"8 sequences x block 32, contexts {list(ctxs)}")
    if name == "tiny":
        cfg = _draft_cfg(256, 4, 2, 512, 2, vocab=1024, block=8)
        return Workload(name, cfg, block=8, ctx=24, description="test shape")
    raise KeyError(name)


ROPE_DEFAULT, ROPE_LINEAR, ROPE_LLAMA3 = 0, 1, 2   # dfl_set_rope_scaling types


def rope_scaling_args(cfg) -> tuple:
    """The RoPE variant of ``cfg.rope_scaling`` as the library's dfl_set_rope_scaling
    arguments (type, factor, low_freq_factor, high_freq_factor,
    original_max_position_embeddings).

    The reference builds its RoPE with mlx_lm's ``initialize_rope(head_dim, base=rope_theta,
    traditional=False, scaling_config=rope_scaling, max_position_embeddings=...)``
    (mirror_sd/dflash.py:254-261; mlx-lm >= 0.23, pyproject.toml:7).  Its rope types:
    "default" (and no scaling) -> plain RoPE; "linear" -> positions scaled by 1 / factor;
    "llama3" -> Llama 3.1 frequency scaling with low_freq_factor 1, high_freq_factor 4 and
    original_max_position_embeddings 8192 when absent.  Other types (yarn, longrope) raise
    NotImplementedError.  The type is read from "type", then "rope_type", as mlx_lm does.
    """
    rs = getattr(cfg, "rope_scaling", None)
    if rs is None:
        return (ROPE_DEFAULT, 1.0, 1.0, 4.0, 8192)
    rope_type = rs.get("type") or rs.get("rope_type", "default")
    if rope_type == "default":
        return (ROPE_DEFAULT, 1.0, 1.0, 4.0, 8192)
    if rope_type == "linear":
        return (ROPE_LINEAR, float(rs["factor"]), 1.0, 4.0, 8192)
    if rope_type == "llama3":
        return (ROPE_LLAMA3, float(rs["factor"]), float(rs.get("low_freq_factor", 1.0)),
                float(rs.get("high_freq_factor", 4.0)),
                int(rs.get("original_max_position_embeddings", 8192)))
    raise NotImplementedError(f"rope_scaling {rs!r}: RoPE types default, linear and llama3 "
                              "are implemented")


def require_supported_rope(cfg) -> None:
    """Raise NotImplementedError for a rope_scaling this library does not implement."""
    rope_scaling_args(cfg)
