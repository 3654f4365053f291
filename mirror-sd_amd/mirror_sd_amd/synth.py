"""Deterministic synthetic weights and inputs for the draft model.

Every tensor gets its own generator, seeded from ``(seed, crc32(name))``, so a
tensor's values do not depend on which other tensors were generated or in what
order.  Two back-ends produce tensors of identical shapes and distributions:

* ``numpy``  - ``numpy.random.default_rng([seed, crc32(name)])`` (PCG64), or
  ``[seed, crc32(name), b]`` for row block b of a tensor above 4 Mi elements.  Portable
  and bit-reproducible (independent of the thread count used to fill it); used for
  every shape that the CPU oracle also runs.
* ``torch``  - ``torch.Generator`` on the target device, seeded with
  ``seed * 2**32 + crc32(name)``.  Used for the full-size benchmark shapes, where
  generating ~2.5 G samples on the host would dominate the run.  Its values differ
  from the numpy back-end (different generator), never its distributions.

Distributions: projection weights fp32 N(0, 0.02) (quantised to W8A16 at load);
fc, embedding and lm_head fp16 N(0, 0.02); RMSNorm gains 1; block/context hidden
and target_hidden fp16 N(0, 1); block ids ``[id0 ~ U[0, V), mask, ..., mask]``.

Tensor names follow the module attributes of the reference draft model
(mirror_sd/dflash.py:246-252, 325-339, 373-379) so that a real checkpoint's
``state_dict`` has the same keys.
"""

from __future__ import annotations

import os
import zlib
from typing import Dict, Iterator, Tuple

import numpy as np

from .config import DFlashConfig

PROJ_NAMES = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


def _crc(name: str) -> int:
    return zlib.crc32(name.encode("utf-8")) & 0xFFFFFFFF


def proj_shapes(cfg: DFlashConfig) -> Dict[str, Tuple[int, int]]:
    """[out, in] of each projection of one layer (dflash.py:246-249, 325-327)."""
    H, D = cfg.hidden_size, cfg.head_dim
    NH, NKV, F = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.intermediate_size
    return {
        "q_proj": (NH * D, H), "k_proj": (NKV * D, H), "v_proj": (NKV * D, H),
        "o_proj": (H, NH * D), "gate_proj": (F, H), "up_proj": (F, H), "down_proj": (H, F),
    }


def proj_key(layer: int, proj: str) -> str:
    sub = "mlp" if proj in ("gate_proj", "up_proj", "down_proj") else "self_attn"
    return f"layers.{layer}.{sub}.{proj}.weight"


def weight_specs(cfg: DFlashConfig, n_feat: int = None, with_vocab: bool = True
                 ) -> Iterator[Tuple[str, Tuple[int, ...], str]]:
    """Yield (name, shape, kind) for every draft tensor.

    kind: 'proj' (fp32 N(0,0.02), quantised later), 'f16' (fp16 N(0,0.02)),
    'ones' (fp16 ones).
    """
    H, D = cfg.hidden_size, cfg.head_dim
    nf = cfg.num_target_features if n_feat is None else n_feat
    yield "fc.weight", (H, nf * H), "f16"
    yield "hidden_norm.weight", (H,), "ones"
    yield "norm.weight", (H,), "ones"
    for i in range(cfg.num_hidden_layers):
        for p, shp in proj_shapes(cfg).items():
            yield proj_key(i, p), shp, "proj"
        yield f"layers.{i}.input_layernorm.weight", (H,), "ones"
        yield f"layers.{i}.post_attention_layernorm.weight", (H,), "ones"
        yield f"layers.{i}.self_attn.q_norm.weight", (D,), "ones"
        yield f"layers.{i}.self_attn.k_norm.weight", (D,), "ones"
    if with_vocab:
        yield "embed_tokens.weight", (cfg.vocab_size, H), "f16"
        yield "lm_head.weight", (cfg.vocab_size, H), "f16"


# Tensors above CHUNK_ELEMS elements are generated in row blocks of about that many
# elements, block b from default_rng([seed, crc32(name), b]), so that large tensors can be
# filled by several threads with a result that does not depend on the thread count.
CHUNK_ELEMS = 1 << 22


def _row_blocks(shape):
    n = int(np.prod(shape))
    if n <= CHUNK_ELEMS or len(shape) < 2:
        return None
    row = int(np.prod(shape[1:]))
    rows = max(1, CHUNK_ELEMS // row)
    return [(r0, min(shape[0], r0 + rows)) for r0 in range(0, shape[0], rows)]


def _fill_normal(out, seed_seq, std):
    rng = np.random.default_rng(seed_seq)
    x = rng.standard_normal(out.shape, dtype=np.float32)
    if std != 1.0:
        x *= np.float32(std)
    out[...] = x


def _normal_jobs(seed: int, name: str, out: np.ndarray, std: float):
    blocks = _row_blocks(out.shape)
    if blocks is None:
        return [(out, [seed, _crc(name)], std)]
    return [(out[r0:r1], [seed, _crc(name), b], std) for b, (r0, r1) in enumerate(blocks)]


def _run_jobs(jobs, threads=None):
    from concurrent.futures import ThreadPoolExecutor
    threads = threads or min(16, os.cpu_count() or 1)
    if threads <= 1 or len(jobs) <= 1:
        for j in jobs:
            _fill_normal(*j)
        return
    with ThreadPoolExecutor(threads) as ex:
        list(ex.map(lambda j: _fill_normal(*j), jobs))


def np_normal(seed: int, name: str, shape, std: float = 1.0, dtype=np.float32) -> np.ndarray:
    out = np.empty(shape, dtype=dtype)
    _run_jobs(_normal_jobs(seed, name, out, std))
    return out


def make_weights_numpy(cfg: DFlashConfig, seed: int = 0, n_feat: int = None,
                       with_vocab: bool = True, with_fc: bool = True) -> Dict[str, np.ndarray]:
    """All draft tensors as numpy arrays (proj fp32, the rest fp16)."""
    out, jobs = {}, []
    for name, shape, kind in weight_specs(cfg, n_feat, with_vocab):
        if name == "fc.weight" and not with_fc:
            continue
        if kind == "ones":
            out[name] = np.ones(shape, dtype=np.float16)
            continue
        out[name] = np.empty(shape, dtype=np.float16 if kind == "f16" else np.float32)
        jobs += _normal_jobs(seed, name, out[name], 0.02)
    _run_jobs(jobs)
    return out


def make_weights_torch(cfg: DFlashConfig, seed: int = 0, device="cuda", n_feat: int = None,
                       with_vocab: bool = True, with_fc: bool = True, only=None):
    """Same tensors as :func:`make_weights_numpy`, generated on ``device`` with torch.

    ``only`` optionally restricts generation to a set of names (to bound memory).
    Yields (name, tensor) pairs so callers can quantise/pack and drop each fp32
    tensor before the next is generated.
    """
    import torch
    for name, shape, kind in weight_specs(cfg, n_feat, with_vocab):
        if name == "fc.weight" and not with_fc:
            continue
        if only is not None and name not in only:
            continue
        if kind == "ones":
            yield name, torch.ones(shape, dtype=torch.float16, device=device)
            continue
        g = torch.Generator(device=device)
        g.manual_seed(seed * (1 << 32) + _crc(name))
        t = torch.randn(shape, generator=g, dtype=torch.float32, device=device)
        t.mul_(0.02)
        yield name, (t.half() if kind == "f16" else t)


def make_inputs_numpy(cfg: DFlashConfig, block: int, ctx: int, seed: int = 0,
                      n_feat: int = None, fused_context: bool = False) -> Dict[str, np.ndarray]:
    """Synthetic inputs for one draft block.

    fused_context=False: ``target_hidden`` [ctx, n_feat*H] fp16 N(0,1) and block ids
    ``[id0, mask * (block-1)]`` with id0 ~ U[0, V).
    fused_context=True : ``context`` [ctx, H] and ``noise`` [block, H], both fp16
    N(0,1) (the single-layer workload, which starts after the fc fusion).
    """
    H = cfg.hidden_size
    nf = cfg.num_target_features if n_feat is None else n_feat
    if fused_context:
        return {
            "noise": np_normal(seed, "input.noise", (block, H), 1.0, np.float16),
            "context": np_normal(seed, "input.context", (ctx, H), 1.0, np.float16),
        }
    rng = np.random.default_rng([seed, _crc("input.ids")])
    ids = np.full((block,), cfg.mask_token_id, dtype=np.int32)
    ids[0] = rng.integers(0, cfg.vocab_size)
    return {
        "target_hidden": np_normal(seed, "input.target_hidden", (ctx, nf * H), 1.0, np.float16),
        "ids": ids,
    }


def make_inputs_torch(cfg: DFlashConfig, block: int, ctx: int, seed: int = 0, device="cuda",
                      n_feat: int = None):
    import torch
    H = cfg.hidden_size
    nf = cfg.num_target_features if n_feat is None else n_feat
    g = torch.Generator(device=device)
    g.manual_seed(seed * (1 << 32) + _crc("input.target_hidden"))
    th = torch.randn((ctx, nf * H), generator=g, dtype=torch.float32, device=device).half()
    rng = np.random.default_rng([seed, _crc("input.ids")])
    ids = np.full((block,), cfg.mask_token_id, dtype=np.int32)
    ids[0] = rng.integers(0, cfg.vocab_size)
    return {"target_hidden": th, "ids": torch.from_numpy(ids).to(device)}


def make_batch_inputs_numpy(cfg: DFlashConfig, block: int, seq_ctx, seed: int = 0,
                            n_feat: int = None):
    """Inputs of a batched draft: per sequence i, ``target_hidden`` [seq_ctx[i], n_feat*H]
    fp16 N(0,1) and block ids ``[id0, mask * (block-1)]`` (tensor names suffixed .s<i>)."""
    H = cfg.hidden_size
    nf = cfg.num_target_features if n_feat is None else n_feat
    out = []
    for i, c in enumerate(seq_ctx):
        rng = np.random.default_rng([seed, _crc(f"input.ids.s{i}")])
        ids = np.full((block,), cfg.mask_token_id, dtype=np.int32)
        ids[0] = rng.integers(0, cfg.vocab_size)
        out.append({"target_hidden": np_normal(seed, f"input.target_hidden.s{i}", (int(c), nf * H),
                                               1.0, np.float16),
                    "ids": ids})
    return out

