"""CPU oracle for the DFlash draft forward -- TEST INFRASTRUCTURE ONLY.

It checks the GPU library and is never part of it: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import
it.  The GPU library never routes through it.

It restates, in numpy, the reference's MLX draft forward and its W8A16 quantiser:

* ``quantize_w8``         ane_model.py:265-279 (symmetric per-output-channel int8)
* ``rms_norm``            nn.RMSNorm / mx.fast.rms_norm as used at dflash.py:251-252,
                          338-339, 378-379; restated in fp32 at
                          scripts/test_qk_isolation.py:69-71
* ``head_rms_norm``       dflash.py:291, 296 (RMSNorm over head_dim per (row, head));
                          scripts/test_qk_isolation.py:74-83
* ``rope_neox``           dflash.py:263-275, 304-305 (mx.fast.rope, traditional=False);
                          scripts/test_qk_isolation.py:86-100; ane/ANE_RULES.md:117-121
* ``sdpa_gqa``            dflash.py:310-317 (mx.repeat over heads + non-causal SDPA)
* ``attention``           Qwen3DFlashAttention.__call__, dflash.py:277-319
* ``mlp``                 Qwen3MLP.__call__, dflash.py:329-330
* ``decoder_layer``       Qwen3DFlashDecoderLayer.__call__, dflash.py:341-362
* ``draft_forward``       DFlashDraftModel.__call__, dflash.py:384-403
* ``OracleKVCache``       DFlashKVCache, dflash.py:139-212
* ``lm_head_argmax``      generate.py:604-606 + target.py:192-197 + dflash.py:133-136
                          (greedy: first index of the maximum, as wrapper.rs:124-134)
* ``soft_anchor``         generate.py:1419-1437 (top-k of the verify logits, fp32 softmax,
                          weighted sum of their embedding rows); ``embed_block`` the block
                          noise embedding of generate.py:1419-1420 with it in row 0

Two arithmetic modes:

* ``fp16=False`` ("ideal"): every value stays in float64; no rounding anywhere.
* ``fp16=True``  ("MLX-like"): values are rounded to fp16 wherever the MLX graph
  materialises an fp16 array (Linear, RMSNorm, RoPE, SDPA, sigmoid, mul, add),
  while each op computes internally in float64.

The W8A16 weight of a projection is ``q * s`` with ``s`` the fp16 scale, taken
exactly (``q`` has 8 significant bits and ``s`` 11, so the product is exact in
fp32 and fp64); ``y = (x @ q.T) * s`` is algebraically identical.  Logits are
never rounded to fp16 before the argmax (ties broken by lowest index).

Summation order: every dot product over the Linear input (``linear_w8``,
``linear_dense``, ``lm_head_logits``) and over the keys (``sdpa_gqa``'s P.V) is one
matmul by default.  Inside ``accumulation_split(n)`` each is summed over n contiguous
ranges of its reduction axis, added in order -- the way a GPU GEMM splits k across
workgroups.  In fp32 this changes only the rounding; the fixtures record the argmax of
such runs so that a row whose argmax depends on the summation order (the oracle itself
cannot decide it) is known.

Parity status of each function is recorded in the tests that pin it
(tests/test_oracle.py): all functions above are pinned by closed forms,
invariants, brute force or library routines; the MLX-internal rounding inside
``mx.fast.*`` remains unpinned beyond the stated tolerances.
"""

from __future__ import annotations

import math
from typing import Dict, List, Optional, Tuple

import numpy as np

F64 = np.float64


# ---------------------------------------------------------------------------
# Summation order of the reduction matmuls
# ---------------------------------------------------------------------------

_SPLIT = [1]


class accumulation_split:
    """Context manager: sum each reduction matmul over n contiguous ranges (see above)."""

    def __init__(self, n: int):
        self.n = int(n)

    def __enter__(self):
        self.prev = _SPLIT[0]
        _SPLIT[0] = self.n
        return self

    def __exit__(self, *exc):
        _SPLIT[0] = self.prev
        return False


_PV16 = [False]


class attention_fp16_p:
    """Context manager: the attention's probabilities go into P.V rounded to fp16, and the
    softmax denominator is the sum of those fp16 values -- the rounding points of a
    flash-attention kernel that feeds fp16 P to its P.V product (p = exp(s - max) unnormalised,
    O = sum fp16(p) v / sum fp16(p)).  MLX's fused SDPA does not state its own rounding
    points, so this is another run whose argmax differences mark rows the oracle cannot
    decide."""

    def __enter__(self):
        self.prev = _PV16[0]
        _PV16[0] = True
        return self

    def __exit__(self, *exc):
        _PV16[0] = self.prev
        return False


def _mm(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """a @ b, the reduction axis (a's last, b's first) summed in _SPLIT[0] ordered ranges."""
    n = _SPLIT[0]
    K = a.shape[-1]
    if n <= 1 or K < n:
        return a @ b
    y = a[..., :K // n] @ b[:K // n]
    for i in range(1, n):
        lo, hi = K * i // n, K * (i + 1) // n
        y = y + a[..., lo:hi] @ b[lo:hi]
    return y


# ---------------------------------------------------------------------------
# Rounding helper
# ---------------------------------------------------------------------------

def _r(x: np.ndarray, fp16: bool, dtype=F64) -> np.ndarray:
    """Round to fp16 (and back to the compute dtype) when in MLX-like mode."""
    if fp16:
        return x.astype(np.float16).astype(dtype)
    return x


# ---------------------------------------------------------------------------
# W8A16 quantiser (ane_model.py:265-279)
# ---------------------------------------------------------------------------

def quantize_w8(w: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """Symmetric per-output-channel int8 quantisation of an [oc, ic] weight.

    Same sequence of fp32 operations as ane_model.py:272-278:
    ``scale = max|w|/127`` per row (an all-zero row's max is replaced by 1.0),
    ``q = clip(round_half_even(w / scale), -127, 127)``, scale stored as fp16.
    Returns (q int8 [oc, ic], scale fp16 [oc]).
    """
    w_np = np.asarray(w, dtype=np.float32)
    max_vals = np.abs(w_np).max(axis=1)
    max_vals = np.where(max_vals == 0, np.float32(1.0), max_vals).astype(np.float32)
    scales = (max_vals / np.float32(127.0)).astype(np.float32)
    q = np.clip(np.round(w_np / scales[:, None]), -127, 127).astype(np.int8)
    return q, scales.astype(np.float16)


def dequantize_w8(q: np.ndarray, s: np.ndarray, dtype=F64) -> np.ndarray:
    return q.astype(dtype) * s.astype(dtype)[:, None]


# ---------------------------------------------------------------------------
# Elementary ops
# ---------------------------------------------------------------------------

def rms_norm(x: np.ndarray, g: np.ndarray, eps: float, fp16: bool, dtype=F64) -> np.ndarray:
    """RMSNorm over the last axis: ``(x * rsqrt(mean(x^2) + eps)) * g``.

    In MLX-like mode the normalised value is rounded to fp16 before the gain is
    applied, and the product is rounded again (two fp16 materialisations inside
    mx.fast.rms_norm's output expression).
    """
    x = x.astype(dtype, copy=False)
    ms = np.mean(x * x, axis=-1, keepdims=True)
    r = 1.0 / np.sqrt(ms + dtype(eps))
    y = _r(x * r, fp16, dtype)
    return _r(y * g.astype(dtype), fp16, dtype)


def head_rms_norm(x: np.ndarray, g: np.ndarray, eps: float, fp16: bool, dtype=F64) -> np.ndarray:
    """Per-(row, head) RMSNorm of x [..., heads, head_dim] with a shared [head_dim] gain."""
    return rms_norm(x, g, eps, fp16, dtype)


def rope_inv_freq(head_dim: int, theta: float, scaling: Optional[dict] = None) -> np.ndarray:
    """inv_freq_j = theta^(-2j/head_dim), j in [0, head_dim/2) (float64), with the rope_scaling
    of the reference's ``initialize_rope(head_dim, base=theta, traditional=False,
    scaling_config=scaling)`` (dflash.py:254-261; mlx-lm >= 0.23, not vendored):

    * "linear": nn.RoPE(scale = 1 / factor), i.e. every frequency divided by factor;
    * "llama3" (mlx_lm Llama3RoPE, the Llama 3.1 scheme): with L0 =
      original_max_position_embeddings (8192), lf = low_freq_factor (1), hf =
      high_freq_factor (4) and wavelength w = 2 pi / inv_freq, frequencies with w > L0 / lf
      are divided by factor, w < L0 / hf are kept, and in between
      inv_freq * ((1 - s) / factor + s) with s = (L0 / w - lf) / (hf - lf).
    """
    j = np.arange(head_dim // 2, dtype=F64)
    inv = 1.0 / (float(theta) ** (2.0 * j / head_dim))
    if scaling is None:
        return inv
    kind = scaling.get("type") or scaling.get("rope_type", "default")
    if kind == "default":
        return inv
    factor = float(scaling["factor"])
    if kind == "linear":
        return inv / factor
    if kind != "llama3":
        raise NotImplementedError(f"rope_scaling type {kind!r}")
    L0 = float(scaling.get("original_max_position_embeddings", 8192))
    lf = float(scaling.get("low_freq_factor", 1.0))
    hf = float(scaling.get("high_freq_factor", 4.0))
    wavelen = 2.0 * np.pi / inv
    s = (L0 / wavelen - lf) / (hf - lf)
    smooth = inv * ((1.0 - s) / factor + s)
    out = np.where(wavelen > L0 / lf, inv / factor, inv)
    mid = (wavelen > L0 / hf) & (wavelen < L0 / lf)
    return np.where(mid, smooth, out)


def rope_neox(x: np.ndarray, positions: np.ndarray, theta: float, fp16: bool,
              dtype=F64, scaling: Optional[dict] = None) -> np.ndarray:
    """Split-half (neox) rotary embedding of x [rows, heads, D] at ``positions`` [rows].

    out[..., :D/2] = x1*cos - x2*sin ; out[..., D/2:] = x2*cos + x1*sin with
    angle = position * inv_freq (float64 angles and cos/sin).
    """
    D = x.shape[-1]
    half = D // 2
    ang = positions.astype(F64)[:, None] * rope_inv_freq(D, theta, scaling)[None, :]
    c = np.cos(ang).astype(dtype)[:, None, :]
    s = np.sin(ang).astype(dtype)[:, None, :]
    x = x.astype(dtype, copy=False)
    x1, x2 = x[..., :half], x[..., half:]
    out = np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)
    return _r(out, fp16, dtype)


def sdpa_gqa(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, fp16: bool,
             dtype=F64) -> np.ndarray:
    """Non-causal grouped-query attention.

    q [NH, Lq, D], k/v [NKV, L, D].  Query head h uses KV head h // (NH // NKV)
    (mx.repeat(k, n_rep, axis=1) at dflash.py:310-313).  Softmax in float64.
    Returns [NH, Lq, D].
    """
    NH, NKV = q.shape[0], k.shape[0]
    rep = NH // NKV
    out = np.empty(q.shape, dtype=dtype)
    for h in range(NH):
        g = h // rep
        s = (q[h].astype(dtype) @ k[g].astype(dtype).T) * dtype(scale)
        s = s - s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        if _PV16[0]:
            p = p.astype(np.float16).astype(dtype)
            out[h] = _mm(p, v[g].astype(dtype)) / p.sum(axis=-1, keepdims=True)
            continue
        p /= p.sum(axis=-1, keepdims=True)
        out[h] = _mm(p, v[g].astype(dtype))
    return _r(out, fp16, dtype)


def linear_w8(x: np.ndarray, qs, fp16: bool, dtype=F64) -> np.ndarray:
    """y = x @ (q*s).T for an int8 weight [oc, ic] with fp16 per-row scales.

    ``qs`` is (q, s) or a pre-dequantised dense [oc, ic] matrix.
    """
    if isinstance(qs, np.ndarray):
        y = _mm(x.astype(dtype, copy=False), qs.T)
    else:
        q, s = qs
        y = _mm(x.astype(dtype, copy=False), q.astype(dtype).T) * s.astype(dtype)[None, :]
    return _r(y, fp16, dtype)


def linear_dense(x: np.ndarray, w: np.ndarray, fp16: bool, dtype=F64) -> np.ndarray:
    y = _mm(x.astype(dtype, copy=False), w.astype(dtype, copy=False).T)
    return _r(y, fp16, dtype)


def sigmoid(x: np.ndarray) -> np.ndarray:
    return 1.0 / (1.0 + np.exp(-x))


# ---------------------------------------------------------------------------
# KV cache (dflash.py:139-212)
# ---------------------------------------------------------------------------

class OracleKVCache:
    """Restatement of ``DFlashKVCache``: append, optional sink+window eviction, trim."""

    def __init__(self, sink_size: int = 0, window_size: int = 0):
        self.keys: Optional[np.ndarray] = None   # [NKV, L, D]
        self.values: Optional[np.ndarray] = None
        self.offset = 0
        self.sink_size = int(sink_size)
        self.window_size = int(window_size)

    def update_and_fetch(self, keys: np.ndarray, values: np.ndarray):
        if self.keys is None:
            self.keys, self.values = keys, values
        else:
            self.keys = np.concatenate([self.keys, keys], axis=1)
            self.values = np.concatenate([self.values, values], axis=1)
        self.offset += keys.shape[1]
        self._apply_window()
        return self.keys, self.values

    def _apply_window(self):
        if self.sink_size <= 0 or self.window_size <= 0 or self.keys is None:
            return
        L = self.keys.shape[1]
        if L <= self.sink_size + self.window_size:
            return
        self.keys = np.concatenate([self.keys[:, :self.sink_size],
                                    self.keys[:, L - self.window_size:]], axis=1)
        self.values = np.concatenate([self.values[:, :self.sink_size],
                                      self.values[:, L - self.window_size:]], axis=1)

    def trim(self, n: int):
        if self.keys is not None and n > 0:
            new_len = max(self.keys.shape[1] - n, 0)
            self.keys = self.keys[:, :new_len]
            self.values = self.values[:, :new_len]
            self.offset -= n


# ---------------------------------------------------------------------------
# Model
# ---------------------------------------------------------------------------

class OracleWeights:
    """Quantised draft weights in reference layout.

    layers[i][proj] = (q int8 [oc, ic], s fp16 [oc]) for proj in q/k/v/o/gate/up/down;
    layers[i]['input_layernorm'|'post_attention_layernorm'|'q_norm'|'k_norm'] = fp16 gains.
    fc [H, nf*H] fp16, hidden_norm/norm [H] fp16, embed/lm_head [V, H] fp16 (optional).
    """

    PROJ = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")

    def __init__(self, cfg, tensors: Dict[str, np.ndarray]):
        self.cfg = cfg
        self.fc = tensors.get("fc.weight")
        self.hidden_norm = tensors["hidden_norm.weight"]
        self.norm = tensors["norm.weight"]
        self.embed = tensors.get("embed_tokens.weight")
        self.lm_head = tensors.get("lm_head.weight")
        self.layers: List[dict] = []
        for i in range(cfg.num_hidden_layers):
            lw = {}
            for p in self.PROJ:
                sub = "mlp" if p in ("gate_proj", "up_proj", "down_proj") else "self_attn"
                lw[p] = quantize_w8(tensors[f"layers.{i}.{sub}.{p}.weight"])
            lw["input_layernorm"] = tensors[f"layers.{i}.input_layernorm.weight"]
            lw["post_attention_layernorm"] = tensors[f"layers.{i}.post_attention_layernorm.weight"]
            lw["q_norm"] = tensors[f"layers.{i}.self_attn.q_norm.weight"]
            lw["k_norm"] = tensors[f"layers.{i}.self_attn.k_norm.weight"]
            self.layers.append(lw)

    def densify(self, dtype=np.float32):
        """Replace every (q, s) by its exact dequantised dense matrix (for fast CPU runs)."""
        for lw in self.layers:
            for p in self.PROJ:
                if not isinstance(lw[p], np.ndarray):
                    lw[p] = dequantize_w8(*lw[p], dtype=dtype)
        return self


def attention(h, ctx, lw, cfg, cache: Optional[OracleKVCache], fp16: bool, dtype=F64):
    """Qwen3DFlashAttention.__call__ (dflash.py:277-319) for one sequence.

    h [q_len, H] (already input-normed), ctx [ctx_len, H] (fused context).
    """
    q_len, C = h.shape[0], ctx.shape[0]
    NH, NKV, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    eps, theta = cfg.rms_norm_eps, cfg.rope_theta
    kv_in = np.concatenate([ctx, h], axis=0)
    q = linear_w8(h, lw["q_proj"], fp16, dtype).reshape(q_len, NH, D)
    q = head_rms_norm(q, lw["q_norm"], eps, fp16, dtype)
    k = linear_w8(kv_in, lw["k_proj"], fp16, dtype).reshape(C + q_len, NKV, D)
    v = linear_w8(kv_in, lw["v_proj"], fp16, dtype).reshape(C + q_len, NKV, D)
    k = head_rms_norm(k, lw["k_norm"], eps, fp16, dtype)
    off = cache.offset if cache is not None else 0
    rs = getattr(cfg, "rope_scaling", None)
    q = rope_neox(q, off + C + np.arange(q_len), theta, fp16, dtype, rs)
    k = rope_neox(k, off + np.arange(C + q_len), theta, fp16, dtype, rs)
    q, k, v = q.transpose(1, 0, 2), k.transpose(1, 0, 2), v.transpose(1, 0, 2)
    if cache is not None:
        k, v = cache.update_and_fetch(k, v)
    o = sdpa_gqa(q, k, v, D ** -0.5, fp16, dtype)          # [NH, q_len, D]
    o = o.transpose(1, 0, 2).reshape(q_len, NH * D)
    return linear_w8(o, lw["o_proj"], fp16, dtype)


def mlp(x, lw, fp16: bool, dtype=F64):
    """Qwen3MLP: down(silu(gate(x)) * up(x)), silu = x * sigmoid(x) (dflash.py:329-330)."""
    g = linear_w8(x, lw["gate_proj"], fp16, dtype)
    u = linear_w8(x, lw["up_proj"], fp16, dtype)
    a = _r(g * _r(sigmoid(g), fp16, dtype), fp16, dtype)
    m = _r(a * u, fp16, dtype)
    return linear_w8(m, lw["down_proj"], fp16, dtype)


def decoder_layer(x, ctx, lw, cfg, cache, fp16: bool, dtype=F64):
    """Pre-norm residual block (dflash.py:341-362)."""
    eps = cfg.rms_norm_eps
    h = rms_norm(x, lw["input_layernorm"], eps, fp16, dtype)
    x = _r(x + attention(h, ctx, lw, cfg, cache, fp16, dtype), fp16, dtype)
    h = rms_norm(x, lw["post_attention_layernorm"], eps, fp16, dtype)
    return _r(x + mlp(h, lw, fp16, dtype), fp16, dtype)


def fuse_context(W: OracleWeights, target_hidden: np.ndarray, fp16: bool, dtype=F64):
    """hidden_norm(fc(target_hidden)) (dflash.py:392)."""
    fc_out = linear_dense(target_hidden, W.fc, fp16, dtype)
    return rms_norm(fc_out, W.hidden_norm, W.cfg.rms_norm_eps, fp16, dtype)


def draft_forward(W: OracleWeights, noise: np.ndarray, target_hidden: np.ndarray,
                  cache: Optional[List[OracleKVCache]] = None, fp16: bool = True,
                  fused_context: bool = False, n_layers: Optional[int] = None,
                  dtype=F64, return_prenorm: bool = False):
    """DFlashDraftModel.__call__ (dflash.py:384-403) for one sequence.

    noise [q_len, H] fp16; target_hidden [C, nf*H] (or [C, H] already fused when
    ``fused_context``).  Returns final-normed hidden [q_len, H] (and the pre-norm
    residual stream when ``return_prenorm``).
    """
    cfg = W.cfg
    ctx = target_hidden.astype(dtype) if fused_context else fuse_context(W, target_hidden, fp16, dtype)
    x = noise.astype(dtype)
    nl = cfg.num_hidden_layers if n_layers is None else n_layers
    for i in range(nl):
        c = cache[i] if cache is not None else None
        x = decoder_layer(x, ctx, W.layers[i], cfg, c, fp16, dtype)
    out = rms_norm(x, W.norm, cfg.rms_norm_eps, fp16, dtype)
    return (out, x) if return_prenorm else out


def embed(W: OracleWeights, ids: np.ndarray) -> np.ndarray:
    """embed_tokens(ids) (generate.py:594-597; target.py:188-189)."""
    return W.embed[np.asarray(ids, dtype=np.int64)]


def soft_anchor(embed_table: np.ndarray, logits: np.ndarray, top_k: int = 8) -> np.ndarray:
    """generate.py:1424-1435: ``top_ids = argsort(-logits)[:k]``; ``w = softmax(fp32 top
    logits)``; anchor = sum_i w_i * embed(top_ids_i) in fp32, cast to the embedding dtype.

    Order: larger logit first, lower index on equal logits (stable sort), NaN after every
    number (mx.argsort's order on ties and NaN is not documented).  The sum runs over the
    selected rows in rank order."""
    lg = np.asarray(logits).astype(np.float32).ravel()
    key = np.where(np.isnan(lg), np.float32(np.inf), -lg)
    order = np.argsort(key, kind="stable")[:top_k]
    order = order[~np.isnan(lg[order])]
    if order.size == 0:
        return np.zeros(embed_table.shape[1], dtype=embed_table.dtype)
    v = lg[order]
    e = np.exp(v - v[0]).astype(np.float32)
    w = (e / e.sum(dtype=np.float32)).astype(np.float32)
    acc = np.zeros(embed_table.shape[1], dtype=np.float32)
    for r, i in enumerate(order):
        acc = acc + w[r] * embed_table[i].astype(np.float32)
    return acc.astype(embed_table.dtype)


def embed_block(embed_table: np.ndarray, ids: np.ndarray, correction_logits=None,
                top_k: int = 8) -> np.ndarray:
    """Block noise embedding: rows embed(ids) (generate.py:1419-1420), row 0 replaced by the
    soft anchor when correction logits are given (generate.py:1422-1437)."""
    out = embed_table[np.asarray(ids, dtype=np.int64)].copy()
    if correction_logits is not None:
        out[0] = soft_anchor(embed_table, correction_logits, top_k)
    return out


def lm_head_logits(h: np.ndarray, w_lm: np.ndarray, dtype=F64, chunk: int = 16384) -> np.ndarray:
    """logits = h @ W_lm.T without fp16 rounding (float64 by default)."""
    h = h.astype(dtype)
    out = np.empty((h.shape[0], w_lm.shape[0]), dtype=dtype)
    for i in range(0, w_lm.shape[0], chunk):
        out[:, i:i + chunk] = _mm(h, w_lm[i:i + chunk].astype(dtype, copy=False).T)
    return out


def argmax_first(logits: np.ndarray) -> np.ndarray:
    """Greedy sample (dflash.py:133-136): index of the first maximum per row."""
    return np.argmax(logits, axis=-1).astype(np.int32)


def lm_head_argmax(h: np.ndarray, w_lm: np.ndarray, dtype=F64):
    logits = lm_head_logits(h, w_lm, dtype)
    return logits, argmax_first(logits)


def draft_block(W: OracleWeights, ids: np.ndarray, target_hidden: np.ndarray,
                cache=None, fp16: bool = True, dtype=F64):
    """One draft block as the serial caller does it (generate.py:594-609).

    ids [B] = [anchor, mask, ...]; returns (final hidden [B, H], logits [B, V],
    argmax ids [B]).  Logits/argmax are returned for all B positions; the caller
    uses positions 1..B-1.
    """
    noise = embed(W, ids)
    h = draft_forward(W, noise, target_hidden, cache=cache, fp16=fp16, dtype=dtype)
    logits, am = lm_head_argmax(h, W.lm_head, dtype)
    if cache is not None:
        for c in cache:
            c.trim(len(ids))
    return h, logits, am
