"""DFlash draft model on MI355X: drop-in for mirror_sd/dflash.py's ``DFlashDraftModel``.

The public surface mirrors the reference:

* ``DFlashDraftModel(config)`` with ``.config``, ``.block_size``, ``.mask_token_id``,
  ``.num_draft_layers`` (mutable) and ``__call__(noise_embedding, target_hidden,
  mask=None, cache=None)`` returning the final-normed hidden states
  (dflash.py:365-403);
* ``make_cache()`` returning per-layer ``DFlashKVCache`` handles with ``.offset``,
  ``.keys`` / ``.values`` and ``.trim(n)`` (dflash.py:139-212, 405-406);
* the split API of the ANE draft that ``_spec_generate_parallel`` drives from a worker
  thread: ``prepare_forward`` / ``run_kernels`` / ``read_output`` /
  ``read_draft_tokens`` / ``set_block_size`` / ``max_ctx_len`` / ``_compute_context``
  (ane_model.py:384-430, 538-637);
* the fused entry point ``draft(ids, target_hidden)`` -> per-position logits and
  argmax ids (generate.py:594-606 in one call).

All arithmetic runs in libdflash_hip.so on the GPU.  Tensors are torch CUDA tensors;
batch size 1 per model instance (the reference draft is single-sequence).
"""

from __future__ import annotations

import ctypes
from typing import Dict, List, Optional

from . import _lib
from .config import DFlashConfig, rope_scaling_args
from .synth import PROJ_NAMES, proj_key

__all__ = ["DFlashDraftModel", "DFlashKVCache", "sample"]


def sample(logits, temperature: float = 0.0):
    """dflash.py:133-136 on host-visible logits: greedy argmax below 1e-5, else categorical.
    (The draft's own lm_head samples on the GPU: DFlashDraftModel.set_sampling.)"""
    import torch
    if temperature < 1e-5:
        return torch.argmax(logits, dim=-1)
    probs = torch.softmax(logits.float() / temperature, dim=-1)
    flat = probs.reshape(-1, probs.shape[-1])
    return torch.multinomial(flat, 1).reshape(probs.shape[:-1])


class DFlashKVCache:
    """Per-layer handle onto the model's device-resident KV cache (dflash.py:139-212).

    ``offset`` counts absolute positions, ``trim(n)`` drops the last n rows exactly as
    the reference does; the device cache is reconciled with these handles at the next
    forward call.  ``keys`` / ``values`` are ``[B_, NKV, L, 128]`` (keys after k_norm and
    RoPE, as the reference stores them; B_ = the batch of the last forward, 1 by default),
    in the reference's row order: with a sink + window the device keeps the window as a
    ring, and the rows are gathered in order (sink rows, then the window oldest first).

    ``keys`` / ``values`` are assignable (``c_new.keys = c_old.keys``, generate.py:917-941)
    and ``update_and_fetch(keys, values)`` appends rows as dflash.py:168-177 does: such a
    handle then holds its rows as its own tensors until the next forward writes every
    layer's rows back into the device cache (dfl_cache_assign).
    """

    def __init__(self, model: "DFlashDraftModel", layer: int, generation: int,
                 sink_size: int = 0, window_size: int = 0):
        self._model = model
        self.layer = layer
        self._gen = generation
        self.sink_size = int(sink_size)
        self.window_size = int(window_size)
        self.offset = 0
        self._len = 0
        self._has_keys = False
        self._k = None   # rows held by the handle (assigned / appended), [B_, NKV, L, D]
        self._v = None

    def trim(self, n: int):
        if self._has_keys and n > 0:
            self._len = max(self._len - n, 0)
            self.offset -= n
            if self._k is not None:
                self._k = self._k[:, :, :self._len]
                self._v = self._v[:, :, :self._len] if self._v is not None else None

    def _appended(self, n: int):
        """Book n appended rows: a sink + window cache holds at most sink + window
        (_apply_window, dflash.py:179-193)."""
        self._len += n
        self.offset += n
        if self.sink_size > 0 and self.window_size > 0:
            self._len = min(self._len, self.sink_size + self.window_size)
        self._has_keys = True

    def _device(self, which: int):
        """The device cache's rows of this layer for every sequence of the last forward
        (the device first takes the length the handles book: a forward leaves its block
        rows uncommitted until the next call, the reference's cache holds them until trim)."""
        import torch
        m = self._model
        if not m._rows_dirty and m._handles:
            m._sync_cache(m._handles, n_seq=m._batch)
        out = []
        for seq in range(m._batch):
            m.select_seq(seq)
            try:
                rows = m._cache_rows()[:self._len]
                k, vt = m._make_cache_views()[self.layer] if seq else m._cache_tensors[self.layer]
                out.append(k[:, rows] if which == 0 else vt[:, :, rows].transpose(1, 2))
            finally:
                m.select_seq(0)
        return torch.stack(out, 0)

    @property
    def keys(self):
        if not self._has_keys:
            return None
        return self._k if self._k is not None else self._device(0)

    @property
    def values(self):
        if not self._has_keys:
            return None
        return self._v if self._v is not None else self._device(1)

    def _hold(self):
        """Take this layer's current rows as the handle's own tensors (all live handles of
        the model do the same, so that no handle reads rows another one rewrote)."""
        self._model._hold_rows()

    @keys.setter
    def keys(self, value):
        self._hold()
        self._k = None if value is None else self._model._as_rows(value)
        self._settle()

    @values.setter
    def values(self, value):
        self._hold()
        self._v = None if value is None else self._model._as_rows(value)
        self._settle()

    def _settle(self):
        self._model._rows_dirty = True
        if self._k is None:
            self._len, self._has_keys, self._v = 0, False, None
        else:
            self._len, self._has_keys = int(self._k.shape[2]), True

    def update_and_fetch(self, keys, values):
        """dflash.py:168-177: append [B_, NKV, n, D] keys / values (post-RoPE), advance the
        offset by n, keep sink + window rows when windowed; returns the cached rows."""
        import torch
        self._hold()
        k, v = self._model._as_rows(keys), self._model._as_rows(values)
        if self._k is not None and self._has_keys:
            k = torch.cat([self._k, k], dim=2)
            v = torch.cat([self._v, v], dim=2)
        self.offset += int(keys.shape[2])
        L, S, Wn = k.shape[2], self.sink_size, self.window_size
        if S > 0 and Wn > 0 and L > S + Wn:   # _apply_window, dflash.py:179-193
            k = torch.cat([k[:, :, :S], k[:, :, L - Wn:]], dim=2)
            v = torch.cat([v[:, :, :S], v[:, :, L - Wn:]], dim=2)
        self._k, self._v = k, v
        self._settle()
        return self._k, self._v

    def state(self):
        if not self._has_keys:
            return []
        return [self.keys, self.values]


class DFlashDraftModel:
    """MI355X draft model behind the reference ``DFlashDraftModel`` interface."""

    def __init__(self, config: DFlashConfig, max_ctx: int = 8192, max_block: Optional[int] = None,
                 device=None, n_target_feat: Optional[int] = None, max_seqs: int = 1):
        import torch
        rope = rope_scaling_args(config)   # raises for a RoPE variant not implemented
        self.config = config
        self.block_size = config.block_size
        self.mask_token_id = config.mask_token_id
        self.num_draft_layers = config.num_hidden_layers
        self.device = torch.device(device if device is not None else "cuda")
        self.max_ctx_len = int(max_ctx)
        self.max_block = int(max_block if max_block is not None else max(config.block_size, 32))
        self.n_feat = config.num_target_features if n_target_feat is None else int(n_target_feat)
        self._L = _lib.load()
        cfg = _lib.DflConfig(
            hidden=config.hidden_size, n_heads=config.num_attention_heads,
            n_kv_heads=config.num_key_value_heads, head_dim=config.head_dim,
            intermediate=config.intermediate_size, n_layers=config.num_hidden_layers,
            n_target_feat=self.n_feat, vocab=config.vocab_size, max_block=self.max_block,
            max_ctx=self.max_ctx_len, rms_eps=config.rms_norm_eps,
            rope_theta=float(config.rope_theta), max_seqs=int(max_seqs))
        self.max_seqs = max(1, int(max_seqs))
        h = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            _lib.check(self._L.dfl_create(ctypes.byref(cfg), ctypes.byref(h)), "dfl_create")
        self._ctx = h
        if rope[0] != 0:
            _lib.check(self._L.dfl_set_rope_scaling(self._ctx, *rope), "dfl_set_rope_scaling")
        self._keep: Dict[str, object] = {}   # caller-owned buffers the library points at
        self._batch = 1                      # sequences of the last forward (cache handles)
        self._handles: List["DFlashKVCache"] = []   # handles of the live cache
        self._rows_dirty = False             # handles hold rows not yet in the device cache
        self._gen = 0
        self._cache_tensors = self._make_cache_views()
        self._layers_loaded = [False] * config.num_hidden_layers
        self._has_fc = False
        self._has_head = False
        self._has_lm = False
        self._has_embed = False
        # split-API state
        self._prepared = None
        self._out_hidden = None
        self._out_ids = None
        self._split_bufs = None
        self._draft_stream = None
        self._done = None

    # ------------------------------------------------------------------ lifecycle
    def close(self):
        if getattr(self, "_ctx", None):
            self._L.dfl_destroy(self._ctx)
            self._ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _stream(self):
        return _lib.stream_handle()

    def _make_cache_views(self):
        import torch
        views = []
        for layer in range(self.config.num_hidden_layers):
            k_ptr, vt_ptr = ctypes.c_void_p(), ctypes.c_void_p()
            cap = ctypes.c_int32()
            _lib.check(self._L.dfl_cache_kv(self._ctx, layer, ctypes.byref(k_ptr),
                                            ctypes.byref(vt_ptr), ctypes.byref(cap)),
                       "dfl_cache_kv")
            nkv, c = self.config.num_key_value_heads, cap.value
            views.append((_wrap_device(k_ptr.value, (nkv, c, 128), self.device),
                          _wrap_device(vt_ptr.value, (nkv, 128, c), self.device)))
        return views

    # ------------------------------------------------------------------ weights
    def load_weights(self, tensors: Dict[str, "torch.Tensor"], quantized: Optional[Dict] = None):
        """Load draft weights named as the reference module attributes.

        Projection weights (``layers.{i}.self_attn.q_proj.weight`` ...) are quantised
        on the GPU with the W8A16 quantiser of ane_model.py:265-279 unless
        ``quantized[name] = (q int8 [oc, ic], scale fp16 [oc])`` is supplied.
        ``fc.weight`` / ``hidden_norm.weight`` / ``norm.weight`` and norm gains are
        fp16; ``embed_tokens.weight`` / ``lm_head.weight`` are optional fp16 [V, H].
        """
        import torch
        dev = self.device
        st = self._stream()
        quantized = quantized or {}
        for i in range(self.config.num_hidden_layers):
            qs, ss = [], []
            for p in PROJ_NAMES:
                key = proj_key(i, p)
                if key in quantized:
                    q, s = quantized[key]
                    q = q.to(dev, torch.int8).contiguous()
                    s = s.to(dev, torch.float16).contiguous()
                else:
                    q, s = self.quantize_w8(tensors[key])
                qs.append(q)
                ss.append(s)
            norms = [tensors[f"layers.{i}.input_layernorm.weight"],
                     tensors[f"layers.{i}.post_attention_layernorm.weight"],
                     tensors[f"layers.{i}.self_attn.q_norm.weight"],
                     tensors[f"layers.{i}.self_attn.k_norm.weight"]]
            norms = [n.to(dev, torch.float16).contiguous() for n in norms]
            self.load_layer_q8(i, qs, ss, *norms)
            del qs, ss
        if "fc.weight" in tensors and self.n_feat > 0:
            self.load_fc(tensors["fc.weight"], tensors["hidden_norm.weight"])
        self.load_head(tensors["norm.weight"], tensors.get("embed_tokens.weight"),
                       tensors.get("lm_head.weight"))
        torch.cuda.current_stream().synchronize()

    def quantize_w8(self, w):
        """W8A16 quantiser on the GPU: returns (q int8 [oc, ic], scale fp16 [oc])."""
        import torch
        w32 = w.to(self.device, torch.float32).contiguous()
        oc, ic = w32.shape
        q = torch.empty((oc, ic), dtype=torch.int8, device=self.device)
        s = torch.empty((oc,), dtype=torch.float16, device=self.device)
        _lib.check(self._L.dfl_quantize_w8(w32.data_ptr(), oc, ic, q.data_ptr(), s.data_ptr(),
                                           self._stream()), "dfl_quantize_w8")
        return q, s

    def load_layer_q8(self, layer, qs, ss, in_norm, post_norm, q_norm, k_norm):
        """Load one layer from W8A16 tensors in the order q,k,v,o,gate,up,down
        (the Q8LayerWeights order, wrapper.rs:363-428)."""
        shapes = self._proj_shapes()
        for (name, shp), q, s in zip(shapes, qs, ss):
            if tuple(q.shape) != shp or tuple(s.shape) != (shp[0],):
                raise ValueError(f"layer {layer} {name}: expected int8 {shp} + fp16 [{shp[0]}], "
                                 f"got {tuple(q.shape)} / {tuple(s.shape)}")
        H, D = self.config.hidden_size, self.config.head_dim
        for n, exp in zip((in_norm, post_norm, q_norm, k_norm), (H, H, D, D)):
            if n.numel() != exp:
                raise ValueError(f"layer {layer}: norm gain of {n.numel()} elements, expected {exp}")
        qa = _lib.PtrArray7(*[q.data_ptr() for q in qs])
        sa = _lib.PtrArray7(*[s.data_ptr() for s in ss])
        _lib.check(self._L.dfl_load_layer_w8(self._ctx, layer, qa, sa, in_norm.data_ptr(),
                                             post_norm.data_ptr(), q_norm.data_ptr(),
                                             k_norm.data_ptr(), self._stream()),
                   "dfl_load_layer_w8")
        # the pack kernels read the inputs asynchronously: keep them alive until done
        import torch
        torch.cuda.current_stream().synchronize()
        self._layers_loaded[layer] = True

    def load_fc(self, fc_weight, hidden_norm):
        import torch
        H = self.config.hidden_size
        w = fc_weight.to(self.device, torch.float16).contiguous()
        g = hidden_norm.to(self.device, torch.float16).contiguous()
        if tuple(w.shape) != (H, self.n_feat * H):
            raise ValueError(f"fc.weight: expected {(H, self.n_feat * H)}, got {tuple(w.shape)}")
        _lib.check(self._L.dfl_load_fc(self._ctx, w.data_ptr(), g.data_ptr(), self._stream()),
                   "dfl_load_fc")
        torch.cuda.current_stream().synchronize()
        self._has_fc = True

    def load_head(self, final_norm, embed=None, lm_head=None):
        """Final norm gain, the target's embedding (kept by reference) and lm_head
        (target.py:188-197)."""
        import torch
        H, V = self.config.hidden_size, self.config.vocab_size
        g = final_norm.to(self.device, torch.float16).contiguous()
        e = None
        if embed is not None:
            e = embed.to(self.device, torch.float16).contiguous()
            if tuple(e.shape) != (V, H):
                raise ValueError(f"embed_tokens: expected {(V, H)}, got {tuple(e.shape)}")
            self._keep["embed"] = e
        lm = None
        if lm_head is not None:
            lm = lm_head.to(self.device, torch.float16).contiguous()
            if tuple(lm.shape) != (V, H):
                raise ValueError(f"lm_head: expected {(V, H)}, got {tuple(lm.shape)}")
        _lib.check(self._L.dfl_load_head(self._ctx, g.data_ptr(), _lib.ptr(e), _lib.ptr(lm),
                                         self._stream()), "dfl_load_head")
        torch.cuda.current_stream().synchronize()
        self._has_head = True
        self._has_embed = e is not None
        self._has_lm = lm is not None

    def _proj_shapes(self):
        from .synth import proj_shapes
        shp = proj_shapes(self.config)
        return [(p, shp[p]) for p in PROJ_NAMES]

    # ------------------------------------------------------------------ cache
    def make_cache(self, sink_size: int = 64, window_size: int = 1024) -> List[DFlashKVCache]:
        """dflash.py:405-406.  One live cache per model: a new cache resets the device
        cache and invalidates older handles.  With sink_size and window_size both set,
        the device cache keeps the first sink_size rows and the newest window_size rows
        (dflash.py:179-193)."""
        self._gen += 1
        for seq in range(self.max_seqs):
            self.select_seq(seq)
            try:
                _lib.check(self._L.dfl_cache_set_window(self._ctx, int(sink_size),
                                                        int(window_size)), "dfl_cache_set_window")
            finally:
                self.select_seq(0)
        self._rows_dirty = False
        self._handles = [DFlashKVCache(self, i, self._gen, sink_size, window_size)
                         for i in range(self.num_draft_layers)]
        return list(self._handles)

    def _as_rows(self, t):
        """[B_, NKV, L, D] (or [NKV, L, D]) fp16 rows on this device, from torch or numpy."""
        import numpy as np
        import torch
        if isinstance(t, np.ndarray):
            t = torch.from_numpy(t)
        t = t.to(self.device, torch.float16)
        if t.dim() == 3:
            t = t.unsqueeze(0)
        NKV, D = self.config.num_key_value_heads, self.config.head_dim
        if t.dim() != 4 or t.shape[1] != NKV or t.shape[3] != D:
            raise ValueError(f"cache rows must be [B_, {NKV}, L, {D}], got {tuple(t.shape)}")
        return t.contiguous()

    def _hold_rows(self):
        """Every live handle takes its layer's device rows as its own tensors (once)."""
        for c in self._handles:
            if c._has_keys and c._k is None:
                c._k = c._device(0).contiguous()
                c._v = c._device(1).contiguous()

    def _write_back(self, cache, n_seq: int):
        """Write the rows the handles hold into the device cache (every layer, every
        sequence), then the handles read the device again."""
        for c in cache:
            B_ = c._k.shape[0] if c._k is not None else n_seq
            if c._has_keys and (c._v is None or c._v.shape != c._k.shape):
                raise ValueError(f"layer {c.layer}: keys and values of different shapes")
            if B_ != n_seq:
                raise ValueError(f"layer {c.layer}: rows for {B_} sequences, the forward has {n_seq}")
        st = self._stream()
        for seq in range(n_seq):
            self.select_seq(seq)
            try:
                for c in cache:
                    k = c._k[seq] if c._has_keys else None
                    v = c._v[seq] if c._has_keys else None
                    L = int(k.shape[1]) if k is not None else 0
                    _lib.check(self._L.dfl_cache_assign(self._ctx, c.layer, _lib.ptr(k),
                                                        _lib.ptr(v), L, st), "dfl_cache_assign")
            finally:
                self.select_seq(0)
        self._keep["cache_rows"] = [(c._k, c._v) for c in cache]
        for c in cache:
            c._k = c._v = None
        self._rows_dirty = False

    def _cache_rows(self):
        """Cache rows of the cached rows in the reference's order (a device index tensor)."""
        import torch
        n = ctypes.c_int32()
        _lib.check(self._L.dfl_cache_rows(self._ctx, None, 0, ctypes.byref(n)), "dfl_cache_rows")
        buf = (ctypes.c_int32 * max(1, n.value))()
        _lib.check(self._L.dfl_cache_rows(self._ctx, buf, n.value, ctypes.byref(n)),
                   "dfl_cache_rows")
        return torch.tensor(list(buf)[:n.value], dtype=torch.long, device=self.device)

    def _device_state(self):
        n = ctypes.c_int32()
        off = ctypes.c_int64()
        _lib.check(self._L.dfl_cache_state(self._ctx, ctypes.byref(n), ctypes.byref(off)),
                   "dfl_cache_state")
        return n.value, off.value

    def _sync_cache(self, cache: List[DFlashKVCache], check_only: bool = False, n_seq: int = 1):
        """Bring the device cache (sequences 0 .. n_seq-1, in lockstep) to the state the
        per-layer handles describe."""
        if any(c._gen != self._gen or c._model is not self for c in cache):
            raise ValueError("stale cache: create caches with this model's make_cache()")
        lens = {c._len for c in cache}
        offs = {c.offset for c in cache}
        if len(lens) != 1 or len(offs) != 1:
            raise ValueError("per-layer caches diverged (different length/offset per layer)")
        want_len, want_off = lens.pop(), offs.pop()
        if check_only:
            return
        if self._rows_dirty:
            self._write_back(cache, n_seq)
        for seq in range(n_seq):
            if seq:
                self.select_seq(seq)
            try:
                dev_len, dev_off = self._device_state()
                if want_len > dev_len:
                    _lib.check(self._L.dfl_cache_commit(self._ctx, want_len - dev_len),
                               "dfl_cache_commit")
                elif want_len < dev_len:
                    _lib.check(self._L.dfl_cache_trim(self._ctx, dev_len - want_len),
                               "dfl_cache_trim")
                _lib.check(self._L.dfl_cache_set_offset(self._ctx, want_off),
                           "dfl_cache_set_offset")
            finally:
                if seq:
                    self.select_seq(0)

    # ------------------------------------------------------------------ forward
    def _apply_num_layers(self):
        n = int(self.num_draft_layers)
        _lib.check(self._L.dfl_set_num_layers(self._ctx, n), "dfl_set_num_layers")

    def ingest_features(self, hidden_states, layer_ids=None):
        """Ingest context rows straight from the target's tapped layer outputs
        (target.py:258-278), in the selection of extract_context_feature
        (dflash.py:122-130) for ``layer_ids`` (default: the config's)."""
        from .config import select_context_features
        ids = self.config.target_layer_ids if layer_ids is None else layer_ids
        feats = select_context_features(hidden_states, ids)
        if len(feats) != self.n_feat:
            raise ValueError(f"{len(feats)} feature tensors, the fc expects {self.n_feat}")
        arr, n, ld, C, keep = _feature_ptrs(feats, self.config.hidden_size, self.device)
        if C:
            _lib.check(self._L.dfl_ingest_features(self._ctx, arr, n, ld, C, self._stream()),
                       "dfl_ingest_features")
        self._keep["ingest_src"] = keep
        return C

    def _ingest(self, target_hidden, fused: bool = False):
        import torch
        if isinstance(target_hidden, (list, tuple)):
            return self.ingest_features(target_hidden)
        th = target_hidden
        if th.dim() == 3:
            if th.shape[0] != 1:
                raise ValueError("batch size must be 1")
            th = th[0]
        th = th.to(self.device, torch.float16).contiguous()
        C = th.shape[0]
        if C == 0:
            return 0
        if fused:
            if th.shape[1] != self.config.hidden_size:
                raise ValueError(f"fused context must be [C, {self.config.hidden_size}]")
            _lib.check(self._L.dfl_ingest_fused(self._ctx, th.data_ptr(), C, self._stream()),
                       "dfl_ingest_fused")
        else:
            if th.shape[1] != self.n_feat * self.config.hidden_size:
                raise ValueError(f"target_hidden must be [C, {self.n_feat * self.config.hidden_size}],"
                                 f" got {tuple(th.shape)}")
            _lib.check(self._L.dfl_ingest_context(self._ctx, th.data_ptr(), C, self._stream()),
                       "dfl_ingest_context")
        self._keep["ingest_src"] = th   # keep alive until the stream passes it
        return C

    def _draft(self, noise=None, ids=None, want_hidden=True, want_prenorm=False,
               want_logits=False, want_ids=False):
        import torch
        H, V = self.config.hidden_size, self.config.vocab_size
        if noise is not None:
            if noise.dim() == 3:
                if noise.shape[0] != 1:
                    raise ValueError("batch size must be 1")
                noise = noise[0]
            noise = noise.to(self.device, torch.float16).contiguous()
            B = noise.shape[0]
            if noise.shape[1] != H:
                raise ValueError(f"noise_embedding must be [B, {H}]")
        else:
            ids = _check_ids(ids, V).to(self.device).contiguous()
            B = ids.numel()
        if not all(self._layers_loaded[:self.num_draft_layers]) or not self._has_head:
            raise RuntimeError("weights not loaded")
        out_h = torch.empty((B, H), dtype=torch.float16, device=self.device) if want_hidden else None
        out_p = torch.empty((B, H), dtype=torch.float16, device=self.device) if want_prenorm else None
        out_l = torch.empty((B, V), dtype=torch.float32, device=self.device) if want_logits else None
        out_i = torch.empty((B,), dtype=torch.int32, device=self.device) if want_ids else None
        _lib.check(self._L.dfl_draft_block(
            self._ctx, _lib.ptr(noise), _lib.ptr(ids), B, _lib.ptr(out_h), _lib.ptr(out_p),
            _lib.ptr(out_l), _lib.ptr(out_i), self._stream()), "dfl_draft_block")
        self._keep["draft_src"] = (noise, ids)
        return out_h, out_p, out_l, out_i

    def __call__(self, noise_embedding, target_hidden, mask=None, cache=None, **kwargs):
        """dflash.py:384-403.  noise_embedding [B_, q, H], target_hidden [B_, C, nf*H] (or,
        for B_ = 1, the list of the nf tapped layer outputs [1, C, H], read without
        concatenating); returns final-normed hidden [B_, q, H] (fp16).  With ``cache`` the
        context rows are appended to the cache and the block rows are left in it (offset
        += C + q) until the caller's ``trim(q)``, exactly as update_and_fetch + trim
        behave.  B_ > 1 runs sequences 0 .. B_-1 of the model (max_seqs >= B_) in lockstep,
        their projections stacked in one pass (dfl_draft_batch)."""
        if mask is not None:
            raise ValueError("DFlash drafting is non-causal; mask must be None (dflash.py:215-233)")
        self._apply_num_layers()
        q = noise_embedding.shape[-2]
        B_ = noise_embedding.shape[0] if noise_embedding.dim() == 3 else 1
        if isinstance(target_hidden, (list, tuple)):
            if B_ != 1:
                raise ValueError("a list of tapped layer outputs is a batch of one")
        elif (target_hidden.shape[0] if target_hidden.dim() == 3 else 1) != B_:
            raise ValueError("noise_embedding and target_hidden differ in batch size")
        if B_ > self.max_seqs:
            raise ValueError(f"batch of {B_} sequences, the model was created with "
                             f"max_seqs={self.max_seqs}")
        if cache is not None:
            cache = list(cache)[:self.num_draft_layers]
            self._sync_cache(cache, n_seq=B_)
        self._batch = B_
        C = 0
        for b in range(B_):
            if b:
                self.select_seq(b)
            try:
                if cache is None:
                    _lib.check(self._L.dfl_cache_reset(self._ctx), "dfl_cache_reset")
                th = target_hidden if B_ == 1 else target_hidden[b]
                C = self._ingest(th)
            finally:
                if b:
                    self.select_seq(0)
        if cache is None:
            self._gen += 1
        if B_ == 1:
            out_h, _, _, _ = self._draft(noise=noise_embedding)
            out_h = out_h.unsqueeze(0)
        else:
            out_h = self._draft_seqs(noise_embedding)
        if cache is None:
            for b in range(B_):
                self.select_seq(b)
                _lib.check(self._L.dfl_cache_reset(self._ctx), "dfl_cache_reset")
            self.select_seq(0)
            self._batch = 1
            return out_h
        for c in cache:       # context + block rows, as update_and_fetch leaves them
            c._appended(C + q)
        return out_h

    def _draft_seqs(self, noise):
        """Final-normed hidden [n_seq, B, H] of one block per sequence (dfl_draft_batch)."""
        import torch
        H = self.config.hidden_size
        noise = noise.to(self.device, torch.float16).contiguous()
        n_seq, B = noise.shape[0], noise.shape[1]
        if noise.shape[2] != H:
            raise ValueError(f"noise_embedding must be [B_, q, {H}]")
        if not all(self._layers_loaded[:self.num_draft_layers]) or not self._has_head:
            raise RuntimeError("weights not loaded")
        out_h = torch.empty((n_seq * B, H), dtype=torch.float16, device=self.device)
        _lib.check(self._L.dfl_draft_batch(self._ctx, n_seq, noise.data_ptr(), None, B,
                                           out_h.data_ptr(), None, None, None, self._stream()),
                   "dfl_draft_batch")
        self._keep["draft_src"] = (noise, None)
        return out_h.reshape(n_seq, B, H)

    def set_sampling(self, temperature: float = 0.0, seed: Optional[int] = None):
        """Draft ids of later calls (draft, draft_batch, run_kernels) are samples from
        softmax(logits / temperature) -- sample(), dflash.py:133-136 -- drawn on the GPU by
        the Gumbel-max rule in the lm_head; greedy (argmax) below 1e-5.  ``seed`` fixes the
        noise (None: a fresh random seed); successive calls draw fresh noise."""
        import random
        if seed is None:
            seed = random.getrandbits(64)
        _lib.check(self._L.dfl_set_sampling(self._ctx, float(temperature), int(seed) & (2**64 - 1)),
                   "dfl_set_sampling")

    def draft(self, ids, target_hidden=None, cache=None, return_logits=False,
              return_hidden=False, fused_context=False, temperature: Optional[float] = None,
              seed: Optional[int] = None):
        """Fused entry point: block token ids [B] (+ new target_hidden rows) in,
        per-position draft ids [B] (and fp32 logits [B, V]) out.

        Equivalent to the serial caller's embed -> draft -> lm_head -> sample ->
        trim sequence (generate.py:594-609) for all B positions; position 0 (the
        anchor) is included, callers use 1..B-1.  The ids are the argmax, or with
        ``temperature`` (set_sampling) samples at that temperature.
        """
        if temperature is not None:
            self.set_sampling(temperature, seed)
        self._apply_num_layers()
        if cache is None:
            _lib.check(self._L.dfl_cache_reset(self._ctx), "dfl_cache_reset")
            self._gen += 1
        else:
            cache = list(cache)[:self.num_draft_layers]
            self._sync_cache(cache)
        if target_hidden is not None:
            C = self._ingest(target_hidden, fused=fused_context)
            if cache is not None:
                for c in cache:
                    c._appended(C)
        out_h, _, out_l, out_i = self._draft(ids=ids, want_hidden=return_hidden,
                                             want_logits=return_logits, want_ids=True)
        res = [out_i]
        if return_logits:
            res.append(out_l)
        if return_hidden:
            res.append(out_h)
        return res[0] if len(res) == 1 else tuple(res)

    # ------------------------------------------------------------------ batched drafting
    def select_seq(self, seq: int):
        """Address sequence ``seq`` with the single-sequence calls (ingest, draft, cache)."""
        _lib.check(self._L.dfl_select_seq(self._ctx, int(seq)), "dfl_select_seq")

    def cache_tensors(self, seq: int = 0):
        """Device views (K [NKV, cap, 128], Vt [NKV, 128, cap]) per layer of one sequence."""
        self.select_seq(seq)
        try:
            return self._make_cache_views()
        finally:
            self.select_seq(0)

    def ingest_seq(self, seq: int, target_hidden, fused_context: bool = False, reset: bool = True):
        """Append context rows to sequence ``seq``'s cache (fc fusion + per-layer K/V),
        after clearing it when ``reset``."""
        self._apply_num_layers()
        self.select_seq(seq)
        try:
            if reset:
                _lib.check(self._L.dfl_cache_reset(self._ctx), "dfl_cache_reset")
            self._ingest(target_hidden, fused=fused_context)
        finally:
            self.select_seq(0)

    def draft_batch(self, ids=None, noise=None, return_logits=False, return_hidden=False,
                    temperature: Optional[float] = None, seed: Optional[int] = None):
        """One block for each of sequences 0 .. n_seq-1 at once: ``ids`` [n_seq, B] (or
        ``noise`` [n_seq, B, H]) -> argmax ids [n_seq, B] (+ fp32 logits [n_seq, B, V],
        final-normed hidden [n_seq, B, H]).  Each sequence attends to its own cached
        context plus its block (the block rows stay uncommitted, as after draft()).  With
        ``temperature`` the ids are samples (set_sampling)."""
        import torch
        if temperature is not None:
            self.set_sampling(temperature, seed)
        self._apply_num_layers()
        H, V = self.config.hidden_size, self.config.vocab_size
        if noise is not None:
            noise = noise.to(self.device, torch.float16).contiguous()
            n_seq, B = noise.shape[0], noise.shape[1]
            if noise.dim() != 3 or noise.shape[2] != H:
                raise ValueError(f"noise must be [n_seq, B, {H}]")
            src_n, src_i = noise, None
        else:
            ids = _check_ids(ids, V, flat=False)
            if ids.dim() != 2:
                raise ValueError("ids must be [n_seq, B]")
            n_seq, B = ids.shape
            src_n, src_i = None, ids.to(self.device).contiguous()
        if not all(self._layers_loaded[:self.num_draft_layers]) or not self._has_lm:
            raise RuntimeError("weights (with lm_head) not loaded")
        M = n_seq * B
        out_h = torch.empty((M, H), dtype=torch.float16, device=self.device) if return_hidden else None
        out_l = torch.empty((M, V), dtype=torch.float32, device=self.device) if return_logits else None
        out_i = torch.empty((M,), dtype=torch.int32, device=self.device)
        _lib.check(self._L.dfl_draft_batch(
            self._ctx, n_seq, _lib.ptr(src_n), _lib.ptr(src_i), B, _lib.ptr(out_h), None,
            _lib.ptr(out_l), _lib.ptr(out_i), self._stream()), "dfl_draft_batch")
        self._keep["draft_src"] = (src_n, src_i)
        res = [out_i.reshape(n_seq, B)]
        if return_logits:
            res.append(out_l.reshape(n_seq, B, V))
        if return_hidden:
            res.append(out_h.reshape(n_seq, B, H))
        return res[0] if len(res) == 1 else tuple(res)

    # ------------------------------------------------------------------ profiling
    def profile(self, enable: bool = True, gemm_only: bool = False):
        """Time kernel groups with HIP events (see dfl_profile_enable).  ``gemm_only``
        times just the stream-K GEMM launches by their dispatch timestamps, which leaves
        the stream's timing unchanged."""
        mode = 0 if not enable else (2 if gemm_only else 1)
        _lib.check(self._L.dfl_profile_enable(self._ctx, mode), "dfl_profile_enable")

    def profile_read(self) -> Dict[str, dict]:
        """Per-category {ms, launches, bytes} since the last read (synchronises)."""
        n = 16
        names = ctypes.create_string_buffer(32 * n)
        ms = (ctypes.c_double * n)()
        cnt = (ctypes.c_int64 * n)()
        by = (ctypes.c_int64 * n)()
        nc = ctypes.c_int32()
        _lib.check(self._L.dfl_profile_read(self._ctx, n, names, ms, cnt, by, ctypes.byref(nc)),
                   "dfl_profile_read")
        out = {}
        for i in range(nc.value):
            name = names.raw[32 * i:32 * i + 32].split(b"\0", 1)[0].decode()
            out[name] = {"ms": ms[i], "launches": cnt[i], "bytes": by[i]}
        return out

    # ------------------------------------------------------------------ split API
    @property
    def ane(self):
        """Dispatch marker used by generate.py:401-408 to select the threaded caller."""
        return self

    @property
    def seq_q(self):
        return self.block_size

    def set_block_size(self, new_seq_q: int):
        """ane_model.py:611-630."""
        if new_seq_q < 1 or new_seq_q > self.max_block:
            raise ValueError(f"new_seq_q={new_seq_q} must be in [1, {self.max_block}]")
        self.block_size = int(new_seq_q)
        self.config.block_size = int(new_seq_q)

    def _compute_context(self, target_hidden):
        """Return the raw target_hidden; fc + hidden_norm run inside the ingest kernel."""
        return target_hidden

    # Dispatch probes of the parallel caller (generate.py:1320-1333): no GPU fallback model
    # is needed (the context limit is max_ctx_len rows of device cache), and b_logits is
    # non-None once an lm_head is loaded, which selects the fused read_draft_tokens path.
    gpu_fallback = None

    @property
    def b_logits(self):
        return True if self._has_lm else None

    def embed_block(self, block_ids, correction_logits=None, top_k: int = 8):
        """Noise embedding [1, B, H] fp16 of the block ids (generate.py:594-597), rows of
        the loaded target embedding.  With ``correction_logits`` ([V] verify logits at the
        correction position, fp32/fp16/bf16) row 0 is the soft anchor of
        generate.py:1419-1437: sum_i softmax(top-k logits)_i * embed(i)."""
        import torch
        if not self._has_embed:
            raise RuntimeError("embedding not loaded")
        V_emb = self.config.vocab_size
        ids = _check_ids(block_ids, V_emb)
        if ids.numel() == 0:
            raise ValueError("block_ids is empty")
        ids = ids.to(self.device).contiguous()
        B, H = ids.numel(), self.config.hidden_size
        out = torch.empty((B, H), dtype=torch.float16, device=self.device)
        lg, code, V = None, 0, 0
        if correction_logits is not None:
            codes = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
            lg = correction_logits.reshape(-1).to(self.device)
            if lg.dtype not in codes:
                lg = lg.float()
            lg = lg.contiguous()
            code, V = codes[lg.dtype], lg.numel()
        _lib.check(self._L.dfl_embed_block(self._ctx, ids.data_ptr(), B, _lib.ptr(lg), code, V,
                                           int(top_k), out.data_ptr(), self._stream()),
                   "dfl_embed_block")
        self._keep["embed_src"] = (ids, lg)
        return out.unsqueeze(0)

    def prepare_forward(self, noise_embedding, precomputed_context, cache, target_hidden):
        """ane_model.py:538-562: stage the inputs and output buffers on the calling thread
        (the caller's current stream); run_kernels does the GPU work on the draft's own
        stream, which first waits for everything queued so far on the caller's stream."""
        import torch
        self._apply_num_layers()
        if not all(self._layers_loaded[:self.num_draft_layers]) or not self._has_head:
            raise RuntimeError("weights not loaded")
        rope_offset = 0
        if cache is not None and len(cache) > 0 and cache[0].offset > 0:
            rope_offset = int(cache[0].offset)
        th = precomputed_context if precomputed_context is not None else target_hidden
        ne = noise_embedding
        if th.dim() == 3:
            if th.shape[0] != 1:
                raise ValueError("batch size must be 1")
            th = th[0]
        if ne.dim() == 3:
            if ne.shape[0] != 1:
                raise ValueError("batch size must be 1")
            ne = ne[0]
        H = self.config.hidden_size
        if th.shape[-2] > self.max_ctx_len:
            raise ValueError(f"ctx_len={th.shape[-2]} exceeds max_ctx_len={self.max_ctx_len}")
        if th.shape[-1] != self.n_feat * H:
            raise ValueError(f"target_hidden must be [C, {self.n_feat * H}], got {tuple(th.shape)}")
        if ne.shape[-1] != H or not 1 <= ne.shape[0] <= self.max_block:
            raise ValueError(f"noise_embedding must be [B <= {self.max_block}, {H}]")
        ne = ne.to(self.device, torch.float16).contiguous()
        th = th.to(self.device, torch.float16).contiguous()
        B = ne.shape[0]
        if self._split_bufs is None or self._split_bufs[0].shape[0] != B:
            self._split_bufs = (torch.empty((B, H), dtype=torch.float16, device=self.device),
                                torch.empty((B,), dtype=torch.int32, device=self.device))
        if self._draft_stream is None:
            self._draft_stream = torch.cuda.Stream(device=self.device)   # default priority
            self._done = torch.cuda.Event()
        ds = self._draft_stream
        ds.wait_stream(torch.cuda.current_stream(self.device))
        for t in (ne, th) + self._split_bufs:
            t.record_stream(ds)
        self._prepared = (ne, th, rope_offset)
        self._out_hidden = self._out_ids = None

    def run_kernels(self, wait: bool = True):
        """ane_model.py:564-589 on the draft's own HIP stream.  Only library calls (ctypes
        releases the GIL around each), so a worker thread can run it while the caller's
        stream does the target verify (generate.py:1339-1345, 1469-1477).  The ANE path
        keeps no K/V: the step's target_hidden is re-ingested at RoPE positions from
        cache.offset.  ``wait`` (default, as the ANE call blocks) returns once the draft
        is done; read_output / read_draft_tokens order the caller's stream after it."""
        if self._prepared is None:
            raise RuntimeError("prepare_forward() must be called first")
        ne, th, rope_offset = self._prepared
        out_h, out_i = self._split_bufs
        L, ctx, st = self._L, self._ctx, self._draft_stream.cuda_stream
        _lib.check(L.dfl_cache_reset(ctx), "dfl_cache_reset")
        _lib.check(L.dfl_cache_set_offset(ctx, int(rope_offset)), "dfl_cache_set_offset")
        self._gen += 1
        if th.shape[0]:
            _lib.check(L.dfl_ingest_context(ctx, th.data_ptr(), th.shape[0], st),
                       "dfl_ingest_context")
        _lib.check(L.dfl_draft_block(ctx, ne.data_ptr(), None, ne.shape[0], out_h.data_ptr(),
                                     None, None, out_i.data_ptr() if self._has_lm else None, st),
                   "dfl_draft_block")
        self._done.record(self._draft_stream)
        if wait:
            self._done.synchronize()
        self._out_hidden, self._out_ids = out_h, (out_i if self._has_lm else None)

    def _after_draft(self, t):
        import torch
        torch.cuda.current_stream(self.device).wait_event(self._done)
        return t.clone()   # the buffers are rewritten by the next run_kernels

    def read_output(self):
        """ane_model.py:591-594: final-normed hidden [1, q, H] fp16."""
        if self._out_hidden is None:
            raise RuntimeError("run_kernels() has not produced an output")
        return self._after_draft(self._out_hidden).unsqueeze(0)

    def read_draft_tokens(self):
        """ane_model.py:596-604 / read_argmax (wrapper.rs:108-140): argmax ids [1, q]."""
        if self._out_ids is None:
            raise RuntimeError("lm_head not loaded -- no draft tokens")
        return self._after_draft(self._out_ids).reshape(1, -1)

    def run_prepared(self):
        self.run_kernels()
        return self.read_output()


def _check_ids(ids, V: int, flat: bool = True):
    """Token ids as an int32 tensor.  Host ids outside [0, V) raise ValueError here; ids
    already on the device are not read back (that would synchronise the host with the
    stream on every call): the kernels flag them in the device error word (bit 0, read with
    dfl_device_errors) and use a zero row."""
    import torch
    t = torch.as_tensor(ids)
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    if flat:
        t = t.reshape(-1)
    if not t.is_cuda and t.numel() and (int(t.min()) < 0 or int(t.max()) >= V):
        raise ValueError(f"token id outside [0, {V})")
    return t


def _feature_ptrs(feats, H: int, device):
    """Device pointer array of fp16 [C, H] feature rows with one common row stride.
    Accepts [1, C, H] or [C, H] tensors; copies only what is not already fp16 on the
    device with unit column stride and a stride shared by all."""
    import torch
    rows = []
    for f in feats:
        t = f
        if t.dim() == 3:
            if t.shape[0] != 1:
                raise ValueError("batch size must be 1")
            t = t[0]
        if t.dim() != 2 or t.shape[1] != H:
            raise ValueError(f"feature tensors must be [C, {H}], got {tuple(f.shape)}")
        if t.device != device or t.dtype != torch.float16:
            t = t.to(device, torch.float16)
        rows.append(t)
    C = rows[0].shape[0]
    if any(t.shape[0] != C for t in rows):
        raise ValueError("feature tensors differ in row count")
    ld = rows[0].stride(0)
    ok = all(t.stride(1) == 1 and t.stride(0) == ld and t.data_ptr() % 16 == 0 for t in rows)
    if not ok or ld % 8 or ld < H:
        # fresh storage is 16-byte aligned (a contiguous view at an odd offset stays unaligned)
        rows = [t.clone(memory_format=torch.contiguous_format) for t in rows]
        ld = H
    arr = (ctypes.c_void_p * len(rows))(*[t.data_ptr() for t in rows])
    return arr, len(rows), ld, C, rows


def concat_features(feats):
    """extract_context_feature of GPU tensors: [1, C, n*H] (or [C, n*H]) fp16 through
    dfl_concat_features."""
    import torch
    first = feats[0]
    H = first.shape[-1]
    arr, n, ld, C, keep = _feature_ptrs(feats, H, first.device)
    out = torch.empty((C, n * H), dtype=torch.float16, device=first.device)
    L = _lib.load()
    _lib.check(L.dfl_concat_features(arr, n, ld, C, H, out.data_ptr(),
                                     _lib.stream_handle()), "dfl_concat_features")
    return out.unsqueeze(0) if first.dim() == 3 else out


def _wrap_device(ptr: int, shape, device):
    """Non-owning torch view of fp16 device memory owned by the library."""
    import torch

    class _Holder:
        def __init__(self, p, shp):
            strides, acc = [], 1
            for d in reversed(shp):
                strides.insert(0, acc)
                acc *= d
            self.__cuda_array_interface__ = {
                "shape": tuple(shp), "typestr": "<f2", "data": (p, False),
                "version": 2, "strides": tuple(s * 2 for s in strides),
            }

    return torch.as_tensor(_Holder(ptr, shape), device=device)
