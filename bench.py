#!/usr/bin/env python3
"""Benchmark: DFlash draft-block latency + achieved HBM bandwidth on one MI355X.

Default workload (the headline): 27B-class draft, 5 layers, H5120, 40/8 heads,
FFN 17408, W8A16 projections, fp16 lm_head [151936, 5120], block 32, context 4096.

A step is one draft block: embedding of the block ids -> 5 decoder layers attending to
the resident context K/V plus the block -> final norm -> lm_head -> argmax ids.  The
context (fc fusion + per-layer K/V of 4096 rows) is ingested before timing; the ingest is
reported as its own phase (``context_ingest_ms``: the median of 5 ingests of the same
context run after the timed blocks, each listed in ``context_ingest_runs_ms``).  Weights
and inputs are synthetic (seeded, random-init).

``steady_step`` times the decode-loop step: 16 or 32 new context rows ingested (the
per-step path) and then the block, next to the ingest alone.

After the headline, the same run times the block step at resident contexts 64, 2048,
16384 and 32768 (``context_sweep``) and the batched-drafting workload (LLaMA-3.1-8B-class,
8 sequences x 32 rows, ragged contexts: ``batched``); both are extra keys, never ``value``.

Prints ONE JSON line.  ``value`` is the mean draft-block latency in microseconds over
the timed steps (inputs resident in HBM), after ``--warmup`` untimed blocks (default 200,
about 0.2 s): the GPU reaches its sustained clocks only after ~0.1 s of continuous work
(blocks run ~3 % slower before, and again after a second of idle), and a drafting loop
runs continuously.  The context sweep and the decode-loop steps run after the headline
(the GPU already warm) with a 5-block warmup each.  ``roofline`` describes the W8A16 projection
GEMM kernel, timed live with HIP events on the library's stream in a separate pass of
``--profile-steps`` blocks.  ``cpu_baseline`` times the CPU oracle (numpy fp32,
dequantised weights) on a bounded number of the same blocks on this host.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mirror-sd_amd"))

METRIC = ("draft-block latency (us) + achieved HBM GB/s, 27B-class W8A16 block=32 ctx=4096")
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0   # dense fp16 MFMA peak of MI355X


def algorithmic_bytes(cfg, block, ctx, n_seq=1):
    """Bytes a draft block must move from HBM: int8 projection weights + fp16 scales,
    context+block K/V read by attention, fp16 lm_head.  ``ctx`` may be a list of per-
    sequence contexts (batched drafting: the weights stream once for all sequences)."""
    H, NH, NKV, F, D = (cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads,
                        cfg.intermediate_size, cfg.head_dim)
    NQKV = (NH + 2 * NKV) * D
    per_layer_w = NQKV * H + H * NH * D + 2 * F * H + H * F
    per_layer_s = 2 * (NQKV + H + 2 * F + H)
    ctxs = list(ctx) if isinstance(ctx, (list, tuple)) else [ctx]
    kv = sum(2 * NKV * (c + block) * D * 2 for c in ctxs)
    nl = cfg.num_hidden_layers
    lm = cfg.vocab_size * H * 2
    return {"proj_weights": nl * per_layer_w, "proj_scales": nl * per_layer_s,
            "kv_read": nl * kv, "lm_head": lm,
            "total": nl * (per_layer_w + per_layer_s + kv) + lm}


def traffic_per_launch(workload_name):
    """HBM bytes per projection-GEMM launch from the committed counter measurement
    (rocprofv3 FETCH_SIZE and WRITE_SIZE passes, scaled by a known-size copy kernel), or
    None when no measurement for this workload is committed."""
    path = os.path.join(ROOT, "profiles", f"hbm_traffic_{workload_name}.json")
    try:
        with open(path) as f:
            return json.load(f)["gemm_w8a16"]["bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def build_model(wl, seed, keep_host: bool, max_ctx: int = 0, max_seqs: int = 1):
    """Synthetic weights generated on the GPU, quantised by the library's W8A16
    quantiser and loaded.  Optionally keeps host copies for the CPU baseline."""
    import torch
    from mirror_sd_amd.dflash import DFlashDraftModel
    from mirror_sd_amd import synth
    cfg = wl.cfg
    m = DFlashDraftModel(cfg, max_ctx=max_ctx or wl.ctx, max_block=max(wl.block, 32),
                         max_seqs=max_seqs)
    host = {}
    names = [n for n, _, _ in synth.weight_specs(cfg)]
    gen = dict(synth.make_weights_torch(cfg, seed=seed, device="cuda",
                                        only=[n for n in names if "layers." not in n]))
    for i in range(cfg.num_hidden_layers):
        lt = dict(synth.make_weights_torch(cfg, seed=seed, device="cuda",
                                           only=[n for n in names if n.startswith(f"layers.{i}.")]))
        qs, ss = [], []
        for p in synth.PROJ_NAMES:
            key = synth.proj_key(i, p)
            q, s = m.quantize_w8(lt.pop(key))
            qs.append(q)
            ss.append(s)
            if keep_host:
                host[key] = (q.cpu().numpy(), s.cpu().numpy())
        norms = [lt[f"layers.{i}.input_layernorm.weight"],
                 lt[f"layers.{i}.post_attention_layernorm.weight"],
                 lt[f"layers.{i}.self_attn.q_norm.weight"], lt[f"layers.{i}.self_attn.k_norm.weight"]]
        m.load_layer_q8(i, qs, ss, *norms)
        if keep_host:
            for k, v in lt.items():
                host[k] = v.cpu().numpy()
        del lt, qs, ss
    m.load_fc(gen["fc.weight"], gen["hidden_norm.weight"])
    m.load_head(gen["norm.weight"], gen["embed_tokens.weight"], gen["lm_head.weight"])
    if keep_host:
        for k in ("norm.weight", "embed_tokens.weight", "lm_head.weight"):
            host[k] = gen[k].cpu().numpy()
    del gen["fc.weight"]
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return m, host


def cpu_baseline(wl, model, host, ids, max_seconds=12.0, max_blocks=8):
    """Time the CPU oracle (numpy fp32, dequantised weights, fp16 materialisation) on
    the same block step: context K/V taken from the GPU cache, block of ``wl.block``
    ids, 5 layers + final norm + lm_head + argmax."""
    import numpy as np
    import torch
    from oracle import dflash_oracle as O
    cfg = wl.cfg
    f32 = np.float32
    W = O.OracleWeights.__new__(O.OracleWeights)
    W.cfg, W.fc = cfg, None
    W.hidden_norm = None
    W.norm = host["norm.weight"]
    W.embed = host["embed_tokens.weight"]
    W.lm_head = host["lm_head.weight"].astype(f32)
    W.layers = []
    for i in range(cfg.num_hidden_layers):
        lw = {p: O.dequantize_w8(*host[f"layers.{i}.{'mlp' if p in ('gate_proj', 'up_proj', 'down_proj') else 'self_attn'}.{p}.weight"], dtype=f32)
              for p in O.OracleWeights.PROJ}
        lw["input_layernorm"] = host[f"layers.{i}.input_layernorm.weight"]
        lw["post_attention_layernorm"] = host[f"layers.{i}.post_attention_layernorm.weight"]
        lw["q_norm"] = host[f"layers.{i}.self_attn.q_norm.weight"]
        lw["k_norm"] = host[f"layers.{i}.self_attn.k_norm.weight"]
        W.layers.append(lw)
    caches = []
    C = wl.ctx
    for i in range(cfg.num_hidden_layers):
        k, vt = model._cache_tensors[i]
        c = O.OracleKVCache()
        c.keys = k[:, :C].float().cpu().numpy()
        c.values = vt[:, :, :C].transpose(1, 2).float().cpu().numpy()
        c.offset = C
        caches.append(c)
    empty = np.zeros((0, cfg.hidden_size), dtype=np.float16)   # no new context rows
    ids_np = ids.cpu().numpy()
    times = []
    t_all = time.perf_counter()
    while len(times) < max_blocks and (len(times) < 2 or time.perf_counter() - t_all < max_seconds):
        t0 = time.perf_counter()
        noise = O.embed(W, ids_np)
        h = O.draft_forward(W, noise, empty, cache=caches, fp16=True, fused_context=True,
                            dtype=f32)
        logits = O.lm_head_logits(h, W.lm_head, dtype=f32)
        O.argmax_first(logits)
        times.append(time.perf_counter() - t0)
        for c in caches:
            c.trim(wl.block)
    try:
        from threadpoolctl import threadpool_info
        cores = max([p.get("num_threads", 1) for p in threadpool_info()] + [1])
    except Exception:
        cores = len(os.sched_getaffinity(0))
    return {"value": float(np.mean(times) * 1e6), "unit": "us", "cores": int(cores),
            "kind": "port",
            "sample": f"{len(times)} full draft blocks of the same workload (numpy fp32 oracle, "
                      f"dequantised W8A16 weights, context K/V precomputed)"}


def python_path_steps(model, wl, args, ids, k=16):
    """The decode-loop step through the Python drop-in interface, as the serial caller
    makes it (generate.py:591-609): ``draft_model(noise_embedding, target_hidden, cache)``
    with k new context rows, the host waiting for the result, then ``c.trim(block)`` on
    every layer's cache; and the fused ``draft(ids, target_hidden, cache)`` (ids instead of
    hidden states) the same way.  Wall-clock per step, host overhead included."""
    import torch
    from mirror_sd_amd import synth
    cfg = wl.cfg
    full = synth.make_inputs_torch(cfg, wl.block, wl.ctx, seed=args.seed, device="cuda")
    rows = synth.make_inputs_torch(cfg, wl.block, k, seed=args.seed + 7,
                                   device="cuda")["target_hidden"][None]
    noise = model.embed_block(ids)
    cache = model.make_cache(0, 0)
    model(noise, full["target_hidden"][None], cache=cache)   # the resident context
    for c in cache:
        c.trim(wl.block)
    del full
    res = {}
    for name, call in (("call", lambda: model(noise, rows, cache=cache)),
                       ("draft", lambda: model.draft(ids, rows, cache=cache))):
        n = 0
        for it in range(5 + args.steps):
            if it == 5:
                torch.cuda.synchronize()
                t0 = time.perf_counter()
            out = call()
            torch.cuda.synchronize()   # the caller reads the result (mx.eval, generate.py:606)
            for c in cache:
                c.trim(wl.block)
            n += 1
        res[f"{name}_step_us"] = round((time.perf_counter() - t0) * 1e6 / args.steps, 2)
    res["what"] = (f"wall-clock per decode-loop step through the Python interface: {k} new "
                   f"context rows + the block ({wl.ctx}-row resident context), host waits for "
                   f"the result, then trim(block) on every layer: call_step_us = "
                   f"draft_model(noise, target_hidden, cache) (hidden states out), "
                   f"draft_step_us = draft(ids, target_hidden, cache) (ids out)")
    print(f"python path, {k} new rows: __call__ {res['call_step_us']:.1f} us, draft() "
          f"{res['draft_step_us']:.1f} us per step", file=sys.stderr, flush=True)
    return res


def run_workload(wl, args, sweep, want_cpu):
    """Build the model of workload ``wl``, ingest its context(s), time ``args.steps`` draft
    blocks (after ``args.warmup``), profile the kernels and optionally sweep the resident
    context length.  Returns the measurement dict (the JSON line's fields)."""
    import torch
    from mirror_sd_amd import synth, _lib

    cfg = wl.cfg
    batched = bool(wl.seq_ctx)   # several independent sequences drafted together
    torch.manual_seed(args.seed)
    t_setup = time.perf_counter()
    n_seq = len(wl.seq_ctx) if batched else 1
    # room for the swept contexts and for the rows the decode-loop steps append
    # sweep and decode-loop steps come after the headline's warmup and timed blocks
    warm_after = min(args.warmup, 5)
    steady_rows = 0 if batched or not args.steady else (warm_after + args.steps) * 32
    model, host = build_model(wl, args.seed, keep_host=want_cpu,
                              max_ctx=max([wl.ctx + steady_rows] + sweep), max_seqs=n_seq)
    if batched:
        seq_inp = [synth.make_inputs_torch(cfg, wl.block, c, seed=args.seed + 1 + i, device="cuda")
                   for i, c in enumerate(wl.seq_ctx)]
        ths = [d["target_hidden"] for d in seq_inp]
        ids = torch.cat([d["ids"] for d in seq_inp]).contiguous()
        del seq_inp
    else:
        inp = synth.make_inputs_torch(cfg, wl.block, wl.ctx, seed=args.seed, device="cuda")
        ths, ids = [inp["target_hidden"]], inp["ids"]
    setup_s = time.perf_counter() - t_setup

    L = model._L
    ctx = model._ctx
    stream = torch.cuda.current_stream()
    sh = stream.cuda_stream
    out_ids = torch.empty((n_seq * wl.block,), dtype=torch.int32, device="cuda")

    # context ingest (fc fusion + per-layer K/V): one untimed ingest here (the first
    # launches load the kernels' code objects); the timed ones run after the headline
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    def ingest_all():
        for i, t in enumerate(ths):
            _lib.check(L.dfl_select_seq(ctx, i), "dfl_select_seq")
            _lib.check(L.dfl_cache_reset(ctx), "dfl_cache_reset")
            _lib.check(L.dfl_ingest_context(ctx, t.data_ptr(), t.shape[0], sh),
                       "dfl_ingest_context")
        _lib.check(L.dfl_select_seq(ctx, 0), "dfl_select_seq")

    t_first = time.perf_counter()
    ingest_all()
    torch.cuda.synchronize()
    first_ingest_s = time.perf_counter() - t_first

    def step():
        if batched:
            rc = L.dfl_draft_batch(ctx, n_seq, None, ids.data_ptr(), wl.block, None, None, None,
                                   out_ids.data_ptr(), sh)
        else:
            rc = L.dfl_draft_block(ctx, None, ids.data_ptr(), wl.block, None, None, None,
                                   out_ids.data_ptr(), sh)
        if rc:
            _lib.check(rc, "dfl_draft_batch" if batched else "dfl_draft_block")

    for _ in range(args.warmup):
        step()
    def timed(k, gemm_events):
        """k back-to-back blocks between two stream events.  With gemm_events the
        stream-K GEMM launches also carry dispatch-timestamp events (no extra packets)."""
        if gemm_events:
            model.profile(True, gemm_only=True)
            model.profile_read()
        torch.cuda.synchronize()
        ev0.record(stream)
        t0 = time.perf_counter()
        for _ in range(k):
            step()
        ev1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        prof = None
        if gemm_events:
            prof = model.profile_read()
            model.profile(False)
        return ev0.elapsed_time(ev1) / k, wall, prof

    ms_per_step, wall_s, _ = timed(args.steps, False)
    first_ids = out_ids.cpu().tolist()
    # The context ingest as its own phase, on the GPU warmed up by the blocks (as a drafting
    # loop's prompt ingest follows the target's prefill): 5 ingests of the same context
    # (cache reset, then the rows again), the median reported and each run listed.
    ingest_runs = []
    for _ in range(5):
        torch.cuda.synchronize()
        ev0.record(stream)
        ingest_all()
        ev1.record(stream)
        torch.cuda.synchronize()
        ingest_runs.append(ev0.elapsed_time(ev1))
    ingest_ms = sorted(ingest_runs)[len(ingest_runs) // 2]
    # The same K steps again with dispatch-timestamp events on the GEMM launches: the
    # kernel durations they give match a kernel trace, but attaching them lengthens the
    # gaps between dispatches, so the headline latency comes from the plain run above.
    ms_events, gprof = None, None
    if not args.no_profile:
        ms_events, _, gprof = timed(args.steps, True)

    nbytes = algorithmic_bytes(cfg, wl.block, list(wl.seq_ctx) if batched else wl.ctx)
    lat_us = ms_per_step * 1e3
    gbs = nbytes["total"] / (ms_per_step * 1e-3) / 1e9

    def rate(r):
        avg_s = r["ms"] * 1e-3 / r["launches"]
        per_launch = r["bytes"] / r["launches"]
        return per_launch, avg_s, per_launch / avg_s / 1e9

    roofline, kernels = None, None
    rows = n_seq * wl.block
    stacked = rows > 64
    gkey = "gemm_tile_rows" if stacked else "gemm_w8a16"
    if gprof and gprof.get(gkey, {}).get("launches"):
        per_launch, avg_s, ach = rate(gprof[gkey])
        # 2 * rows flop per int8 weight byte: above the MFMA/HBM ridge the projections are
        # bounded by the matrix cores (stacked blocks), below it by HBM (one block)
        if 2.0 * rows > MFMA_F16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9):
            tf = 2.0 * rows * per_launch / avg_s / 1e12
            roofline = {"bound": "mfma", "achieved": round(tf, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                        "unit": "TFLOP/s", "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                        "hbm_gbps": round(ach, 1)}
        else:
            roofline = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4)}
        kname = ("tile_gemm_kernel<int8> (LDS-staged MFMA tile GEMM of the stacked rows: qkv, "
                 "o, gate_up, down)" if stacked else
                 "gsk_gemm_kernel<int8,*> (stream-K W8A16 projections qkv/o/gate_up/down, one "
                 "launch each per layer)")
        roofline.update({"traffic": traffic_per_launch(wl.name), "kernel": kname,
                         "bytes_per_launch": per_launch, "avg_launch_us": round(avg_s * 1e6, 3),
                         "launches": gprof[gkey]["launches"]})
        lm = gprof.get("lm_head_argmax", {})
        if lm.get("launches"):
            per_launch, avg_s, ach = rate(lm)
            lm_name = ("tile_gemm_kernel<fp16> (stacked rows; row argmax after)" if stacked else
                       "gsk_dyn_kernel<fp16,ARGMAX> (balanced)")
            roofline["lm_head"] = {"kernel": lm_name, "achieved": round(ach, 1),
                                   "frac": round(ach / HBM_PEAK_GBS, 4),
                                   "bytes_per_launch": per_launch,
                                   "avg_launch_us": round(avg_s * 1e6, 3)}
            if stacked:   # fp16 weights: rows flop per weight byte
                tf = rows * per_launch / avg_s / 1e12
                roofline["lm_head"].update({"tflops": round(tf, 1),
                                            "mfma_frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4)})
    if not args.no_profile and args.profile_steps > 0:
        # per-group breakdown; groups other than the GEMMs are bracketed by marker events,
        # which add a few microseconds of dispatch latency each
        model.profile(True)
        model.profile_read()
        for _ in range(args.profile_steps):
            step()
        torch.cuda.synchronize()
        prof = model.profile_read()
        model.profile(False)
        kernels = {}
        for name, r in prof.items():
            if r["launches"] == 0:
                continue
            ent = {"ms_per_block": r["ms"] / args.profile_steps,
                   "launches_per_block": r["launches"] / args.profile_steps}
            if r["bytes"]:
                ent["gbs"] = r["bytes"] / (r["ms"] * 1e-3) / 1e9
                ent["bytes_per_launch"] = r["bytes"] / r["launches"]
            kernels[name] = ent

    steady = None
    if not batched and args.steady:
        # the decode-loop step: k new context rows ingested (the per-step stream-K path),
        # then the block; and the ingest alone (its rows trimmed again)
        steady = {}
        for k in (16, 32):
            rows = synth.make_inputs_torch(cfg, wl.block, k, seed=args.seed + 7,
                                           device="cuda")["target_hidden"]
            def ingest_k():
                _lib.check(L.dfl_ingest_context(ctx, rows.data_ptr(), k, sh), "dfl_ingest_context")
            def ingest_only():
                ingest_k()
                _lib.check(L.dfl_cache_trim(ctx, k), "dfl_cache_trim")
            for _ in range(warm_after):
                ingest_only()
            torch.cuda.synchronize()
            ev0.record(stream)
            for _ in range(args.steps):
                ingest_only()
            ev1.record(stream)
            torch.cuda.synchronize()
            ing_us = ev0.elapsed_time(ev1) * 1e3 / args.steps
            n_app = 0
            for _ in range(warm_after):
                ingest_k()
                step()
                n_app += k
            torch.cuda.synchronize()
            ev0.record(stream)
            for _ in range(args.steps):
                ingest_k()
                step()
                n_app += k
            ev1.record(stream)
            torch.cuda.synchronize()
            step_us = ev0.elapsed_time(ev1) * 1e3 / args.steps
            _lib.check(L.dfl_cache_trim(ctx, n_app), "dfl_cache_trim")   # back to the context
            steady[str(k)] = {"step_us": round(step_us, 2), "ingest_us": round(ing_us, 2),
                              "context_rows": f"{wl.ctx} + {k} per step"}
            print(f"steady step, {k} new rows: {step_us:.1f} us (ingest {ing_us:.1f} us)",
                  file=sys.stderr, flush=True)
            del rows

    context_sweep = None
    if sweep:
        # the block step against other resident context lengths (same weights)
        context_sweep = {}
        for C in sweep:
            sw = synth.make_inputs_torch(cfg, wl.block, C, seed=args.seed, device="cuda")
            model.make_cache(0, 0)
            torch.cuda.synchronize()
            ev0.record(stream)
            _lib.check(L.dfl_ingest_context(ctx, sw["target_hidden"].data_ptr(), C, sh),
                       "dfl_ingest_context")
            ev1.record(stream)
            torch.cuda.synchronize()
            ing = ev0.elapsed_time(ev1)
            del sw
            for _ in range(warm_after):
                step()
            ms_c, _, _ = timed(args.steps, False)
            nb = algorithmic_bytes(cfg, wl.block, C)["total"]
            context_sweep[str(C)] = {"block_us": round(ms_c * 1e3, 2),
                                     "hbm_gbps": round(nb / (ms_c * 1e-3) / 1e9, 1),
                                     "ingest_ms": round(ing, 3)}
            print(f"context {C}: block {ms_c * 1e3:.1f} us, ingest {ing:.2f} ms",
                  file=sys.stderr, flush=True)

    python_path = None
    if not batched and args.steady:
        python_path = python_path_steps(model, wl, args, ids)

    cpu = None
    if want_cpu:
        try:
            cpu = cpu_baseline(wl, model, host, ids)
        except Exception as e:  # report, never lose the GPU line
            cpu = {"value": None, "error": f"{type(e).__name__}: {e}"}
    model.close()
    del model, host, ths
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return {"lat_us": lat_us, "ms_per_step": ms_per_step, "wall_s": wall_s, "gbs": gbs,
            "nbytes": nbytes, "roofline": roofline, "kernels": kernels, "cpu": cpu,
            "ingest_ms": ingest_ms, "ingest_runs": ingest_runs, "first_ingest_s": first_ingest_s,
            "setup_s": setup_s,
            "ms_events": ms_events, "context_sweep": context_sweep, "steady": steady,
            "python_path": python_path, "first_ids": first_ids,
            "n_seq": n_seq, "batched": batched}


# The context sweep of the headline draft (contexts 64 .. 32768; 4096 is the headline itself)
# and the batched-drafting workload run by default after the headline, as extra keys.
DEFAULT_SWEEP = "64,2048,16384,32768"
EXTRA_WORKLOAD = "llama8b_batch"


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=200,
                    help="untimed blocks before the timed ones (the GPU's clocks ramp up "
                         "over the first ~0.1 s of continuous work)")
    ap.add_argument("--workload", default="dflash_27b")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--profile-steps", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-profile", action="store_true")
    ap.add_argument("--sweep", default=None,
                    help="comma-separated contexts: after the headline, time the block step "
                         f"at each of these context lengths too (default for the headline "
                         f"workload: {DEFAULT_SWEEP}; '' for none)")
    ap.add_argument("--no-steady", dest="steady", action="store_false",
                    help="skip the decode-loop step timing (16 / 32 new context rows + block)")
    ap.add_argument("--no-extra", action="store_true",
                    help=f"skip the batched-drafting workload ({EXTRA_WORKLOAD}) that the "
                         "headline run reports as an extra key")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="run a plain device copy of this many MiB 3 times first (a known-size "
                         "kernel for scaling FETCH_SIZE / WRITE_SIZE counter readings)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: runs on exactly one GPU; --gpus {args.gpus} is not supported (the "
              f"multi-GPU sharding is designed, not implemented)", file=sys.stderr)
        sys.exit(2)

    import torch
    from mirror_sd_amd.config import workload

    wl = workload(args.workload)
    cfg = wl.cfg
    batched = bool(wl.seq_ctx)
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    headline = wl.name == "dflash_27b"
    want_cpu = not args.no_cpu_baseline and not batched
    if args.copy_probe_mib > 0:
        n = (args.copy_probe_mib << 20) // 4
        src = torch.ones(n, dtype=torch.int32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):   # elementwise kernel: reads n*4 bytes, writes n*4 bytes
            torch.bitwise_not(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    sweep_arg = args.sweep if args.sweep is not None else (DEFAULT_SWEEP if headline else "")
    sweep = [int(c) for c in sweep_arg.split(",") if c.strip()] if not batched else []
    r = run_workload(wl, args, sweep, want_cpu)

    extra = None
    if headline and not args.no_extra:
        # the batched drafting workload (8 sequences x 32 rows, ragged contexts): stacked
        # M = 256 projections, MFMA-bound
        xw = workload(EXTRA_WORKLOAD)
        x = run_workload(xw, args, [], False)
        tokens = x["n_seq"] * xw.block
        extra = {"workload": xw.name, "config": {"hidden": xw.cfg.hidden_size,
                                                  "layers": xw.cfg.num_hidden_layers,
                                                  "ffn": xw.cfg.intermediate_size,
                                                  "vocab": xw.cfg.vocab_size,
                                                  "sequences": x["n_seq"], "block": xw.block,
                                                  "ctx": list(xw.seq_ctx)},
                 "block_us": round(x["lat_us"], 2),
                 "draft_tokens_per_s": round(tokens / (x["ms_per_step"] * 1e-3), 1),
                 "hbm_gbps": round(x["gbs"], 1),
                 "algorithmic_bytes_per_block": x["nbytes"]["total"],
                 "roofline": x["roofline"], "kernels": x["kernels"],
                 "context_ingest_ms": round(x["ingest_ms"], 3),
                 "context_ingest_runs_ms": [round(v, 3) for v in x["ingest_runs"]]}
        print(f"{xw.name}: block {x['lat_us']:.1f} us", file=sys.stderr, flush=True)

    metric = METRIC if headline else \
        f"draft-block latency (us) + achieved HBM GB/s, {wl.description}"
    out = {
        "metric": metric, "value": round(r["lat_us"], 2), "unit": "us", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(r["ms_per_step"], 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (seeded random-init weights, N(0,1) target_hidden)",
        "config": {"workload": wl.name, "hidden": cfg.hidden_size, "layers": cfg.num_hidden_layers,
                   "heads": cfg.num_attention_heads, "kv_heads": cfg.num_key_value_heads,
                   "ffn": cfg.intermediate_size, "vocab": cfg.vocab_size, "block": wl.block,
                   "ctx": list(wl.seq_ctx) if batched else wl.ctx, "sequences": r["n_seq"],
                   "weights": "W8A16 (int8 + fp16 per-row scale), fp16 lm_head"},
        "hbm_gbps": round(r["gbs"], 1),
        "algorithmic_bytes_per_block": r["nbytes"]["total"],
        "roofline": r["roofline"],
        "cpu_baseline": r["cpu"],
        "phases": {"context_ingest_ms": round(r["ingest_ms"], 3),
                   "context_ingest_runs_ms": [round(v, 3) for v in r["ingest_runs"]],
                   "first_ingest_s": round(r["first_ingest_s"], 3), "setup_s": round(r["setup_s"], 1),
                   "ms_per_step_with_gemm_events": (round(r["ms_events"], 5) if r["ms_events"]
                                                    else None),
                   "wall_ms_per_step": round(r["wall_s"] * 1e3 / args.steps, 4)},
        "kernels": r["kernels"],
        "steady_step": r["steady"],
        "python_path": r["python_path"],
        "context_sweep": r["context_sweep"],
        "batched": extra,
        "draft_ids_head": r["first_ids"][:4],
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
