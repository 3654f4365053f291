"""Write the golden fixtures of the draft forward (run on the CPU, from the repo root):

    python tests/golden/make_golden.py [case ...]

Each fixture holds the oracle's outputs for one named workload on the seeded synthetic
inputs of ``mirror_sd_amd.synth`` (numpy back-end), plus crc32 digests of those inputs
so a test can tell a change of the input recipe from a change of the results:

  qwen3_4b_layer  1 layer, H2560, 32/8 heads, FFN 9728, block 16, context 64, inputs
                  already fused (noise [16, 2560], context [64, 2560]); output the
                  final-normed hidden [16, 2560] and the residual stream before it.
  qwen3_8b_draft  5 layers, H4096, 32/8, FFN 12288, block 16, context 2048, fc fusion of
                  5 x 4096 features, V151936; outputs hidden [16, 4096], argmax ids [16],
                  the top-2 logits per row.
  dflash_27b      5 layers, H5120, 40/8, FFN 17408, block 32, context 4096, V151936;
                  same outputs for 32 rows.
  dflash_27b_ctxN the 27B-class draft at context N in {64, 2048, 16384, 32768} (the context
                  sweep; N = 4096 is dflash_27b): same weights (seed 0), inputs of N rows.
  dflash_27b_steady  the 27B-class draft in a decode loop: context rows 0..4096, then 1,
                  16 and 32 more rows; after each of those ingests a block of 32 is drafted.
                  One fixture entry per step (prefix s0, s1, s2), each the oracle's single
                  pass over that step's context prefix (4097, 4113, 4145 rows).
  llama8b_batch   5 layers, H4096, 32/8, FFN 14336, V128256, theta 5e5; 8 independent
                  sequences x block 32 with contexts [4146, 4443, 6312, 7812, 779, 1619, 6833,
                  7798]; each sequence run through the single-sequence oracle; outputs stacked
                  sequence-major: hidden [256, 4096], ids [256], top-2 logits per row.

The oracle runs in its fp16-boundary mode (the MLX rounding points) with fp32
accumulation for the two full models, fp64 for the single layer.

Every fixture with argmax ids also holds ``ids_f64`` / ``top2_val_f64``: the same forward
with fp64 accumulation (same fp16 rounding points), and ``ids_ksplit`` [len(KSPLITS), rows]:
the fp32 forward with every reduction matmul summed over 2, 4 and 8 ordered ranges of its
reduction axis (``dflash_oracle.accumulation_split``: how a GPU GEMM splits k, as rounding
alone).  A row whose argmax differs between these runs is decided by accumulation
rounding alone; those rows are the only ones the GPU parity tests may exempt from exact
argmax agreement.  ``--add-f64`` / ``--add-ksplit`` add these arrays to existing fixtures
without touching the rest.
"""

from __future__ import annotations

import os
import sys
import time
import zlib

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "mirror-sd_amd"))

from mirror_sd_amd import synth  # noqa: E402
from mirror_sd_amd.config import workload  # noqa: E402
from oracle import dflash_oracle as O  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
DIGEST_BYTES = 1 << 20


def digest(a: np.ndarray) -> int:
    """crc32 of the first MiB of the array's bytes, mixed with its shape and dtype."""
    b = np.ascontiguousarray(a).view(np.uint8).ravel()[:DIGEST_BYTES].tobytes()
    return zlib.crc32(f"{a.shape}{a.dtype}".encode() + b) & 0xFFFFFFFF


def input_digests(tensors, inp):
    names = sorted(tensors)
    d = {f"w:{n}": digest(tensors[n]) for n in names}
    d.update({f"in:{k}": digest(v) for k, v in inp.items()})
    return d


def top2(logits):
    idx = np.argsort(-logits, axis=-1, kind="stable")[:, :2].astype(np.int32)
    val = np.take_along_axis(logits, idx, axis=-1).astype(np.float32)
    return idx, val


def case_layer(name="qwen3_4b_layer", seed=0):
    wl = workload(name)
    cfg = wl.cfg
    t = synth.make_weights_numpy(cfg, seed=seed, with_vocab=False, with_fc=False)
    inp = synth.make_inputs_numpy(cfg, wl.block, wl.ctx, seed=seed, fused_context=True)
    W = O.OracleWeights(cfg, t)
    out, pre = O.draft_forward(W, inp["noise"], inp["context"], fp16=True, fused_context=True,
                               return_prenorm=True)
    return dict(hidden=out.astype(np.float16), prenorm=pre.astype(np.float16)), \
        input_digests(t, inp)


KSPLITS = (2, 4, 8)


def ksplit_ids(W, inp):
    """[len(KSPLITS), rows] argmax ids of the fp32 forward in the other summation orders."""
    out = []
    for n in KSPLITS:
        with O.accumulation_split(n):
            _, _, ids = O.draft_block(W, inp["ids"], inp["target_hidden"], fp16=True,
                                      dtype=np.float32)
        out.append(ids.astype(np.int32))
    return np.stack(out)


def f64_outputs(W, inp):
    """ids and top-2 logits of the fp64-accumulation run (fp16 rounding points kept)."""
    _, logits, ids = O.draft_block(W, inp["ids"], inp["target_hidden"], fp16=True,
                                   dtype=np.float64)
    _, tv = top2(logits)
    return ids.astype(np.int32), tv


def case_full(name, seed=0, only=None):
    wl = workload(name)
    cfg = wl.cfg
    t = synth.make_weights_numpy(cfg, seed=seed)
    inp = synth.make_inputs_numpy(cfg, wl.block, wl.ctx, seed=seed)
    dig = input_digests(t, inp)
    W = O.OracleWeights(cfg, t)
    del t
    if only == "ksplit":
        return dict(ids_ksplit=ksplit_ids(W, inp)), dig
    ids64, tv64 = f64_outputs(W, inp)
    if only == "f64":
        return dict(ids_f64=ids64, top2_val_f64=tv64), dig
    h, logits, ids = O.draft_block(W, inp["ids"], inp["target_hidden"], fp16=True,
                                   dtype=np.float32)
    ti, tv = top2(logits)
    return dict(hidden=h.astype(np.float16), ids=ids.astype(np.int32), top2_idx=ti,
                top2_val=tv, ids_f64=ids64, top2_val_f64=tv64, ids_ksplit=ksplit_ids(W, inp)), dig


STEADY_BASE, STEADY_STEPS = 4096, (1, 16, 32)


def case_steady(name="dflash_27b_steady", seed=0, only=None):
    """The decode-loop protocol: the context grows by STEADY_STEPS rows after a 4096-row
    prefix; a draft after each step equals a single pass over the prefix (context K/V
    depend only on the fused context rows and their positions)."""
    wl = workload("dflash_27b")
    cfg = wl.cfg
    total = STEADY_BASE + sum(STEADY_STEPS)
    t = synth.make_weights_numpy(cfg, seed=seed)
    inp = synth.make_inputs_numpy(cfg, wl.block, total, seed=seed)
    dig = input_digests(t, inp)
    W = O.OracleWeights(cfg, t)
    del t
    out = {}
    n = STEADY_BASE
    for i, k in enumerate(STEADY_STEPS):
        n += k
        sub = {"ids": inp["ids"], "target_hidden": inp["target_hidden"][:n]}
        if only != "f64":
            out[f"s{i}_ids_ksplit"] = ksplit_ids(W, sub)
        if only == "ksplit":
            print(f"{name}: step {i} ({n} context rows) done", flush=True)
            continue
        ids64, tv64 = f64_outputs(W, sub)
        out[f"s{i}_ids_f64"], out[f"s{i}_top2_val_f64"] = ids64, tv64
        if only == "f64":
            continue
        h, logits, ids = O.draft_block(W, sub["ids"], sub["target_hidden"], fp16=True,
                                       dtype=np.float32)
        ti, tv = top2(logits)
        out.update({f"s{i}_hidden": h.astype(np.float16), f"s{i}_ids": ids.astype(np.int32),
                    f"s{i}_top2_idx": ti, f"s{i}_top2_val": tv})
        print(f"{name}: step {i} ({n} context rows) done", flush=True)
    return out, dig


def case_batch(name="llama8b_batch", seed=0, only=None):
    wl = workload(name)
    cfg = wl.cfg
    t = synth.make_weights_numpy(cfg, seed=seed)
    inps = synth.make_batch_inputs_numpy(cfg, wl.block, wl.seq_ctx, seed=seed)
    dig = input_digests(t, {f"{k}.s{i}": v for i, inp in enumerate(inps) for k, v in inp.items()})
    W = O.OracleWeights(cfg, t)
    del t
    hs, idss, tis, tvs, i64s, v64s, kss = [], [], [], [], [], [], []
    for inp in inps:
        if only != "f64":
            kss.append(ksplit_ids(W, inp))
        if only == "ksplit":
            continue
        ids64, tv64 = f64_outputs(W, inp)
        i64s.append(ids64)
        v64s.append(tv64)
        if only == "f64":
            continue
        h, logits, ids = O.draft_block(W, inp["ids"], inp["target_hidden"], fp16=True,
                                       dtype=np.float32)
        ti, tv = top2(logits)
        hs.append(h.astype(np.float16))
        idss.append(ids.astype(np.int32))
        tis.append(ti)
        tvs.append(tv)
    f64 = dict(ids_f64=np.concatenate(i64s), top2_val_f64=np.concatenate(v64s)) if i64s else {}
    if only == "f64":
        return f64, dig
    ks = dict(ids_ksplit=np.concatenate(kss, axis=1))
    if only == "ksplit":
        return ks, dig
    return dict(hidden=np.concatenate(hs), ids=np.concatenate(idss), top2_idx=np.concatenate(tis),
                top2_val=np.concatenate(tvs), **f64, **ks), dig


CASES = {
    "qwen3_4b_layer": lambda only=None: case_layer("qwen3_4b_layer"),
    "qwen3_8b_draft": lambda only=None: case_full("qwen3_8b_draft", only=only),
    "dflash_27b": lambda only=None: case_full("dflash_27b", only=only),
    **{f"dflash_27b_ctx{c}": (lambda only=None, c=c:
                              case_full(f"dflash_27b_ctx{c}", only=only))
       for c in (64, 2048, 16384, 32768)},
    "llama8b_batch": lambda only=None: case_batch("llama8b_batch", only=only),
    "dflash_27b_steady": lambda only=None: case_steady(only=only),
}
ARGMAX_CASES = [n for n in CASES if n != "qwen3_4b_layer"]


def main(argv):
    # None: write whole fixtures; "f64" / "ksplit": add those runs' arrays to existing ones
    add = "ksplit" if "--add-ksplit" in argv else ("f64" if "--add-f64" in argv else None)
    names = [a for a in argv if not a.startswith("--")] or \
        (ARGMAX_CASES if add else list(CASES))
    for n in names:
        t0 = time.time()
        path = os.path.join(HERE, f"{n}.npz")
        out, dig = CASES[n](only=add)
        keys = sorted(dig)
        if add:   # keep the stored outputs; the inputs must be the ones they came from
            with np.load(path) as old:
                kept = {k: old[k] for k in old.files}
            assert dict(zip(kept["digest_names"].tolist(),
                            kept["digest_values"].tolist())) == dig, f"{n}: inputs changed"
            kept.update(out)
            np.savez_compressed(path, **kept)
        else:
            np.savez_compressed(path, **out, digest_names=np.array(keys),
                                digest_values=np.array([dig[k] for k in keys], dtype=np.uint32))
        print(f"{n}: {time.time() - t0:.1f} s, outputs {sorted(out)}", flush=True)


if __name__ == "__main__":
    main(sys.argv[1:])
