"""The oracle's argmax of one fixture row in other rounding mixes (run on the CPU, from the
repo root):

    python tests/golden/oracle_variants.py llama8b_batch 64

Each variant is the fp16-boundary forward with different accumulation only: fp32 or fp64,
every reduction summed over n ordered ranges (dflash_oracle.accumulation_split), and the
attention's P.V taking fp16 P (dflash_oracle.attention_fp16_p).  A row whose top-2 gap
changes sign across variants is decided by rounding order; parity_util.KNOWN_UNBACKED
cites this script's output for the one row the GPU decides differently from every variant.
"""

from __future__ import annotations

import contextlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "mirror-sd_amd"))

from mirror_sd_amd import synth  # noqa: E402
from mirror_sd_amd.config import workload  # noqa: E402
from oracle import dflash_oracle as O  # noqa: E402

VARIANTS = ([("fp32", 1, False, np.float32), ("fp64", 1, False, np.float64),
             ("fp64, fp16 P", 1, True, np.float64), ("fp32, fp16 P", 1, True, np.float32)] +
            [(f"fp32, split {n}", n, False, np.float32) for n in (2, 3, 4, 5, 7, 8, 12, 16, 32)] +
            [(f"fp32, fp16 P, split {n}", n, True, np.float32) for n in (2, 4, 8, 16)])


def main(name: str, row: int):
    wl = workload(name)
    cfg = wl.cfg
    t = synth.make_weights_numpy(cfg, seed=0)
    if wl.seq_ctx:   # batched fixture: rows stacked sequence-major
        seq, r = divmod(row, wl.block)
        inp = synth.make_batch_inputs_numpy(cfg, wl.block, wl.seq_ctx, seed=0)[seq]
    else:
        r = row
        inp = synth.make_inputs_numpy(cfg, wl.block, wl.ctx, seed=0)
    W = O.OracleWeights(cfg, t)
    del t
    for tag, n, pv16, dtype in VARIANTS:
        with O.accumulation_split(n), (O.attention_fp16_p() if pv16 else contextlib.nullcontext()):
            _, lg, ids = O.draft_block(W, inp["ids"], inp["target_hidden"], fp16=True, dtype=dtype)
        top = np.argsort(-lg[r], kind="stable")[:2]
        print(f"{name} row {row}: {tag:24s} id {int(ids[r])}  top-2 {top.tolist()}  gap "
              f"{float(lg[r, top[0]] - lg[r, top[1]]):.3e}", flush=True)


if __name__ == "__main__":
    main(sys.argv[1], int(sys.argv[2]))
