"""Condense rocprofv3 output of a bench run into the short text kept under profiles/.

Inputs (csv output of rocprofv3):
  --stats   <dir>/<name>_kernel_stats.csv from ``--kernel-trace --stats``, or
  --trace   <dir>/<name>_kernel_trace.csv from ``--kernel-trace`` with ``--skip-blocks N``:
            the durations of every dispatch except those of the first N draft blocks (the
            bench's warmup, run while the GPU's clocks ramp up), so that the averages cover
            the same blocks as the bench's timed region
  --fetch   <dir>/<name>_counter_collection.csv from ``--pmc FETCH_SIZE``
  --write   <dir>/<name>_counter_collection.csv from ``--pmc WRITE_SIZE``
  --mfma    <dir>/<name>_counter_collection.csv from ``--pmc MfmaUtil MfmaFlopsF16``: per
            group, the matrix cores' busy share (MfmaUtil: MFMA-busy cycles over the active
            cycles of every SIMD) and the fp16 MFMA rate (MfmaFlopsF16 over the dispatch's
            own duration in that run; counters are collected with the dispatches serialised)
Both counter runs include a plain elementwise copy of known size (bench.py
``--copy-probe-mib``); its readings give the factor that turns each counter into bytes
(FETCH_SIZE / WRITE_SIZE are reported in KiB, but what one KiB of reading means depends
on the request sizes the memory system sees, so it is calibrated rather than assumed).

Writes a markdown summary and a json file with the per-launch HBM traffic of the
W8A16 projection GEMMs and the lm_head GEMM (read by bench.py for ``roofline.traffic``).
"""

from __future__ import annotations

import argparse
import collections
import csv
import json
import re
import sys

# kernel groups: (label, regex on the kernel name)
GROUPS = [
    ("proj_gemm_w8a16", r"gsk_gemm_kernel<0, [145], (true|false), 4, false>"),
    ("qkv (norm-on-load; Q/K norm + RoPE + cache scatter in the epilogue)",
     r"gsk_gemm_kernel<0, 5, true, 4, false>"),
    ("o / down (RESID)", r"gsk_gemm_kernel<0, 4, false, 4, false>"),
    ("gate|up (SWIGLU, norm-on-load)", r"gsk_gemm_kernel<0, 1, true, 4, false>"),
    ("lm_head (fp16, ARGMAX, norm-on-load)", r"gsk_(gemm_kernel<1, 2, true, 4, false|dyn_kernel<1, 2, true, 4)>"),
    ("M-split stream-K (stacked rows up to 64)", r"gsk_gemm_m_kernel"),
    ("per-step ingest fc (fp16, zero-residual RESID: rows + row sums), up to 16 rows read in "
     "place", r"gsk_gemm_kernel<1, 4, false, 4, true>"),
    ("per-step ingest fc, rows gathered into fragment layout first (17-32, or unaligned)",
     r"gsk_gemm_kernel<1, 4, false, 4, false>"),
    ("per-step ingest K|V, all layers (int8 STORE, hidden_norm on load)",
     r"gsk_gemm_kernel<0, 3, true, 4, false>"),
    ("tile GEMM int8, fp32 rows (stacked qkv; split-K planes of o, down; prompt-sized ingest K|V)",
     r"tile_gemm_kernel<0, 0,"),
    ("tile GEMM int8, RESID (stacked o, down without split-K)", r"tile_gemm_kernel<0, 1,"),
    ("split-K plane sum + epilogue (stacked o, down: RESID)", r"tile_reduce_kernel"),
    ("tile GEMM int8, SWIGLU (stacked gate|up)", r"tile_gemm_kernel<0, 2,"),
    ("tile GEMM fp16, ARGMAX (stacked lm_head)", r"tile_gemm_kernel<1, 3,"),
    ("tile GEMM fp16, fp32 rows (prompt-sized ingest fc)", r"tile_gemm_kernel<1, 0, 2,"),
    ("tile GEMM fp16 128x128 (the fc's last round, re-tiled)", r"tile_gemm_kernel<1, 0, 1,"),
    ("rows into fragment layout (ingest input, fused-rows ingest)", r"feats_to_afl_kernel"),
    ("argmax of the partial keys (stacked lm_head)", r"argmax_parts_kernel"),
    ("fc rows: fp16 rounding + hidden_norm (prompt-sized ingest)", r"fc_norm_rows_kernel"),
    ("RMSNorm rows (stacked blocks)", r"afl_rows_kernel"),
    ("block attention", r"block_attn_kernel"),
    ("attention merge", r"attn_merge_kernel"),
    ("qk norm + rope (context ingest, stacked blocks)", r"qk_rope_kernel"),
    ("RoPE angle table (prompt-sized ingest)", r"rope_table_kernel"),
    ("embed + norm", r"embed_norm_kernel"),
    ("argmax finalize", r"argmax_finalize_kernel"),
]
COPY_RE = r"bitwise_not"


def read_stats(path):
    rows = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            rows[r["Name"]] = (int(r["Calls"]), float(r["TotalDurationNs"]))
    return rows


def read_trace(path, skip_blocks, block_rx, from_rx=None, from_index=0, until_rx=None,
               until_back=0):
    """(calls, total ns) per kernel name from a kernel trace, leaving out the dispatches
    from the first draft block's start (a dispatch matching block_rx) to the start of
    block skip_blocks + 1; dispatches before the first block (context ingest) are kept.
    With from_rx, every dispatch before the from_index-th (0-based) one matching from_rx
    is left out first; with until_rx, the first dispatch after that point matching until_rx,
    the until_back dispatches before it and everything after it are left out too."""
    with open(path) as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    if from_rx:
        hits = [i for i, r in enumerate(rows) if re.search(from_rx, r["Kernel_Name"])]
        rows = rows[hits[from_index]:] if from_index < len(hits) else []
    if until_rx:
        hits = [i for i, r in enumerate(rows) if re.search(until_rx, r["Kernel_Name"])]
        if hits:
            rows = rows[:max(0, hits[0] - until_back)]
    starts = [i for i, r in enumerate(rows) if re.search(block_rx, r["Kernel_Name"])]
    lo = hi = 0
    if skip_blocks > 0 and starts:
        lo = starts[0]
        hi = starts[skip_blocks] if skip_blocks < len(starts) else len(rows)
    stats = {}
    for i, r in enumerate(rows):
        if lo <= i < hi:
            continue
        c, t = stats.get(r["Kernel_Name"], (0, 0.0))
        stats[r["Kernel_Name"]] = (c + 1, t + int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    return stats


def read_counter(path):
    per = collections.defaultdict(list)
    with open(path) as f:
        for r in csv.DictReader(f):
            per[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    return per


def read_counters(path):
    """{kernel: [ {counter: value, "_ns": duration} per dispatch ]}"""
    disp = collections.defaultdict(dict)
    with open(path) as f:
        for r in csv.DictReader(f):
            d = disp[(r["Kernel_Name"], r["Dispatch_Id"])]
            d[r["Counter_Name"]] = float(r["Counter_Value"])
            d["_ns"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    per = collections.defaultdict(list)
    for (k, _), d in disp.items():
        per[k].append(d)
    return per


def match(names, rx):
    return [n for n in names if re.search(rx, n)]


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--stats")
    ap.add_argument("--trace")
    ap.add_argument("--skip-blocks", type=int, default=0)
    ap.add_argument("--block-start", default=r"embed_norm_kernel",
                    help="regex of the first kernel of a draft block (trace mode)")
    ap.add_argument("--from-kernel", default=None,
                    help="trace mode: drop every dispatch before the --from-index-th one "
                         "whose name matches this regex")
    ap.add_argument("--from-index", type=int, default=0)
    ap.add_argument("--until-kernel", default=None,
                    help="trace mode: drop the first dispatch (after --from-kernel's) whose "
                         "name matches this regex, the --until-back dispatches before it and "
                         "everything after it")
    ap.add_argument("--until-back", type=int, default=0)
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--mfma")
    ap.add_argument("--copy-mib", type=int, default=1024)
    ap.add_argument("--workload", required=True)
    ap.add_argument("--commands", default="", help="text of the commands that made the inputs")
    ap.add_argument("--note", default="", help="a line describing the run")
    ap.add_argument("--md", required=True)
    ap.add_argument("--json")
    a = ap.parse_args(argv)

    if bool(a.stats) == bool(a.trace):
        print("pass exactly one of --stats / --trace", file=sys.stderr)
        return 2
    stats = read_stats(a.stats) if a.stats else read_trace(a.trace, a.skip_blocks, a.block_start,
                                                             a.from_kernel, a.from_index,
                                                             a.until_kernel, a.until_back)
    out = [f"# rocprofv3 summary: {a.workload} draft block", ""]
    if a.note:
        out += [a.note, ""]
    if a.commands:
        out += ["Commands:", "", "```", a.commands.strip(), "```", ""]
    head = ("## Kernel durations (--kernel-trace --stats)" if a.stats else
            f"## Kernel durations (--kernel-trace; the {a.skip_blocks} warmup blocks left out)"
            if not a.from_kernel else
            f"## Kernel durations (--kernel-trace; from dispatch {a.from_index} of "
            f"{a.from_kernel} on" + (f", up to the first {a.until_kernel} less "
                                      f"{a.until_back}" if a.until_kernel else "") + ")")
    out += [head, "",
            "| group | calls | avg us | total ms |", "|---|---:|---:|---:|"]
    for label, rx in GROUPS:
        ns = match(stats, rx)
        if not ns:
            continue
        calls = sum(stats[n][0] for n in ns)
        tot = sum(stats[n][1] for n in ns)
        out.append(f"| {label} | {calls} | {tot / calls / 1e3:.2f} | {tot / 1e6:.3f} |")
    out.append("")

    traffic = {}
    if a.fetch and a.write:
        fetch, write = read_counter(a.fetch), read_counter(a.write)
        copy_bytes = a.copy_mib << 20
        fc = [v for n in match(fetch, COPY_RE) for v in fetch[n]]
        wc = [v for n in match(write, COPY_RE) for v in write[n]]
        if not fc or not wc:
            print("copy probe kernel not found in the counter runs", file=sys.stderr)
            return 1
        f_scale = copy_bytes / (sum(fc) / len(fc))   # bytes per unit of FETCH_SIZE
        w_scale = copy_bytes / (sum(wc) / len(wc))
        out += ["## HBM traffic per dispatch (--pmc FETCH_SIZE, --pmc WRITE_SIZE)", "",
                f"Calibration: an elementwise copy of {a.copy_mib} MiB reads FETCH_SIZE "
                f"{sum(fc) / len(fc):.1f} and WRITE_SIZE {sum(wc) / len(wc):.1f}; scale factors "
                f"{f_scale / 1024:.3f} KiB per FETCH_SIZE unit, {w_scale / 1024:.3f} KiB per "
                f"WRITE_SIZE unit.", "",
                "| group | dispatches | read MB | written MB | total MB |", "|---|---:|---:|---:|---:|"]
        for label, rx in GROUPS:
            fv = [v for n in match(fetch, rx) for v in fetch[n]]
            wv = [v for n in match(write, rx) for v in write[n]]
            if not fv or not wv:
                continue
            rd = sum(fv) / len(fv) * f_scale
            wr = sum(wv) / len(wv) * w_scale
            out.append(f"| {label} | {len(fv)} | {rd / 1e6:.2f} | {wr / 1e6:.2f} | "
                       f"{(rd + wr) / 1e6:.2f} |")
            traffic[label] = {"read_bytes": rd, "write_bytes": wr, "bytes_per_launch": rd + wr}
        out.append("")
    if a.mfma:
        mf = read_counters(a.mfma)
        out += ["## Matrix cores (--pmc MfmaUtil MfmaFlopsF16)", "",
                "MfmaUtil: MFMA-busy cycles over the active cycles of every SIMD of the GPU, in "
                "percent (rocprofv3's derived metric). fp16 MFMA TFLOP/s: MfmaFlopsF16 (fp16 MFMA "
                "operations of the dispatch) over its duration in the counter run; dense fp16 "
                "peak 2500 TFLOP/s.", "",
                "| group | dispatches | MfmaUtil % | fp16 MFMA TFLOP/s | % of peak |",
                "|---|---:|---:|---:|---:|"]
        for label, rx in GROUPS:
            ds = [d for n in match(mf, rx) for d in mf[n] if "MfmaUtil" in d]
            if not ds:
                continue
            util = sum(d["MfmaUtil"] for d in ds) / len(ds)
            tf = sum(d.get("MfmaFlopsF16", 0.0) / max(d["_ns"], 1) / 1e3 for d in ds) / len(ds)
            out.append(f"| {label} | {len(ds)} | {util:.1f} | {tf:.1f} | {tf / 2500 * 100:.1f} |")
        out.append("")
    with open(a.md, "w") as f:
        f.write("\n".join(out) + "\n")
    if a.json and traffic:
        doc = {"workload": a.workload,
               "gemm_w8a16": traffic.get("proj_gemm_w8a16"),
               "lm_head": traffic.get("lm_head (fp16, ARGMAX, norm-on-load)"),
               "attention": traffic.get("block attention")}
        with open(a.json, "w") as f:
            json.dump(doc, f, indent=1)
            f.write("\n")
    print("\n".join(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
