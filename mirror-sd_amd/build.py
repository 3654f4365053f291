"""Build libdflash_hip.so (gfx950) from csrc/*.hip with hipcc.

Usage: python build.py [--jobs N] [--debug]

Each translation unit is compiled separately (in parallel) into _build/ and linked
into mirror_sd_amd/libdflash_hip.so next to the Python host package.  Packed FP32
instructions are disabled for all device code (-target-feature -packed-fp32-ops).
"""

from __future__ import annotations

import argparse
import glob
import json
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "mirror_sd_amd", "libdflash_hip.so")
# Per-kernel register, scratch, LDS and occupancy figures of the last build (the compiler's
# kernel-resource-usage remarks), one record per kernel symbol.
RESOURCES = os.path.join(BUILD, "kernel_resources.json")
_USAGE_FLAG = "-Rpass-analysis=kernel-resource-usage"
ARCH = os.environ.get("DFL_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for c in (os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc"),
              shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found (set ROCM_PATH)")


def common_flags(debug: bool):
    f = [f"--offload-arch={ARCH}", "-std=c++17", "-fPIC", "-I", INCLUDE, "-I", CSRC,
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wno-unused-result"]
    f += ["-O1", "-g"] if debug else ["-O3"]
    return f


# The packed-FP32 guard (-target-feature -packed-fp32-ops) reaches hipcc's host (x86) pass
# too, which reports it as an unknown feature on every compile; hipcc cannot scope -Xclang
# arguments to the device pass (-Xarch_device refuses them), so that one line is dropped and
# every other compiler message is shown.
_HOST_FEATURE_NOTE = "'-packed-fp32-ops' is not a recognized feature for this target"


def compiler_messages(text: str) -> str:
    """Compiler output minus the host feature note and the resource-usage remarks (with the
    source-snippet lines printed under each remark)."""
    keep, in_remark = [], False
    for l in text.splitlines():
        if _USAGE_FLAG in l:
            in_remark = True
            continue
        gutter, bar, _ = l.partition("|")
        if in_remark and bar and (not gutter.strip() or gutter.strip().isdigit()):
            continue   # "  23 | source" and "     | ^" under the remark
        in_remark = False
        if l.strip() and _HOST_FEATURE_NOTE not in l and "--hip-link" not in l:
            keep.append(l)
    return "\n".join(keep)


def resource_usage(text: str) -> dict:
    """Parse the kernel-resource-usage remarks ("Function Name: f" followed by "Key: value"
    lines) into {kernel: {key: value}}; numeric values become ints."""
    out, cur = {}, None
    for line in text.splitlines():
        if _USAGE_FLAG not in line or "remark:" not in line:
            continue
        body = line.split("remark:", 1)[1].split("[" + _USAGE_FLAG, 1)[0].strip()
        key, _, val = body.partition(":")
        val = val.strip()
        if key == "Function Name":
            cur = out.setdefault(val, {})
        elif cur is not None:
            cur[key.strip()] = int(val) if val.lstrip("-").isdigit() else val
    return out


def compile_one(src: str, debug: bool):
    obj = os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o"))
    cmd = [hipcc(), *common_flags(debug), _USAGE_FLAG, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    msgs = compiler_messages(r.stdout + "\n" + r.stderr)
    if msgs:
        print(f"{os.path.basename(src)}:\n{msgs}", file=sys.stderr)
    return obj, resource_usage(r.stdout + "\n" + r.stderr)


def build(jobs: int = 8, debug: bool = False, verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        done = list(ex.map(lambda s: compile_one(s, debug), srcs))
    objs = [o for o, _ in done]
    usage = {k: v for _, u in done for k, v in u.items()}
    with open(RESOURCES, "w") as f:
        json.dump(usage, f, indent=1, sort_keys=True)
    spills = sorted(k for k, v in usage.items() if v.get("ScratchSize [bytes/lane]", 0))
    if spills and not debug:
        print(f"warning: kernels using scratch (register spills): {spills}", file=sys.stderr)
    tmp = OUT + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {len(srcs)} sources")
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--debug", action="store_true")
    args = ap.parse_args()
    try:
        build(args.jobs, args.debug)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
