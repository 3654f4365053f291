"""Build libdflash_hip.so (gfx950) from csrc/*.hip with hipcc.

Usage: python build.py [--jobs N] [--debug]

Each translation unit is compiled separately (in parallel) into _build/ and linked
into mirror_sd_amd/libdflash_hip.so next to the Python host package.  Packed FP32
instructions are disabled for all device code (-target-feature -packed-fp32-ops).
"""

from __future__ import annotations

import argparse
import glob
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
    return "\n".join(l for l in text.splitlines()
                     if l.strip() and _HOST_FEATURE_NOTE not in l and "--hip-link" not in l)


def compile_one(src: str, debug: bool) -> str:
    obj = os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o"))
    cmd = [hipcc(), *common_flags(debug), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    msgs = compiler_messages(r.stdout + "\n" + r.stderr)
    if msgs:
        print(f"{os.path.basename(src)}:\n{msgs}", file=sys.stderr)
    return obj


def build(jobs: int = 8, debug: bool = False, verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(lambda s: compile_one(s, debug), srcs))
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
