"""Build libattnres_hip.so (gfx950) in-tree from lr-attnres_amd/csrc/*.hip.

    python lr-attnres_amd/build.py [--arch gfx950] [--jobs 4]

Each translation unit is compiled with hipcc in parallel, then linked into one
shared library next to this file.  Packed-fp32 instruction selection is
switched off (-packed-fp32-ops) for every device compile.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libattnres_hip.so")

SOURCES = ["attnres_capi.hip", "attnres_lr.hip", "attnres_lr_fast_fwd.hip", "attnres_lr_fast_bwd.hip",
           "attnres_base.hip", "attnres_base_bwd.hip",
           "attnres_base_fast_fwd.hip", "attnres_base_fast_bwd.hip", "attnres_phase1.hip", "attnres_phase1_fast.hip", "attnres_phase2.hip", "attnres_phase2_fast.hip", "attnres_keysplit.hip",
           "attnres_keyed_logits.hip", "attnres_value_key.hip", "attnres_site_logits.hip"]

DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.isabs(cand) and os.path.exists(cand) or not os.path.isabs(cand)):
            return cand
    return "hipcc"


def compile_one(src: str, arch: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [_hipcc(), f"--offload-arch={arch}", "-O3", "-std=c++17", "-fPIC", "-c",
           "-Wno-unused-command-line-argument", *DEVICE_FLAGS,
           "-I", os.path.join(HERE, "..", "include"), os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(arch: str = "gfx950", jobs: int = 4, verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(lambda s: compile_one(s, arch), SOURCES))
    tmp = LIB + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={arch}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--arch", default="gfx950")
    ap.add_argument("--jobs", type=int, default=4)
    a = ap.parse_args()
    try:
        build(a.arch, a.jobs, verbose=True)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
