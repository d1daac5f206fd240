"""Build libslo_attn.so in-tree for gfx950 with hipcc (no JIT, no cmake).

Usage: python build.py [--jobs N]
The library lands next to the Python host layer (slo_attn/libslo_attn.so) so
that it travels with the source tree.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "slo_attn")
LIB = os.path.join(OUT_DIR, "libslo_attn.so")
SOURCES = ["store_kv.hip", "qk_norm_rope.hip", "lm_head.hip", "metadata.hip", "paged_attention.hip", "capi.cpp"]
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    # Packed fp32 VALU forms are kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Work-list fetches and split-K tickets are single-lane atomics whose
    # results are consumed late on purpose; the atomic optimizer's wave-level
    # rewrite would read them back immediately and stall the loads in flight.
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-I", os.path.join(HERE, "..", "include"),
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found")
    return path


# Kernels whose every instantiation must keep its registers out of scratch
# memory (a spill there puts per-lane memory traffic into the tile loops).
NO_SCRATCH = {"paged_attention.hip"}


def _compile(src: str, obj: str) -> None:
    extra = ["-Rpass-analysis=kernel-resource-usage"] if src in NO_SCRATCH else []
    cmd = [hipcc(), *FLAGS, *extra, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed on {src}")
    if extra:
        spills = [ln for ln in res.stderr.splitlines()
                  if "ScratchSize [bytes/lane]:" in ln and not ln.rstrip().split("ScratchSize [bytes/lane]:")[1]
                  .split()[0] == "0"]
        if spills:
            raise RuntimeError(f"{src}: a kernel instantiation uses scratch memory:\n" + "\n".join(spills))


def build(jobs: int = 4) -> str:
    obj_dir = os.path.join(HERE, "_build")
    os.makedirs(obj_dir, exist_ok=True)
    objs = [os.path.join(obj_dir, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        list(pool.map(lambda so: _compile(*so), zip(SOURCES, objs)))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("link failed")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    print(build(ap.parse_args().jobs))
