"""Build libhsdpa.so (the C ABI and its gfx950 kernels) in-tree with hipcc.

    python build.py            # compile
    python build.py --asm      # also keep the gfx950 assembly next to the sources

The library lands in hsdpa/libhsdpa.so, next to the Python binding.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "hsdpa", "libhsdpa.so")
SOURCES = ["hsdpa_kernels.hip", "hsdpa_api.cpp"]
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

# -ffp-contract=off: the exponential and the score scaling must round exactly
# as written; -packed-fp32-ops: no packed f32 arithmetic is emitted.
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wall", "-Wno-unused-function", "-I", os.path.join(ROOT, "include"), "-I", SRC]


def build(asm: bool = False, verbose: bool = False) -> str:
    tmp = OUT + ".tmp"
    cmd = [HIPCC] + FLAGS + ["-shared", "-o", tmp] + [os.path.join(SRC, s) for s in SOURCES]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "unknown target feature"
    err = "\n".join(line for line in r.stderr.splitlines() if noise not in line and "-packed-fp32-ops" not in line)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    os.replace(tmp, OUT)
    if asm:
        d = os.path.join(HERE, "_asm")
        os.makedirs(d, exist_ok=True)
        subprocess.run([HIPCC] + FLAGS + ["--cuda-device-only", "-S", "-o", os.path.join(d, "hsdpa_kernels.s"),
                                          os.path.join(SRC, "hsdpa_kernels.hip")], check=True)
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--asm", action="store_true")
    args = ap.parse_args()
    print(build(asm=args.asm, verbose=True))
