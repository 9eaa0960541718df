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
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "hsdpa", "libhsdpa.so")
# translation units, compiled in parallel and linked: the tuned attention
# kernels and the element kernels, the attention kernels of the other head
# dimensions, the decode passes under the Fused form, the short-chunk
# prefill, the static scratch of the entry point that allocates nothing, the
# decode passes of frame calls (rows and past read at run time), the causal
# prefill with the softmax sink, the C ABI
SOURCES = ["hsdpa_kernels.hip", "hsdpa_attn_more.hip", "hsdpa_fused.hip", "hsdpa_prefill_short.hip",
           "hsdpa_static.hip", "hsdpa_frame.hip", "hsdpa_sink.hip", "hsdpa_api.cpp"]
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

# -ffp-contract=off: the exponential and the score scaling must round exactly
# as written; -packed-fp32-ops: no packed f32 arithmetic is emitted.
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wall", "-Wno-unused-function", "-I", os.path.join(ROOT, "include"), "-I", SRC]


def _errors(stderr: str) -> str:
    # hipcc's host pass warns that it does not know the packed-fp32 feature
    return "\n".join(line for line in stderr.splitlines()
                     if "unknown target feature" not in line and "-packed-fp32-ops" not in line)


def build(asm: bool = False, verbose: bool = False) -> str:
    tmp = OUT + ".tmp"
    with tempfile.TemporaryDirectory(prefix="hsdpa_build_") as objdir:
        objs, procs = [], []
        for src in SOURCES:
            obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
            cmd = [HIPCC] + FLAGS + ["-c", "-o", obj, os.path.join(SRC, src)]
            if verbose:
                print(" ".join(cmd), flush=True)
            objs.append(obj)
            procs.append(subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True))
        failed = []
        for src, p in zip(SOURCES, procs):
            _, stderr = p.communicate()
            err = _errors(stderr)
            if p.returncode != 0:
                failed.append(f"{src} ({p.returncode}):\n{err}")
            elif err.strip() and verbose:
                print(err, file=sys.stderr)
        if failed:
            raise RuntimeError("hipcc failed: " + "\n".join(failed))
        cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc link failed ({r.returncode}):\n{_errors(r.stderr)}")
    os.replace(tmp, OUT)
    if asm:
        d = os.path.join(HERE, "_asm")
        os.makedirs(d, exist_ok=True)
        for src in SOURCES:
            if src.endswith(".hip"):
                out = os.path.join(d, os.path.splitext(src)[0] + ".s")
                subprocess.run([HIPCC] + FLAGS + ["--cuda-device-only", "-S", "-o", out, os.path.join(SRC, src)],
                               check=True)
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--asm", action="store_true")
    args = ap.parse_args()
    print(build(asm=args.asm, verbose=True))
