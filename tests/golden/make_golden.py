#!/usr/bin/env python3
"""Write the golden fixtures of the attention step (tests/golden/*.npz).

Each fixture holds one seeded workload (q, the K/V cache, geometry) and the
output of the oracle's scalar emulation of the reference's emitted SDPA on
it. The reference ships no fixtures of its own (it has no tests); these pin
the oracle against regressions, and the GPU tests compare the HIP path with
them without running the oracle.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "herbert-jit-bf16_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import oracle  # noqa: E402
from hsdpa import workloads as W  # noqa: E402

# name, heads, kv_heads, head_dim, rows, past, seed, extra
FIXTURES = [
    ("decode_n1_d256", 8, 2, 256, 1, 0, 101, {}),
    ("decode_n37_d256", 8, 2, 256, 1, 36, 102, {}),
    ("decode_n150_d128_g4", 16, 4, 128, 1, 149, 103, {}),
    ("decode_n129_d64_g1", 4, 4, 64, 1, 128, 104, {}),
    ("decode_n300_d256_outliers", 16, 2, 256, 1, 299, 105, dict(outlier_keys=4, outlier_rows_frac=0.01)),
    ("prefill_r8_p0_d256", 8, 2, 256, 8, 0, 106, {}),
    ("prefill_r19_p37_d256", 8, 2, 256, 19, 37, 107, {}),
    ("prefill_r40_p5_d128_g1", 8, 8, 128, 40, 5, 108, {}),
    ("prefill_r33_p100_d64_g2", 8, 4, 64, 33, 100, 109, {}),
    ("prefill_r2_p1_d256_g3", 6, 2, 256, 2, 1, 110, {}),
]


def make(name, h, kvh, d, rows, past, seed, extra):
    w = W.make(name, heads=h, kv_heads=kvh, head_dim=d, rows=rows, past=past, seed=seed, **extra)
    out = oracle.attention(w, "scalar")
    return w, out


def main():
    for name, h, kvh, d, rows, past, seed, extra in FIXTURES:
        w, out = make(name, h, kvh, d, rows, past, seed, extra)
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, q=w.q, k=w.k, v=w.v, out=out,
                            geometry=np.array([w.heads, w.kv_heads, w.head_dim, w.rows, w.past, w.capacity],
                                              dtype=np.int64),
                            scale=np.float32(w.scale))
        print(path, os.path.getsize(path))


if __name__ == "__main__":
    main()
