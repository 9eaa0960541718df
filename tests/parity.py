"""The parity criterion of the attention step, shared by the tests.

Two outputs agree when at least 99.9 % of the bf16 elements are within one
ulp (distance <= 1 in the ordered-bits integer order, +0 and -0 equal) and,
for every output row, max |out - ref| <= 2^-6 * max |V| over the keys that
row sees.
"""
from __future__ import annotations

import numpy as np

ULP_SHARE = 0.999
ABS_FACTOR = 2.0 ** -6


def ordered(b: np.ndarray) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint16).astype(np.int32)
    return np.where(b & 0x8000, -(b & 0x7FFF), b)


def bf16_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def row_vmax(w) -> np.ndarray:
    """max |V| over the visible keys of each (row, head): [rows][heads]."""
    vabs = np.abs(bf16_f32(w.v))                      # [kvh][cap][d]
    per_pos = vabs.max(axis=2)                        # [kvh][cap]
    run = np.maximum.accumulate(per_pos, axis=1)      # prefix max over positions
    out = np.empty((w.rows, w.heads), dtype=np.float32)
    for h in range(w.heads):
        kvh = h // w.gqa
        out[:, h] = run[kvh, w.past + np.arange(w.rows)]
    return out


def compare(out: np.ndarray, ref: np.ndarray, w) -> dict:
    out = np.asarray(out, dtype=np.uint16).reshape(w.rows, w.heads, w.head_dim)
    ref = np.asarray(ref, dtype=np.uint16).reshape(w.rows, w.heads, w.head_dim)
    dist = np.abs(ordered(out) - ordered(ref))
    share = float((dist <= 1).mean())
    err = np.abs(bf16_f32(out).astype(np.float64) - bf16_f32(ref).astype(np.float64)).max(axis=2)
    ratio = float((err / row_vmax(w)).max())
    return {"ulp1_share": share, "max_abs_over_vmax": ratio, "max_ulp": int(dist.max()),
            "exact_share": float((dist == 0).mean()), "nan": bool(np.isnan(bf16_f32(out)).any())}


def assert_parity(out, ref, w, tag=""):
    r = compare(out, ref, w)
    assert not r["nan"], f"{tag}: NaN in output {r}"
    assert r["ulp1_share"] >= ULP_SHARE, f"{tag}: only {r['ulp1_share']:.5%} within 1 ulp {r}"
    assert r["max_abs_over_vmax"] <= ABS_FACTOR, f"{tag}: max abs error too large {r}"
    return r
