"""Seeded synthetic inputs for the attention step, in the engine's layouts.

The reference engine has no input generator of its own, so this one is
defined here and used by the tests, the smoke check and the benchmark:
SplitMix64(seed) -> Box-Muller N(0,1) in f64 -> f32 -> bf16 (round to nearest
even). q, k and v use independent streams (seed, seed+1, seed+2).

Layouts follow the engine:
  q, out : token-major [rows][heads][head_dim]  (q_row = heads*head_dim,
           q_head = head_dim; src/jit/schedule.rs:184-202)
  K, V   : head-major cache [kv_heads][capacity][head_dim], position p of
           head h at h*capacity*head_dim + p*head_dim
           (src/jit/model.rs:340-366, src/jit/execution/abi.rs:156-180)
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, count: int, offset: int = 0) -> np.ndarray:
    """`count` outputs of SplitMix64 seeded with `seed`, starting at `offset`."""
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + count + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round f32 to bf16 bits, nearest even (src/jit/model.rs:904-908)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((b + np.uint64(0x7FFF) + ((b >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal_f32(seed: int, count: int, chunk: int = 1 << 24) -> np.ndarray:
    """N(0,1) as f32 by Box-Muller on pairs of 24-bit uniforms in (0, 1]."""
    out = np.empty(count, dtype=np.float32)
    pairs = (count + 1) // 2
    for p0 in range(0, pairs, chunk):
        n = min(chunk, pairs - p0)
        z = splitmix64(seed, 2 * n, 2 * p0)
        u = ((z >> np.uint64(40)).astype(np.float64) + 1.0) * (1.0 / (1 << 24))
        r = np.sqrt(-2.0 * np.log(u[0::2]))
        t = 2.0 * math.pi * u[1::2]
        pair = np.empty(2 * n, dtype=np.float64)
        pair[0::2] = r * np.cos(t)
        pair[1::2] = r * np.sin(t)
        lo = 2 * p0
        hi = min(count, lo + 2 * n)
        out[lo:hi] = pair[: hi - lo].astype(np.float32)
    return out


def normal_bf16(seed: int, shape) -> np.ndarray:
    return f32_to_bf16(normal_f32(seed, int(np.prod(shape)))).reshape(shape)


def _distinct(seed: int, k: int, n: int) -> np.ndarray:
    """k distinct indices in [0, n) from a partial Fisher-Yates on SplitMix64."""
    perm = np.arange(n, dtype=np.int64)
    z = splitmix64(seed, k)
    for i in range(k):
        j = i + int(z[i] % np.uint64(n - i))
        perm[i], perm[j] = perm[j], perm[i]
    return np.sort(perm[:k])


@dataclasses.dataclass
class Workload:
    """One attention call: the per-layer geometry and the seeded buffers."""

    name: str
    heads: int
    kv_heads: int
    head_dim: int
    rows: int
    past: int
    capacity: int
    q: np.ndarray      # uint16 [rows][heads][head_dim]
    k: np.ndarray      # uint16 [kv_heads][capacity][head_dim]
    v: np.ndarray      # uint16 [kv_heads][capacity][head_dim]
    scale: float

    @property
    def gqa(self) -> int:
        return self.heads // self.kv_heads

    @property
    def q_row(self) -> int:
        return self.heads * self.head_dim

    @property
    def out_row(self) -> int:
        return self.heads * self.head_dim

    @property
    def kv_stride(self) -> int:
        return self.capacity * self.head_dim

    def decode_bytes(self) -> int:
        """Algorithmic HBM bytes of a decode call: K and V read once, q read, out written."""
        n = self.past + self.rows
        return 2 * self.kv_heads * n * self.head_dim * 2 + 2 * self.heads * self.head_dim * 2 * self.rows

    def prefill_flops(self) -> int:
        """4*Hq*d*sum_i(past+i+1): the causally visible (query, key) pairs only."""
        m, p = self.rows, self.past
        return 4 * self.heads * self.head_dim * (m * p + m * (m + 1) // 2)


def make(name: str, heads: int, kv_heads: int, head_dim: int, rows: int, past: int,
         seed: int = 0, capacity: int | None = None, scale: float | None = None,
         outlier_keys: int = 0, outlier_key_scale: float = 20.0,
         outlier_rows_frac: float = 0.0, outlier_row_scale: float = 8.0) -> Workload:
    """Seeded inputs. The cache holds past+rows positions (the chunk's K/V are
    already appended), padded with zeros up to `capacity`."""
    n = past + rows
    cap = n if capacity is None else capacity
    if cap < n:
        raise ValueError("capacity below past + rows")
    q = normal_bf16(seed, (rows, heads, head_dim))
    kf = normal_f32(seed + 1, kv_heads * n * head_dim).reshape(kv_heads, n, head_dim)
    vf = normal_f32(seed + 2, kv_heads * n * head_dim).reshape(kv_heads, n, head_dim)
    if outlier_keys:
        for h in range(kv_heads):
            ch = _distinct(seed + 3 + 16 * h, outlier_keys, head_dim)
            kf[h][:, ch] *= np.float32(outlier_key_scale)
    if outlier_rows_frac > 0.0:
        cnt = int(math.ceil(outlier_rows_frac * n))
        for h in range(kv_heads):
            rows_sel = _distinct(seed + 4 + 16 * h, cnt, n)
            vf[h][rows_sel, :] *= np.float32(outlier_row_scale)
    k = np.zeros((kv_heads, cap, head_dim), dtype=np.uint16)
    v = np.zeros((kv_heads, cap, head_dim), dtype=np.uint16)
    k[:, :n] = f32_to_bf16(kf)
    v[:, :n] = f32_to_bf16(vf)
    del kf, vf
    s = (1.0 / math.sqrt(head_dim)) if scale is None else scale
    return Workload(name, heads, kv_heads, head_dim, rows, past, cap, q, k, v, float(np.float32(s)))


# The five configurations of the benchmark: two decode shapes, two causal
# prefill shapes, one long-context decode with outlier keys and values.
CONFIGS = {
    "decode_1k": dict(heads=8, kv_heads=2, head_dim=256, rows=1, past=1023),
    "decode_32k": dict(heads=16, kv_heads=2, head_dim=256, rows=1, past=32767),
    "prefill_512": dict(heads=16, kv_heads=4, head_dim=256, rows=512, past=0),
    "prefill_4096_after_8192": dict(heads=16, kv_heads=2, head_dim=256, rows=4096, past=8192),
    "decode_128k_outliers": dict(heads=16, kv_heads=2, head_dim=256, rows=1, past=131071,
                                 outlier_keys=4, outlier_rows_frac=0.01),
}


def config(name: str, seed: int = 0, **over) -> Workload:
    kw = dict(CONFIGS[name])
    kw.update(over)
    return make(name, seed=seed, **kw)
