"""A seeded sweep over shapes, through the C ABI, against the oracle.

The named cases elsewhere pin each kernel at the shapes chosen for it; this
sweep draws 80 calls at random (fixed seed) over group shapes (1 to 80 query
heads per KV head), every kind of head_dim the reference accepts (32 to 512),
1 to 512 rows after 0 to 12 000 cached positions, and 24 more of up to 8 rows
after 12 000 to 131 071 positions, under both decode forms
(sdpa_form Chained and Fused, src/jit/target/x86/emit_sdpa/x86/decode.rs:
212-293 and 501-669), so that routing and kernel choices meet shapes nobody
picked. The host test checks, without a GPU, that the draw still reaches
every route class it reached when it was written (a change of the selector
that narrows it shows here); the GPU test compares every call with the
oracle, the one-ulp share pooled over the calls as small shapes need.
"""
import numpy as np
import pytest

import hsdpa
import oracle
from hsdpa import workloads as W
from parity import ABS_FACTOR, ULP_SHARE, compare

from gpu_util import run_hsdpa

GROUPS = [(8, 2), (16, 2), (16, 4), (12, 1), (32, 1), (6, 3), (34, 2), (24, 2), (4, 4), (48, 1), (10, 2), (64, 4),
          (80, 1)]
DIMS = [64, 128, 256, 256, 128, 32, 96, 160, 512]
ROWS = [1, 1, 1, 1, 2, 3, 5, 8, 9, 16, 17, 31, 33, 64, 100, 257, 512]
SEED = 20261202
COUNT = 80
MAX_WORK = 4e8          # rows x keys x heads x head_dim: the oracle takes well under a second


def _draw():
    rng = np.random.default_rng(SEED)
    out = []
    while len(out) < COUNT:
        h, kvh = GROUPS[rng.integers(len(GROUPS))]
        d = int(DIMS[rng.integers(len(DIMS))])
        rows = int(ROWS[rng.integers(len(ROWS))])
        past = int([0, rng.integers(1, 64), rng.integers(64, 1100), rng.integers(1100, 12000)][rng.integers(4)])
        form = "fused" if rng.random() < 0.3 else "chained"
        if rows * (past + rows) * h * d > MAX_WORK:
            continue
        out.append((f"s{len(out):02d}_h{h}k{kvh}_d{d}_r{rows}_p{past}_{form}", h, kvh, d, rows, past, form))
    return out


CASES = _draw()

# long caches: 12 000 to 131 071 positions, up to 8 rows (the decode and
# few-rows kernels' tile loops, chunked pass 2 and all-group forms)
LONG_DIMS = [64, 128, 256, 256, 96, 512]
LONG_ROWS = [1, 1, 1, 2, 3, 4, 5, 8]
LONG_COUNT = 24
LONG_MAX_WORK = 6e8


def _draw_long():
    rng = np.random.default_rng(SEED + 1)
    out = []
    while len(out) < LONG_COUNT:
        h, kvh = GROUPS[rng.integers(len(GROUPS))]
        d = int(LONG_DIMS[rng.integers(len(LONG_DIMS))])
        rows = int(LONG_ROWS[rng.integers(len(LONG_ROWS))])
        past = int(rng.integers(12000, 131072))
        form = "fused" if rng.random() < 0.3 else "chained"
        if rows * (past + rows) * h * d > LONG_MAX_WORK:
            continue
        out.append((f"l{len(out):02d}_h{h}k{kvh}_d{d}_r{rows}_p{past}_{form}", h, kvh, d, rows, past, form))
    return out


LONG_CASES = _draw_long()

# (main kernels, main numerics, tail kernels, launches, split over keys) that
# the draw reaches
REACHED = {
    ("causal", "chained", "decode_rows", 13, False),
    ("causal", "chained", "decode", 3, False),
    ("causal", "chained", "decode", 4, False),
    ("causal", "chained", "few_rows", 4, False),
    ("causal", "chained", "none", 1, False),
    ("causal_short", "chained", "none", 1, False),
    ("causal_split", "chained", "decode", 6, True),
    ("causal_split", "chained", "few_rows", 6, True),
    ("causal_split", "chained", "none", 3, True),
    ("decode", "chained", "none", 2, False),
    ("decode", "chained", "none", 3, False),
    ("decode", "fused", "none", 2, False),
    ("decode", "fused", "none", 3, False),
    ("few_rows", "chained", "none", 2, False),
    ("few_rows", "chained", "none", 3, False),
    ("few_rows", "fused", "none", 3, False),
}
REACHED_LONG = {
    ("causal_split", "chained", "none", 3, True),
    ("decode", "chained", "none", 3, False),
    ("decode", "fused", "none", 3, False),
    ("few_rows", "chained", "none", 3, False),
    ("few_rows", "fused", "none", 3, False),
}


def _plan(h, kvh, d, rows, past, form):
    return hsdpa.Plan(h, h // kvh, d, past + rows, form=form)


def _route_class(r):
    return (r["main"], r["main_form"], r["tail"], r["launches"], r["splits"] > 1)


@pytest.mark.parametrize("cases,reached", [(CASES, REACHED), (LONG_CASES, REACHED_LONG)], ids=["short", "long"])
def test_sweep_reaches_every_route_class(cases, reached):
    seen = set()
    for _, h, kvh, d, rows, past, form in cases:
        seen.add(_route_class(_plan(h, kvh, d, rows, past, form).route(rows, past)))
    assert reached <= seen, sorted(reached - seen)


@pytest.mark.gpu
@pytest.mark.parametrize("cases,seed0", [(CASES, 31), (LONG_CASES, 131)], ids=["short", "long"])
def test_sweep_parity(torch_cuda, cases, seed0):
    """Each call: no NaN, the per-row bound max |out - ref| <= 2^-6 max |V|;
    a call of at least 4096 outputs at least 99.9 % of them within one ulp,
    a smaller one at most max(2, 1 %) past one ulp (a call of 128 outputs
    cannot show a 99.9 % share, a wrong kernel misses by far more); over the
    calls together at least 99.9 % of outputs within one ulp."""
    within = total = 0
    for i, (name, h, kvh, d, rows, past, form) in enumerate(cases):
        w = W.make(name, heads=h, kv_heads=kvh, head_dim=d, rows=rows, past=past, seed=seed0 + i)
        plan = _plan(h, kvh, d, rows, past, form)
        print(f"case {name} route {_route_class(plan.route(rows, past))}", flush=True)
        out = run_hsdpa(w, plan)
        ref = oracle.attention(w, form=form)
        r = compare(out, ref, w)
        assert not r["nan"], (name, r)
        assert r["max_abs_over_vmax"] <= ABS_FACTOR, (name, r)
        n = out.size
        off = int(round((1.0 - r["ulp1_share"]) * n))
        if n >= 4096:
            assert r["ulp1_share"] >= ULP_SHARE, (name, r)
        else:
            assert off <= max(2, n // 100), (name, r)
        within += n - off
        total += n
    assert within / total >= ULP_SHARE, (within, total)
