"""GPU parity of the head dimensions other than 64, 128 and 256: every multiple
of 32 from 32 to 512 that the reference's SdpaShape::check accepts
(src/jit/ir.rs:130-162), against the oracle on seeded inputs, through the C ABI.
Each decode configuration the head dimension allows is exercised: pass 1 with
one tile per wave and, up to 256, looping over several; pass 2 with 4 waves
and, where the V tiles fit, 8; groups of at most 8 heads and of up to 16; and
the causal kernel for prefill chunks and for a decode row of a group beyond 16.

The one-ulp share is judged over at least 4 096 outputs (the output count of
the decode configuration the criterion is quoted on), pooling seeded samples
of the same shape when one has fewer: about 0.02-0.05 % of outputs, the ones
near zero, land two or more ulps from the oracle at every head dimension
(64, 128 and 256 included), so two of them in a sample of 1 000-2 000 outputs
would fail a 99.9 % share that a larger sample meets. The per-row absolute
bound holds for every sample."""
import numpy as np
import pytest

import oracle
from hsdpa import workloads as W
from parity import ABS_FACTOR, ULP_SHARE, compare

from gpu_util import run_hsdpa

pytestmark = pytest.mark.gpu

MORE_DIMS = [32, 96, 160, 192, 224, 288, 320, 352, 384, 416, 448, 480, 512]

CASES = []
for d in MORE_DIMS:
    # name, heads, kv_heads, head_dim, rows, past
    CASES.append((f"decode_d{d}_n300", 8, 2, d, 1, 299))
    CASES.append((f"prefill_d{d}_r70_p33", 8, 2, d, 70, 33))
CASES += [
    ("decode_d96_g16_n1000", 16, 1, 96, 1, 999),                 # two P column blocks
    ("decode_d512_g12_n700", 12, 1, 512, 1, 699),
    ("decode_d32_wide_n9000", 16, 4, 32, 1, 8999),                # 8-wave pass 2 (more than one round)
    ("decode_d192_wide_n9000", 16, 4, 192, 1, 8999),
    ("decode_d224_wide_n9000", 8, 4, 224, 1, 8999),
    ("decode_d96_loop_n40001", 16, 2, 96, 1, 40000),              # pass 1 loops; 4-wave pass 2 only
    ("decode_d160_loop_n40001", 16, 2, 160, 1, 40000),
    ("decode_d384_n40001", 16, 2, 384, 1, 40000),                 # one tile per wave past 256
    ("decode_d96_g32_two_groups", 32, 1, 96, 1, 500),
    ("decode_d96_g80_through_prefill", 80, 1, 96, 1, 500),
    ("prefill_d448_r300_p0_g1", 4, 4, 448, 300, 0),
    ("prefill_d160_r257_p1000", 8, 1, 160, 257, 1000),
]


POOL = 4096


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_head_dims(torch_cuda, case):
    name, h, kvh, d, rows, past = case
    samples = -(-POOL // (h * d * rows))
    within, total = 0, 0
    for k in range(samples):
        print(f"case {name} sample {k}", flush=True)
        w = W.make(name, heads=h, kv_heads=kvh, head_dim=d, rows=rows, past=past, seed=d + rows + 1000 * k)
        r = compare(run_hsdpa(w), oracle.attention(w), w)
        assert not r["nan"], f"{name} sample {k}: NaN in output {r}"
        assert r["max_abs_over_vmax"] <= ABS_FACTOR, f"{name} sample {k}: max abs error too large {r}"
        n = h * d * rows
        within += int(round(r["ulp1_share"] * n))
        total += n
    share = within / total
    print(name, f"{samples} samples, {total} outputs, {share:.5%} within 1 ulp", flush=True)
    assert share >= ULP_SHARE, f"{name}: only {share:.5%} of {total} outputs within 1 ulp"
