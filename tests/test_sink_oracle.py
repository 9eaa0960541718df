"""The oracle's softmax sink (SdpaShape::sink, src/jit/ir.rs:55-60), pinned
without re-typing its formula: emit_softmax with sink_on
(src/jit/target/x86/emit_sdpa/x86/decode.rs:239-290) takes the maximum as
vmaxss(hmax, sink), adds the exponential of sink - max to the sum after the
lane tree, and multiplies the scores by 1/sum; the AVX2 arm does the same
(emit_sdpa_avx2.rs:362-400). The checks:
  - closed forms with q = 0 (every score 0) and V rows all one vector c,
    where each exponential is exact: out = c n P / (n P + S) with
    P = exp(-M), S = exp(sink - M), M = max(0, sink);
  - float64 softmax with the sink term on seeded inputs (a dropped term, a
    sign error or the term in the maximum only fails);
  - sink -> -inf gives the no-sink head up to the reciprocal's rounding;
  - the reference's block = repeated-decode invariant with the sink on;
  - the AVX2 arm with the sink within the bar of the Chained one."""
import numpy as np
import pytest

import oracle
from hsdpa import workloads as W
from parity import compare


def _bf16(x):
    x = np.asarray(x, dtype=np.float32)
    return (x.view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def _f32(b):
    return W.bf16_to_f32(b)


@pytest.mark.parametrize("sink", [0.0, 0.6931472, -1.0, 3.0, -50.0])
@pytest.mark.parametrize("n", [1, 5, 16, 33])
def test_sink_closed_form_constant_values(sink, n):
    d = 64
    q = np.zeros(d, dtype=np.uint16)                       # every score 0
    k = _bf16(np.random.default_rng(n).standard_normal((n, d)))
    c = np.random.default_rng(7).uniform(-2, 2, d).astype(np.float32)
    v = np.tile(_bf16(c), (n, 1))
    m = max(0.0, sink)
    p = float(oracle.exp_poly(np.float32([0.0 - m]))[0])   # the exponential the code evaluates
    s = float(oracle.exp_poly(np.float32([sink - m]))[0])
    want = _f32(_bf16(c)).astype(np.float64) * (n * p) / (n * p + s)
    got = _f32(oracle.head(q, k, v, n, 0.0625, sink=sink)).astype(np.float64)
    # the output is bf16: within one bf16 ulp of the closed form
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -7 + 1e-30), (sink, n)
    got2 = _f32(oracle.avx2_head(q, k, v, n, 0.0625, sink=sink)).astype(np.float64)
    assert np.all(np.abs(got2 - want) <= np.abs(want) * 2.0 ** -7 + 1e-30), (sink, n)


def _softmax64(q, k, v, n, scale, sink):
    s = (_f32(k[:n]).astype(np.float64) @ _f32(q).astype(np.float64)) * scale
    m = max(s.max(), sink) if sink is not None else s.max()
    e = np.exp(s - m)
    tot = e.sum() + (np.exp(sink - m) if sink is not None else 0.0)
    return (e / tot) @ _f32(v[:n]).astype(np.float64)


@pytest.mark.parametrize("seed", range(6))
def test_sink_matches_float64_softmax(seed):
    rng = np.random.default_rng(100 + seed)
    d, n = 128, 300
    q = _bf16(rng.standard_normal(d))
    k = _bf16(rng.standard_normal((n, d)))
    v = _bf16(rng.standard_normal((n, d)))
    scale = 1.0 / np.sqrt(d)
    s = (_f32(k).astype(np.float64) @ _f32(q).astype(np.float64)) * scale
    # the sink at the largest score, above it, and well below it
    for sink, dominant in ((float(s.max()), True), (float(s.max()) + 2.0, True), (float(np.median(s)), False)):
        want = _softmax64(q, k, v, n, scale, sink)
        got = _f32(oracle.head(q, k, v, n, scale, sink=sink)).astype(np.float64)
        assert np.max(np.abs(got - want)) <= 2.0 ** -7 * np.max(np.abs(_f32(v))), sink
        if dominant:
            # a sink at or above the largest score takes a visible share:
            # without its term the outputs move by far more than the error
            plain = _softmax64(q, k, v, n, scale, None)
            assert np.max(np.abs(plain - want)) > 4 * np.max(np.abs(got - want)), sink


def test_sink_at_minus_infinity_is_the_plain_head():
    rng = np.random.default_rng(5)
    d, n = 256, 700
    q = _bf16(rng.standard_normal(d))
    k = _bf16(rng.standard_normal((n, d)))
    v = _bf16(rng.standard_normal((n, d)))
    a = oracle.head(q, k, v, n, 1.0 / 16, sink=-np.inf)
    b = oracle.head(q, k, v, n, 1.0 / 16)
    # multiplication by 1/sum against division by the sum: at most one f32
    # rounding apart before the bf16 conversion
    diff = np.abs(a.astype(np.int32) - b.astype(np.int32))
    assert diff.max() <= 1 and (diff == 0).mean() > 0.98


@pytest.mark.parametrize("past", [0, 9, 40])
def test_sink_block_equals_repeated_decode(past):
    rng = np.random.default_rng(past)
    d, rows = 128, 8
    n = past + rows
    q = _bf16(rng.standard_normal((rows, d)))
    k = _bf16(rng.standard_normal((n, d)))
    v = _bf16(rng.standard_normal((n, d)))
    sink = 0.75
    blk = oracle.prefill_block(q, k, v, past, 0.09, sink=sink)
    for i in range(rows):
        one = oracle.head(q[i], k, v, past + i + 1, 0.09, sink=sink)
        assert np.array_equal(blk[i], one), i


def test_sink_node_forms():
    """The attention node with the sink: full 8-row chunks through the block,
    other rows through the head (form 4), the AVX2 arm row by row (form 5)
    within the parity bar of it; a sink the rows never approach leaves the
    Chained node's outputs up to the reciprocal's rounding."""
    w = W.make("sink_node", heads=8, kv_heads=2, head_dim=64, rows=13, past=20, seed=3)
    a = oracle.attention(w, sink=0.5)
    b = oracle.attention(w, form="avx2", sink=0.5)
    r = compare(a, b, w)
    assert r["ulp1_share"] >= 0.999 and r["max_abs_over_vmax"] <= 2.0 ** -6
    far = oracle.attention(w, sink=-1e4)
    plain = oracle.attention(w)
    diff = np.abs(far.astype(np.int32) - plain.astype(np.int32))
    assert diff.max() <= 1
    # a sink among the scores changes the outputs
    assert not np.array_equal(a, plain)
