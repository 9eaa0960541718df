"""The oracle's restatements of the element kernels around the attention
(head RMS norm, RoPE, output gate; src/jit/target/x86/emit_elem.rs) pinned by
known answers, a witness of the summation order, and float64 bounds."""
import numpy as np
import pytest

import oracle
from hsdpa import workloads as W


def bf(x):
    return W.f32_to_bf16(np.asarray(x, np.float32))


def f(b):
    return W.bf16_to_f32(np.asarray(b, np.uint16)).astype(np.float64)


def ulp_dist(a, b):
    def ordered(u):
        u = u.astype(np.int32)
        return np.where(u & 0x8000, -(u & 0x7FFF), u & 0x7FFF)
    return np.abs(ordered(np.asarray(a, np.uint16)) - ordered(np.asarray(b, np.uint16)))


def test_sumsq_follows_the_chains_and_the_tree():
    # x0 = 4096 and 255 ones: lane 0 of chain 0 absorbs its ones into 2^24, every
    # other lane keeps 4 ones, the chain sums and the hsum tree then add them in
    # pairs: 2^24 + 252. A sequential sum gives 2^24, the exact sum 2^24 + 255.
    x = np.full(256, bf(1.0), np.uint16)
    x[0] = bf([4096.0])[0]
    assert oracle.rms_sumsq(x) == 2.0 ** 24 + 252
    # three blocks: three chains, lane 0 absorbs one 1 per block it sees
    x3 = np.full(96, bf(1.0), np.uint16)
    x3[0] = bf([4096.0])[0]
    assert oracle.rms_sumsq(x3) == 2.0 ** 24 + 94


def test_rmsnorm_known_answers():
    w = bf(np.random.default_rng(1).normal(0, 0.1, 256))
    for c in (1.0, -4.0, 0.25):
        x = np.full(256, bf(c), np.uint16)
        y = oracle.rmsnorm(x, w, 0.0, plus_one=True)
        # sum = 256 c^2 exactly, rms = |c|, x * inv = sign(c) exactly, then * (1 + w)
        assert np.array_equal(y, bf(np.sign(c) * (1.0 + f(w).astype(np.float32))))
        y0 = oracle.rmsnorm(x, w, 0.0, plus_one=False)
        assert np.array_equal(y0, bf(np.sign(c) * f(w).astype(np.float32)))


@pytest.mark.parametrize("dim", [64, 96, 128, 256, 512])
def test_rmsnorm_float64_bound(dim):
    rng = np.random.default_rng(dim)
    for _ in range(20):
        x = bf(rng.normal(0, rng.uniform(0.1, 30), dim))
        w = bf(rng.normal(0, 0.2, dim))
        y = oracle.rmsnorm(x, w, 1e-6, plus_one=True)
        xf = f(x)
        ref = xf / np.sqrt(np.mean(xf * xf) + 1e-6) * (1.0 + f(w))
        assert ulp_dist(y, bf(ref)).max() <= 1


def test_rope_known_rotations():
    rng = np.random.default_rng(2)
    x = bf(rng.normal(0, 1, 64))
    ones, zeros = np.full(32, bf(1.0), np.uint16), np.zeros(32, np.uint16)
    assert np.array_equal(oracle.rope(x, ones, zeros), x)                        # angle 0
    y = oracle.rope(x, zeros, ones)                                              # angle pi/2
    assert np.array_equal(y[:32], x[32:] ^ 0x8000) and np.array_equal(y[32:], x[:32])


def test_rope_float64_bound():
    rng = np.random.default_rng(3)
    for _ in range(20):
        x = bf(rng.normal(0, 2, 128))
        ang = rng.uniform(0, 2 * np.pi, 64)
        c, s = bf(np.cos(ang)), bf(np.sin(ang))
        y = oracle.rope(x, c, s)
        a, b, cf, sf = f(x[:64]), f(x[64:]), f(c), f(s)
        # bf16 operands: both products are exact in f32, so the FMA and the
        # rounded difference agree; one rounding to f32, one to bf16
        ref = np.concatenate([a * cf - b * sf, a * sf + b * cf])
        assert ulp_dist(y, bf(ref)).max() <= 1


def test_sigmoid_mul_known_answers():
    a = bf([2.0, -3.0, 1.0, 5.0, 1.0, 7.0])
    b = bf([0.0, 0.0, -100.0, 100.0, np.nan, np.inf])
    y = f(oracle.sigmoid_mul(a, b))
    assert y[0] == 1.0 and y[1] == -1.5           # exp(0) = 1 exactly: a / 2
    assert y[2] == 0.0                             # exp(88): a tiny quotient, flushed by the conversion
    assert y[3] == 5.0                             # exp(-87.34) vanishes next to 1
    assert y[4] == 0.0                             # NaN gate: vminps returns the bound 88
    assert y[5] == 7.0                             # +inf gate: exp clamps at -87.34


def test_sigmoid_mul_float64_bound():
    rng = np.random.default_rng(4)
    a = bf(rng.normal(0, 2, 4096))
    b = bf(rng.normal(0, 4, 4096))
    y = oracle.sigmoid_mul(a, b)
    ref = f(a) / (1.0 + np.exp(-f(b)))
    # the polynomial's relative error (6.4e-5) is below half a bf16 ulp
    assert ulp_dist(y, bf(ref)).max() <= 1


def test_head_norm_rope_is_norm_then_partial_rope():
    rng = np.random.default_rng(5)
    heads, hd, rot, rows, past = 3, 256, 64, 4, 7
    row_stride = 2 * heads * hd
    data = bf(rng.normal(0, 1, rows * row_stride))
    w = bf(rng.normal(0, 0.1, hd))
    ang = rng.uniform(0, 6.3, (past + rows, rot // 2))
    cos, sin = bf(np.cos(ang)), bf(np.sin(ang))
    out = oracle.head_norm_rope(data, w, cos, sin, rows, past, heads, hd, hd, row_stride, rot, 1e-6)
    for r in range(rows):
        for h in range(heads):
            x = data[r * row_stride + h * hd:r * row_stride + (h + 1) * hd]
            y = oracle.rmsnorm(x, w, 1e-6)
            y[:rot] = oracle.rope(y[:rot], cos[past + r], sin[past + r])
            assert np.array_equal(out[r * row_stride + h * hd:r * row_stride + (h + 1) * hd], y)
        # the rest of the row (the gate half on the gated model) is untouched
        assert np.array_equal(out[r * row_stride + heads * hd:(r + 1) * row_stride],
                              data[r * row_stride + heads * hd:(r + 1) * row_stride])
