"""CPU tests that pin the oracle's other decode forms, and the softmax order of
the default one, before the GPU is compared with them.

The reference emits three x86 decode head kernels:
  * Chained (the default, sdpa_scalar.c): exact maximum, lane sums over
    16-wide blocks then the hsum tree, division by the sum;
  * Fused (the sdpa_form = fused knob, sdpa_forms.c): an online softmax over
    blocks of 16 positions (src/jit/target/x86/emit_sdpa/x86/decode.rs:501-669);
  * AVX2 (a host without AVX-512 BF16, sdpa_forms.c): the Chained form on
    eight lanes (src/jit/target/x86/emit_sdpa_avx2.rs:231-470).

Each test below is a case whose answer follows from the arithmetic by hand
(exact powers of two, integer sums, one-hot values), chosen so that a
plausible mistake in the restatement gives another answer: a sequential sum
instead of the lane sums and tree, a multiplication by the reciprocal instead
of the division, a missing rescale, a global maximum instead of the running
one, one accumulation chain instead of four, odd-first instead of
even-first products.
"""
import ctypes

import numpy as np
import pytest

import oracle
from hsdpa import workloads as W
from parity import compare

L = oracle.lib()
f32 = np.float32
ONE, NEG_ONE = 0x3F80, 0xBF80                     # bf16 bits of 1.0 and -1.0
LN2_F32 = f32(0.6931472)                          # fl(x * 1.442695) == 1 exactly
X24_F32 = f32(16.635532)                          # fl(x * 1.442695) == 24 exactly


def bf(x):
    return W.f32_to_bf16(np.asarray(x, dtype=np.float32))


def ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def test_exact_exponent_constants():
    """The constants of these witnesses: exp_poly is exactly 2^k there."""
    assert f32(LN2_F32 * f32(1.442695)) == 1.0 and f32(-LN2_F32 * f32(1.442695)) == -1.0
    assert f32(X24_F32 * f32(1.442695)) == 24.0
    assert L.oracle_exp_poly(float(-LN2_F32)) == 0.5
    assert L.oracle_exp_poly(float(-X24_F32)) == 2.0 ** -24
    assert L.oracle_exp_poly(0.0) == 1.0


def chained_scores(q, k, v, n, scale):
    """oracle_sdpa_head on one head, returning (out, the probabilities the
    softmax leaves in the scores buffer)."""
    d = q.shape[-1]
    q, k, v = (np.ascontiguousarray(a, dtype=np.uint16) for a in (q, k, v))
    sc = np.zeros(((n + 15) // 16) * 16, dtype=np.float32)
    out = np.zeros(d, dtype=np.uint16)
    L.oracle_sdpa_head(ptr(q), ptr(k), ptr(v), ptr(sc), ptr(out), n, scale, d)
    return out, sc


def level_keys(levels, d=32):
    """q = -e0; key j has K_j[0] = levels[j] (0 or 1): the score of key j is
    -levels[j] * scale exactly."""
    q = np.zeros(d, np.uint16)
    q[0] = NEG_ONE
    k = np.zeros((len(levels), d), np.uint16)
    k[:, 0] = np.where(np.asarray(levels) == 1, ONE, 0)
    return q, k


# ---- Chained: the softmax's sum order and its division ---------------------------

def test_chained_softmax_lane_sums_then_tree():
    """Key 0 scores 0 (e = 1), keys 1..31 score -x24 (e = 2^-24 exactly).
    The emitted order (lane sums across the two 16-wide blocks, then the hsum
    tree, decode.rs:247-257) gives 1 + 15*2^-23; a sequential sum over the
    positions gives 1.0 (each 1 + 2^-24 rounds to even); the exact sum
    1 + 31*2^-24 rounds to 1 + 2^-19."""
    n = 32
    q, k = level_keys([0] + [1] * 31)
    v = np.zeros((n, 32), np.uint16)
    _, p = chained_scores(q, k, v, n, float(X24_F32))
    total = f32(1.0 + 15 * 2.0 ** -23)
    assert p[0] == f32(1.0) / total
    assert np.all(p[1:n] == f32(2.0 ** -24) / total)
    assert p[0] != f32(1.0) / f32(1.0) and p[0] != f32(1.0) / f32(1.0 + 2.0 ** -19)


def test_chained_softmax_divides():
    """Two keys, scores 0 and -y: the sum is fl(1 + a), a = P(-y), exactly in
    any order. The probability of key 1 is the IEEE quotient fl(a / sum)
    (vdivps, decode.rs:283-291), which for this y differs from a times the
    reciprocal."""
    q, k = level_keys([0, 1])
    v = np.zeros((2, 32), np.uint16)
    hits = 0
    for y in np.linspace(0.1, 9.0, 400, dtype=np.float32):
        a = f32(L.oracle_exp_poly(float(-y)))
        s = f32(f32(1.0) + a)
        if f32(a / s) == f32(a * (f32(1.0) / s)):
            continue
        _, p = chained_scores(q, k, v, 2, float(y))
        assert p[0] == f32(1.0) / s and p[1] == f32(a / s), y
        hits += 1
    assert hits >= 5


# ---- Fused ------------------------------------------------------------------------

def test_fused_empty_context_is_zero():
    """n = 0: the accumulators stay zero and no division happens (decode.rs:536-541)."""
    rng = np.random.default_rng(1)
    q = bf(rng.standard_normal(64))
    kv = bf(rng.standard_normal((4, 64)))
    out, acc = oracle.fused_head(q, kv, kv, 0, 0.125, acc=True)
    assert np.all(out == 0) and np.all(acc == 0)


@pytest.mark.parametrize("d", [32, 64, 128, 256])
def test_fused_one_key_is_v0(d):
    rng = np.random.default_rng(d)
    q = bf(rng.standard_normal(d))
    k = bf(rng.standard_normal((3, d)))
    v = bf(rng.standard_normal((3, d)))
    assert np.array_equal(oracle.fused_head(q, k, v, 1, 1.0 / np.sqrt(d)), v[0])


@pytest.mark.parametrize("n", [1, 15, 16, 17, 100, 1000])
def test_fused_zero_keys_sum_in_order_times_reciprocal(n):
    """K = 0: every score is 0, so every block keeps the maximum 0 (corr = 1)
    and every weight is 1. The accumulator is the sequential f32 sum of the V
    rows (FMA by 1), the lane sums count to n exactly, and the output is
    bf16(sum * fl(1/n)): the Fused form multiplies by the reciprocal
    (decode.rs:653-659) where the Chained form sums fl(1/n) * V_j."""
    rng = np.random.default_rng(n)
    d = 64
    q = bf(rng.standard_normal(d))
    k = np.zeros((n, d), np.uint16)
    v = bf(rng.standard_normal((n, d)))
    seq = np.add.accumulate(W.bf16_to_f32(v), axis=0, dtype=np.float32)[-1]
    want_acc = (seq * (f32(1.0) / f32(n))).astype(np.float32)
    want = np.array([L.oracle_cvtneps2bf16(float(x)) for x in want_acc], np.uint16)
    out, acc = oracle.fused_head(q, k, v, n, 0.125, acc=True)
    assert np.array_equal(acc, want_acc) and np.array_equal(out, want)
    if n >= 15 and n & (n - 1):
        # (1/n not a power of two) the Chained form's accumulators: FMA of fl(1/n) * V_j in order
        p = np.float64(f32(1.0) / f32(n))
        ch = np.zeros(d, np.float32)
        for j in range(n):
            ch = (ch.astype(np.float64) + W.bf16_to_f32(v[j]).astype(np.float64) * p).astype(np.float32)
        assert not np.array_equal(ch, want_acc), "the forms must be told apart"


def test_fused_rescales_when_the_maximum_rises():
    """Two blocks, one-hot V (V_j = e_j) so the output reads out the weights.
    Block 0 scores 0 (maximum 0, weights 1). Block 1: key 16 scores ln2
    (the new maximum), keys 17..31 score 0. corr = P(0 - ln2) = 1/2 exactly,
    so block 0's weights become 1/2, key 16 weighs 1, keys 17..31 weigh 1/2;
    the lane sums are 1.5 and fifteen 1.0, total 16.5; out = weights * fl(1/16.5)."""
    d, n = 32, 32
    q = np.zeros(d, np.uint16)
    q[0] = ONE
    k = np.zeros((n, d), np.uint16)
    k[16, 0] = ONE
    v = np.zeros((n, d), np.uint16)
    v[np.arange(n), np.arange(n)] = ONE
    out, acc = oracle.fused_head(q, k, v, n, float(LN2_F32), acc=True)
    wts = np.full(d, 0.5, np.float32)
    wts[16] = 1.0
    want_acc = (wts * (f32(1.0) / f32(16.5))).astype(np.float32)
    assert np.array_equal(acc, want_acc)
    # without the rescale block 0 would weigh 1 and the sum be 24.5
    assert not np.array_equal(acc[:16], np.full(16, f32(1.0) * (f32(1.0) / f32(24.5)), np.float32))


def test_fused_sum_in_lanes_then_tree():
    """Key 0 scores 0 (e = 1), keys 1..31 score -x24 (e = 2^-24); the maximum
    stays 0, so every correction is P(0) = 1. The sum lives in 16 lanes
    across the blocks and the hsum tree adds them at the end (decode.rs:605-606,
    653): 1 + 15 * 2^-23, where a sequential sum gives 1. One-hot V reads the
    weights out: key 0's is fl(1 / sum) after the reciprocal."""
    n, d = 32, 32
    q, k = level_keys([0] + [1] * 31, d)
    v = np.zeros((n, d), np.uint16)
    v[np.arange(n), np.arange(n)] = ONE
    _, acc = oracle.fused_head(q, k, v, n, float(X24_F32), acc=True)
    inv = f32(1.0) / f32(1.0 + 15 * 2.0 ** -23)
    assert acc[0] == inv and np.all(acc[1:] == f32(f32(2.0 ** -24) * inv))
    assert acc[0] != f32(1.0)


def test_fused_evaluates_at_the_running_maximum():
    """Block 0: key 0 scores 0, key 1 scores z < 0, keys 2..15 score 0.
    Block 1: key 16 scores ln2. Key 1's weight is P(z) from block 0, then
    halved exactly by corr = 1/2: fl(P(z) / 2); evaluating it at the final
    maximum instead would give P(z - ln2), which differs for this z. The lane
    sums are those of the emitted order, added by the hsum tree."""
    d, n = 32, 32
    v = np.zeros((n, d), np.uint16)
    v[np.arange(n), np.arange(n)] = ONE
    q = np.zeros(d, np.uint16)
    q[0] = ONE
    found = 0
    for t in np.linspace(-4.0, -0.25, 120, dtype=np.float32):
        tb = int(bf(t)[0])
        z = f32(W.bf16_to_f32(np.uint16(tb)) * LN2_F32)       # score of key 1
        pz = f32(L.oracle_exp_poly(float(z)))
        running = f32(pz * f32(0.5))
        glob = f32(L.oracle_exp_poly(float(f32(z - LN2_F32))))
        if running == glob:
            continue
        k = np.zeros((n, d), np.uint16)
        k[1, 0] = tb
        k[16, 0] = ONE
        lanes = np.ones(16, np.float32)
        lanes[1] = pz
        lanes *= f32(0.5)
        lanes += np.float32(0.5)                                # P(0 - ln2) for keys 17..31
        lanes[0] = f32(0.5) + f32(1.0)                          # key 16 at the new maximum
        lanes[1] = f32(f32(pz * f32(0.5)) + f32(0.5))
        total = f32(L.oracle_hsum16(ptr(lanes)))
        _, acc = oracle.fused_head(q, k, v, n, float(LN2_F32), acc=True)
        assert acc[1] == f32(running * (f32(1.0) / total)), t
        assert acc[1] != f32(glob * (f32(1.0) / total))
        found += 1
    assert found >= 5


def test_fused_qk_runs_four_chains():
    """Lane 0 holds 2^24 in chunk 0's odd pair and 1 in the odd pair of chunks
    1..7. The Fused form's four chains (chunk c into chain c % 4, then
    (w0 + w1) + (w2 + w3)) give 2^24 + 6; the Chained form's single chain
    gives 2^24 (every 2^24 + 1 rounds to even); the exact sum is 2^24 + 7."""
    d = 256
    q = np.zeros(d, np.uint16)
    k = np.zeros(d, np.uint16)
    q[1] = k[1] = int(bf(4096.0)[0])
    for c in range(1, 8):
        q[32 * c + 1] = k[32 * c + 1] = ONE
    assert L.oracle_fused_qk_dot(ptr(q), ptr(k), d) == 2.0 ** 24 + 6
    assert L.oracle_qk_dot(ptr(q), ptr(k), d) == 2.0 ** 24


def test_fused_declines_above_256():
    q = np.zeros(288, np.uint16)
    with pytest.raises(ValueError):
        oracle.fused_head(q, np.zeros((2, 288), np.uint16), np.zeros((2, 288), np.uint16), 2, 0.1)


@pytest.mark.parametrize("d,n", [(64, 40), (128, 300), (256, 1000)])
def test_fused_against_float64(d, n):
    """Random N(0,1) inputs: the Fused head is the float64 softmax-weighted sum
    to within one bf16 rounding (2^-8 relative) plus the polynomial's error:
    each weight is P at one point times up to a few corrections, 6.4e-5
    relative each, so 2e-4 of max |V| bounds them."""
    rng = np.random.default_rng(d + n)
    for h in range(4):
        q = bf(rng.standard_normal(d))
        k = bf(rng.standard_normal((n, d)))
        v = bf(rng.standard_normal((n, d)))
        scale = f32(1.0 / np.sqrt(d))
        s = (W.bf16_to_f32(k).astype(np.float64) @ W.bf16_to_f32(q).astype(np.float64)) * float(scale)
        p = np.exp(s - s.max())
        ref = (p @ W.bf16_to_f32(v).astype(np.float64)) / p.sum()
        got = W.bf16_to_f32(oracle.fused_head(q, k, v, n, float(scale))).astype(np.float64)
        assert np.all(np.abs(got - ref) <= 2 ** -8 * np.abs(ref) + 2e-4 * np.abs(W.bf16_to_f32(v)).max())


def test_fused_node_blocks_and_tails():
    """The node under the Fused form: full 8-row chunks still run the prefill
    block (bit-identical to the Chained node there), the other rows the
    Fused head with n = past + r + 1; above head_dim 256 everything is
    Chained (the fallback of src/jit/sdpa.rs:491-510)."""
    w = W.make("fused_node", heads=4, kv_heads=2, head_dim=64, rows=13, past=21, seed=5)
    fused = oracle.attention(w, form="fused", threads=2)
    chained = oracle.attention(w, "scalar")
    assert np.array_equal(fused[:8], chained[:8])
    for r in range(8, 13):
        for h in range(w.heads):
            kvh = h // w.gqa
            want = oracle.fused_head(w.q[r, h], w.k[kvh], w.v[kvh], w.past + r + 1, w.scale)
            assert np.array_equal(fused[r, h], want)
    w2 = W.make("fused_node_288", heads=2, kv_heads=1, head_dim=288, rows=3, past=5, seed=6)
    assert np.array_equal(oracle.attention(w2, form="fused", threads=2), oracle.attention(w2, "scalar"))


# ---- AVX2 ---------------------------------------------------------------------------

def test_avx2_cvt_is_integer_rne_without_flush():
    """The AVX2 epilogue rounds with integer arithmetic (emit_sdpa_avx2.rs:208-217):
    nearest even like the host helper, denormals kept (vcvtneps2bf16 flushes them)."""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(3000) * 10.0 ** rng.integers(-30, 30, 3000)).astype(np.float32)
    den = np.array([1e-39, -2.5e-39, 3e-42], np.float32)
    for v in np.concatenate([x, den]):
        assert L.oracle_avx2_cvt_bf16(float(v)) == L.oracle_f32_to_bf16_rne(float(v))
    assert L.oracle_avx2_cvt_bf16(float(den[0])) != 0 and L.oracle_cvtneps2bf16(float(den[0])) == 0


def test_avx2_qk_order():
    """Lane 0 of the AVX2 QK: block b (16 elements) into chain b % 4, the
    even element of each pair before the odd one.
      * chains: 2^24 at block 0, 1 at blocks 1..15 (even slots): chain 0 keeps
        2^24 (each + 1 rounds to even), chains 1-3 hold 4 each, so
        (c0 + c1) + (c2 + c3) = 2^24 + 12; one chain would give 2^24;
      * even first: after 2^24 in block 0, block 4 holds 1 (even) and 2 (odd):
        2^24 + 1 -> 2^24, + 2 -> 2^24 + 2; odd first would give 2^24 + 4."""
    d = 256
    q = np.zeros(d, np.uint16)
    k = np.zeros(d, np.uint16)
    q[0] = k[0] = int(bf(4096.0)[0])
    for b in range(1, 16):
        q[16 * b] = k[16 * b] = ONE
    assert L.oracle_avx2_qk_dot(ptr(q), ptr(k), d) == 2.0 ** 24 + 12
    q2 = np.zeros(d, np.uint16)
    k2 = np.zeros(d, np.uint16)
    q2[0] = k2[0] = int(bf(4096.0)[0])
    q2[64] = k2[64] = ONE                          # block 4, even: product 1
    q2[65], k2[65] = ONE, int(bf(2.0)[0])             # block 4, odd: product 2
    assert L.oracle_avx2_qk_dot(ptr(q2), ptr(k2), d) == 2.0 ** 24 + 2


def test_avx2_softmax_eight_lanes():
    """Key 0 scores 0, keys 1..15 score -x24 (e = 2^-24). Eight lanes over two
    blocks of 8: lane 0 = 1 + 2^-24 -> 1, lanes 1..7 = 2^-23; the 8-lane tree
    (x_i = l_i + l_{i+4}, then (x0 + x1) + (x2 + x3)) gives 1 + 7*2^-23, where
    the 16-lane form gives 1 + 15*2^-24 -> 1 + 7*2^-23 as well; a sequential
    sum gives 1. Then the probabilities are quotients by that sum."""
    n = 16
    q, k = level_keys([0] + [1] * 15)
    v = np.zeros((n, 32), np.uint16)
    v[0, 0] = ONE
    sc = np.zeros(24, np.float32)
    out = np.zeros(32, np.uint16)
    qq, kk, vv = (np.ascontiguousarray(a) for a in (q, k, v))
    assert L.oracle_avx2_head(ptr(qq), ptr(kk), ptr(vv), ptr(sc), ptr(out), n, float(X24_F32), 32) == 0
    total = f32(1.0 + 7 * 2.0 ** -23)
    assert sc[0] == f32(1.0) / total and np.all(sc[1:n] == f32(2.0 ** -24) / total)
    # V_0 = e0: out[0] = bf16(p_0), rounded as the integer RNE does
    assert out[0] == L.oracle_avx2_cvt_bf16(float(f32(1.0) / total))


def test_avx2_pads_to_eight():
    """n = 9: the scores buffer is padded with -inf to 16 (two blocks of 8),
    whose exponentials (2^-126 * p) vanish in the sums. Key 0 at the maximum
    (e = 1), keys 1..8 at -x24 (e = 2^-24): lane 0 holds 1 + 2^-24 -> 1 (key 8),
    lanes 1..7 hold 2^-24; the tree folds lane i + 4 onto lane i (1, then
    2^-23 three times) and gives (1 + 2^-23) + 2^-22 = 1 + 3 * 2^-23, where
    the exact sum 1 + 8 * 2^-24 would be 1 + 2^-21."""
    n = 9
    q, k = level_keys([0] + [1] * 8)
    v = np.zeros((n, 32), np.uint16)
    sc = np.zeros(16, np.float32)
    out = np.zeros(32, np.uint16)
    qq, kk, vv = (np.ascontiguousarray(a) for a in (q, k, v))
    L.oracle_avx2_head(ptr(qq), ptr(kk), ptr(vv), ptr(sc), ptr(out), n, float(X24_F32), 32)
    total = f32(1.0 + 3 * 2.0 ** -23)
    assert sc[0] == f32(1.0) / total and sc[0] != f32(1.0) / f32(1.0 + 2.0 ** -21)
    assert np.all(sc[n:16] < 1e-37)


@pytest.mark.parametrize("d,n", [(32, 9), (64, 40), (256, 700)])
def test_avx2_closed_forms(d, n):
    """n = 1 gives V_0 exactly; K = 0 gives p = fl(1/n) summed in order by FMA."""
    rng = np.random.default_rng(d * n)
    q = bf(rng.standard_normal(d))
    v = bf(rng.standard_normal((n, d)))
    assert np.array_equal(oracle.avx2_head(q, bf(rng.standard_normal((n, d))), v, 1, 0.3), v[0])
    k = np.zeros((n, d), np.uint16)
    p = f32(1.0) / f32(n)
    acc = np.zeros(d, np.float32)
    vf = W.bf16_to_f32(v)
    for j in range(n):
        acc = (acc.astype(np.float64) + vf[j].astype(np.float64) * np.float64(p)).astype(np.float32)
    want = np.array([L.oracle_avx2_cvt_bf16(float(x)) for x in acc], np.uint16)
    assert np.array_equal(oracle.avx2_head(q, k, v, n, 0.3), want)


def test_avx2_node_runs_every_row_on_the_head():
    """No block kernel without AVX-512 BF16: every row of a prefill is the
    AVX2 head with n = past + r + 1."""
    w = W.make("avx2_node", heads=4, kv_heads=1, head_dim=128, rows=11, past=30, seed=9)
    got = oracle.attention(w, form="avx2", threads=2)
    for r in range(w.rows):
        for h in range(w.heads):
            want = oracle.avx2_head(w.q[r, h], w.k[0], w.v[0], w.past + r + 1, w.scale)
            assert np.array_equal(got[r, h], want)


def test_forms_against_each_other_on_decode():
    """The three forms are different bits of the same attention. The AVX2 arm
    differs from the Chained form only in summation orders and agrees with it
    within the parity bar. The Fused form stays within the bar's absolute
    bound but not always within its ulp share (its exponentials are taken at
    running maxima): 1K keys, seed 2, 99.85 %. So the GPU computes the Fused
    form's own weights rather than the Chained ones."""
    w = W.config("decode_1k", seed=2)
    ch = oracle.attention(w)
    r = compare(oracle.attention(w, form="avx2"), ch, w)
    assert r["ulp1_share"] >= 0.999 and r["max_abs_over_vmax"] <= 2.0 ** -6, r
    r = compare(oracle.attention(w, form="fused"), ch, w)
    assert r["max_abs_over_vmax"] <= 2.0 ** -6 and r["ulp1_share"] < 0.999, r


# ---- the GPU's numeric scheme for the Fused form ---------------------------------------

def _split(e):
    hi = W.bf16_to_f32(W.f32_to_bf16(e))
    lo = W.bf16_to_f32(W.f32_to_bf16((e - hi).astype(np.float32)))
    return hi.astype(np.float64) + lo


def test_fused_gpu_scheme_meets_the_bar_and_online_flash_does_not():
    """A model of the GPU's Fused decode (scores as f32 dot products; each
    block of 16 keys evaluated at the running maximum M_b, weights times the
    product C_b of the later blocks' corrections P(M_{b-1} - M_b), P split hi +
    lo for the matrix cores, the sum multiplied by its reciprocal) meets the
    parity bar against the Fused oracle at the 32K configuration. A one-pass
    flash decode (each 256-key split at its own maximum, rescaled by
    P(m_split - M) in the combine) does not: its exponentials are evaluated
    at other points than the reference's."""
    w = W.config("decode_32k", seed=0)
    ref = oracle.attention(w, form="fused")
    n = w.past + 1
    good = np.zeros_like(ref)
    flash = np.zeros_like(ref)
    for h in range(w.heads):
        kf = W.bf16_to_f32(w.k[h // w.gqa][:n]).astype(np.float64)
        vf = W.bf16_to_f32(w.v[h // w.gqa][:n]).astype(np.float64)
        s = ((kf @ W.bf16_to_f32(w.q[0, h]).astype(np.float64)).astype(f32) * f32(w.scale)).astype(f32)
        nb = (n + 15) // 16
        bm = np.full(nb * 16, -np.inf, f32)
        bm[:n] = s
        M = np.maximum.accumulate(bm.reshape(nb, 16).max(1))
        corr = np.ones(nb, f32)
        corr[1:] = oracle.exp_poly((M[:-1] - M[1:]).astype(f32))
        C = np.ones(nb, f32)
        for b in range(nb - 2, -1, -1):
            C[b] = f32(C[b + 1] * corr[b + 1])
        wgt = (oracle.exp_poly((s - np.repeat(M, 16)[:n]).astype(f32)) * np.repeat(C, 16)[:n]).astype(f32)
        good[0, h] = bf((_split(wgt) @ vf).astype(f32) * (f32(1.0) / f32(wgt.astype(np.float64).sum())))
        S = 256
        ms = np.array([s[i:i + S].max() for i in range(0, n, S)], f32)
        fw = oracle.exp_poly((ms - ms.max()).astype(f32)).astype(np.float64)
        O = np.zeros(w.head_dim)
        lsum = 0.0
        for i, j0 in enumerate(range(0, n, S)):
            e = oracle.exp_poly((s[j0:j0 + S] - ms[i]).astype(f32))
            O += fw[i] * (_split(e) @ vf[j0:j0 + S])
            lsum += fw[i] * e.astype(np.float64).sum()
        flash[0, h] = bf(O.astype(f32) * (f32(1.0) / f32(lsum)))
    assert compare(good, ref, w)["ulp1_share"] >= 0.999
    assert compare(flash, ref, w)["ulp1_share"] < 0.999


def test_one_pass_decode_fails_the_chained_bar_at_32k():
    """The default (Chained) form evaluates every exponential at the exact row
    maximum (src/jit/target/x86/emit_sdpa/x86/decode.rs:212-293). A model of
    the GPU's two-pass scheme (f32 scores, the exact maximum, P split hi + lo,
    one division at the end) meets the bar against the Chained oracle at the
    32K configuration. A one-pass split-KV decode, which would stream K and V
    in one kernel (each key range at its own maximum m_w, its O and l rescaled
    by P(m_w - M) in the combine), does not, with ranges of 256 or 1024 keys:
    the polynomial's error depends on where it is evaluated, and near-zero
    outputs move by more than an ulp (seeds 0-2: 99.76-99.88 % within one ulp;
    an exact exp for the rescale factor does no better). So the decode keeps
    its two passes."""
    w = W.config("decode_32k", seed=0)
    ref = oracle.attention(w)
    n = w.past + 1
    exact = np.zeros_like(ref)
    one = {256: np.zeros_like(ref), 1024: np.zeros_like(ref)}
    for h in range(w.heads):
        kf = W.bf16_to_f32(w.k[h // w.gqa][:n]).astype(np.float64)
        vf = W.bf16_to_f32(w.v[h // w.gqa][:n]).astype(np.float64)
        s = ((kf @ W.bf16_to_f32(w.q[0, h]).astype(np.float64)).astype(f32) * f32(w.scale)).astype(f32)
        e = oracle.exp_poly((s - s.max()).astype(f32))
        exact[0, h] = bf((_split(e) @ vf).astype(f32) / f32(e.astype(np.float64).sum()))
        for S, out in one.items():
            ms = np.array([s[i:i + S].max() for i in range(0, n, S)], f32)
            fw = oracle.exp_poly((ms - ms.max()).astype(f32)).astype(np.float64)
            O = np.zeros(w.head_dim)
            lsum = 0.0
            for i, j0 in enumerate(range(0, n, S)):
                e = oracle.exp_poly((s[j0:j0 + S] - ms[i]).astype(f32))
                O += fw[i] * (_split(e) @ vf[j0:j0 + S])
                lsum += fw[i] * e.astype(np.float64).sum()
            out[0, h] = bf(O.astype(f32) / f32(lsum))
    assert compare(exact, ref, w)["ulp1_share"] >= 0.999
    for S, out in one.items():
        r = compare(out, ref, w)
        assert r["ulp1_share"] < 0.999 and r["max_abs_over_vmax"] <= 2.0 ** -6, (S, r)


# ---- the knob sdpa_qk_group = 0: the Chained form with four QK chains ----------

def _chain_witness(d=256):
    """q, K rows and V rows of a two-key head whose first score is 0 in one
    chain and 2 in four: lane 0 of chunk 0 adds 2^24, chunks 1 and 2 add 1
    each, chunk 4 subtracts 2^24. One chain: 2^24 + 1 rounds to 2^24 (a tie,
    to even) twice, then 0. Four chains (chunk c into chain c % 4): chain 0
    is 2^24 - 2^24 = 0, chains 1 and 2 are 1, (0 + 1) + (1 + 0) = 2."""
    q = np.zeros(d, np.uint16)
    k = np.zeros((2, d), np.uint16)
    v = np.zeros((2, d), np.uint16)
    two12, neg_two12 = 0x4580, 0xC580                       # bf16 of 2^12 and -2^12
    q[1], k[0, 1] = two12, two12                            # chunk 0, lane 0, odd element: 2^24
    q[32 + 1], k[0, 32 + 1] = ONE, ONE                      # chunk 1: 1
    q[64 + 1], k[0, 64 + 1] = ONE, ONE                      # chunk 2: 1
    q[128 + 1], k[0, 128 + 1] = neg_two12, two12            # chunk 4: -2^24
    v[0, :] = ONE                                           # key 0's values 1, key 1's 0
    return q, k, v


def test_qk_group0_four_chain_witness():
    """The restatement of the knob sdpa_qk_group = 0 (src/jit/sdpa.rs:178-202):
    emit_qk with four chains (decode.rs:59-128), the tree (c0 + c1) + (c2 +
    c3). On the witness the default form's scores are (0, 0), so every
    output is exactly 1/2; the four-chain scores are (2, 0), so the outputs
    are bf16(1 / (1 + P(-2))) (the padded lanes' P(-inf) ~ 1e-38 vanish in
    the sum)."""
    q, k, v = _chain_witness()
    assert L.oracle_qk_dot(ptr(q), ptr(np.ascontiguousarray(k[0])), 256) == 0.0
    assert L.oracle_fused_qk_dot(ptr(q), ptr(np.ascontiguousarray(k[0])), 256) == 2.0
    assert (oracle.head(q, k, v, 2, 1.0) == 0x3F00).all()                  # 0.5
    want = bf(f32(1.0) / (f32(1.0) + f32(oracle.exp_poly(np.array([-2.0], f32))[0])))
    assert (oracle.head(q, k, v, 2, 1.0, qk_group0=True) == want).all()
    assert want != 0x3F00


def test_qk_group0_node_block_equals_repeated_decode():
    """Under sdpa_qk_group = 0 the prefill block sums its scores like the
    four-chain head (emit_qk_block with chains = 4, prefill.rs:104-157, 780),
    so the reference's invariant holds for it too: each row of an 8-row chunk
    equals the head at n = past + r + 1, bit for bit. The two orders give
    different score bits for part of the scores (the reference measured
    96.8 % identical on its data, src/jit/sdpa.rs:190-193; 84 % on these
    N(0,1) inputs)."""
    w = W.make("qk0_block", heads=4, kv_heads=2, head_dim=256, rows=19, past=41, seed=5)
    got = oracle.attention(w, form="chained_qk0", threads=2)
    for r in range(w.rows):
        for h in range(w.heads):
            want = oracle.head(w.q[r, h], w.k[h // w.gqa], w.v[h // w.gqa], w.past + r + 1, w.scale,
                               qk_group0=True)
            assert np.array_equal(got[r, h], want), (r, h)
    same = [L.oracle_qk_dot(ptr(np.ascontiguousarray(w.q[r, h])), ptr(np.ascontiguousarray(w.k[h // w.gqa, j])), 256)
            == L.oracle_fused_qk_dot(ptr(np.ascontiguousarray(w.q[r, h])),
                                     ptr(np.ascontiguousarray(w.k[h // w.gqa, j])), 256)
            for r in range(w.rows) for h in range(w.heads) for j in range(w.past + w.rows)]
    assert 0.5 < np.mean(same) < 0.99, np.mean(same)
