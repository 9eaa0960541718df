"""CPU tests that pin the oracle (the CPU restatement of the reference's
emitted SDPA) before the parity tests compare the GPU with it.

What pins what:
  * bf16 conversions   : closed forms over all 65 536 bf16 values, and an
                         exact nearest-even model over random and tie inputs;
  * vdpbf16ps lane     : an independent float64 model of "odd pair, then even
                         pair, each one rounding" and, on an AVX-512 BF16 host,
                         the hardware instruction itself;
  * exp polynomial     : P(0) = 1 exactly, P(-inf) = 2^-126 * p, an
                         independent float32 model of each step, and the
                         relative-error bound against exp;
  * QK score           : an independent model of one accumulation chain plus
                         the reduction tree, and a float64 dot bound;
  * whole head         : n = 1 gives V_0, K = 0 gives uniform weights
                         fl(1/n) summed in order, V = c gives c, one dominant
                         key gives its V row, float64 SDPA within a bound;
  * the reference's own invariants: a prefill block equals repeated decode
                         bit for bit, GQA head mapping, the AVX-512
                         restatement equals the scalar emulation bit for bit;
  * golden fixtures    : tests/golden/*.npz reproduce bit for bit.
"""
import glob
import math
import os

import numpy as np
import pytest

import oracle
from hsdpa import workloads as W
from parity import compare

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
L = oracle.lib()
f32 = np.float32


def bits(x):
    return np.asarray(x, dtype=np.float32).view(np.uint32)


def from_bits(b):
    return np.asarray(b, dtype=np.uint32).view(np.float32)


# ---- bf16 conversions --------------------------------------------------------

def test_bf16_widen_all_values():
    b = np.arange(65536, dtype=np.uint32)
    got = np.array([L.oracle_bf16_to_f32(int(x)) for x in b[::257]], dtype=np.float32)
    assert np.array_equal(bits(got), (b[::257] << 16).astype(np.uint32))
    w = W.bf16_to_f32(b.astype(np.uint16))
    assert np.array_equal(bits(w), b << 16)


def _rne_model(x):
    """Nearest-even to bf16 by comparing the two neighbours exactly in float64."""
    out = []
    for v in np.asarray(x, dtype=np.float32):
        b = int(bits(v))
        lo, hi = b >> 16, (b >> 16) + 1
        dlo = abs(float(v) - float(from_bits(lo << 16)))
        dhi = abs(float(from_bits((hi & 0xFFFF) << 16)) - float(v)) if (hi & 0xFFFF) else math.inf
        if dlo < dhi or (dlo == dhi and lo % 2 == 0):
            out.append(lo & 0xFFFF)
        else:
            out.append(hi & 0xFFFF)
    return np.array(out, dtype=np.uint16)


def test_f32_to_bf16_rne_against_model():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(4000) * 10.0 ** rng.integers(-6, 6, 4000)).astype(np.float32)
    ties = from_bits((rng.integers(0x3F000000, 0x40800000, 500, dtype=np.uint32) & 0xFFFF0000) | 0x8000)
    x = np.concatenate([x, ties, np.array([0.0, -0.0, 1.0, -1.0, 65504.0], dtype=np.float32)])
    model = _rne_model(x)
    got = np.array([L.oracle_f32_to_bf16_rne(float(v)) for v in x], dtype=np.uint16)
    assert np.array_equal(got, model)
    assert np.array_equal(W.f32_to_bf16(x), model)


def test_cvtneps2bf16_special_values():
    cases = {0x00000001: 0x0000, 0x807FFFFF: 0x8000, 0x7F800000: 0x7F80, 0xFF800000: 0xFF80,
             0x7FC00001: 0x7FC0, 0x7F800001: 0x7FC0, 0x3F808000: 0x3F80, 0x3F818000: 0x3F82,
             0x3F80FFFF: 0x3F81}
    for src, want in cases.items():
        assert L.oracle_cvtneps2bf16(float(from_bits(src))) == want, hex(src)


# ---- vdpbf16ps ---------------------------------------------------------------

def _dp_model(acc, a, b):
    """acc += a.odd*b.odd then += a.even*b.even; each step one f32 rounding of
    an exact sum (float64 holds both exactly here), DAZ in, FTZ out."""
    def daz(v):
        v = np.float32(v)
        return np.float32(0.0) * np.sign(v) if (abs(v) < 2.0 ** -126 and v != 0) else v

    a1 = daz(W.bf16_to_f32(np.uint16(a >> 16))[()])
    a0 = daz(W.bf16_to_f32(np.uint16(a & 0xFFFF))[()])
    b1 = daz(W.bf16_to_f32(np.uint16(b >> 16))[()])
    b0 = daz(W.bf16_to_f32(np.uint16(b & 0xFFFF))[()])
    s = daz(np.float32(np.float64(daz(acc)) + np.float64(a1) * np.float64(b1)))
    s = daz(np.float32(np.float64(s) + np.float64(a0) * np.float64(b0)))
    return s


def test_dpbf16_lane_against_model():
    rng = np.random.default_rng(2)
    for _ in range(3000):
        a = int(rng.integers(0, 2**32))
        b = int(rng.integers(0, 2**32))
        # keep exponents moderate so that float64 holds every sum exactly
        a = (a & 0x807F807F) | 0x3C003C00 | (int(rng.integers(0, 16)) << 23) | (int(rng.integers(0, 16)) << 7)
        b = (b & 0x807F807F) | 0x3C003C00
        acc = np.float32(rng.standard_normal() * 4)
        got = np.float32(L.oracle_dpbf16_lane(float(acc), a, b))
        want = _dp_model(acc, a, b)
        assert bits(got) == bits(want), (hex(a), hex(b), acc)


def test_dpbf16_order_matters_and_is_odd_first():
    # acc = 1 + u (u = 2^-23), odd product +u/2, even product -u/2.
    # Odd first: 1 + 1.5u ties to 1 + 2u, then 1 + 1.5u ties to 1 + 2u.
    # Even first: 1 + 0.5u ties to 1, then 1 + 0.5u ties to 1.
    a = (0x3380 << 16) | 0xB380          # odd 2^-24, even -2^-24
    b = (0x3F80 << 16) | 0x3F80          # both 1.0
    acc = from_bits(np.uint32(0x3F800001))[()]
    got = np.float32(L.oracle_dpbf16_lane(float(acc), a, b))
    assert bits(got) == 0x3F800002
    assert bits(got) == bits(_dp_model(acc, a, b))


@pytest.mark.skipif(not oracle.avx512_available(), reason="host lacks AVX-512 BF16")
def test_dpbf16_matches_hardware():
    assert L.oracle_dpbf16_selfcheck(7, 1_000_000) == 0


@pytest.mark.skipif(not oracle.avx512_available(), reason="host lacks AVX-512 BF16")
def test_cvt_and_exp_match_hardware_sequence():
    assert L.oracle_cvt_exp_selfcheck(8, 500_000) == 0


# ---- the exponential ------------------------------------------------------------

def _exp_model(x):
    """The emitted polynomial step by step in float32 (base.rs:189-212)."""
    x = np.float32(max(np.float32(x), np.float32(-87.33654)))
    t = np.float32(x * np.float32(1.442695))
    k = np.float32(np.rint(t))
    f = np.float32(t - k)

    def fma(p, q, r):  # exact product and sum in float64 for these magnitudes
        return np.float32(np.float64(p) * np.float64(q) + np.float64(r))

    p = fma(f, np.float32(0.00967248), np.float32(0.05550411))
    p = fma(f, p, np.float32(0.2402265))
    p = fma(f, p, np.float32(0.6931472))
    p = fma(f, p, np.float32(1.0))
    return np.float32(p * np.float32(2.0 ** int(k)))


def test_exp_known_answers():
    assert L.oracle_exp_poly(0.0) == 1.0
    pinf = L.oracle_exp_poly(-math.inf)
    assert 1.17e-38 < pinf < 1.18e-38
    assert L.oracle_exp_poly(-200.0) == pinf


def test_exp_against_step_model():
    rng = np.random.default_rng(3)
    xs = np.concatenate([-rng.random(20000).astype(np.float32) * 90, np.float32([-1e-30, -0.5, -0.3465736, -87.3, -87.4])])
    for x in xs:
        got = np.float32(L.oracle_exp_poly(float(x)))
        assert bits(got) == bits(_exp_model(x)), x


def test_exp_error_bound():
    xs = np.linspace(-87.0, 0.0, 200001, dtype=np.float32)
    got = np.array([L.oracle_exp_poly(float(x)) for x in xs[::7]], dtype=np.float64)
    rel = np.abs(got / np.exp(xs[::7].astype(np.float64)) - 1.0)
    assert rel.max() < 7e-5
    assert rel.max() > 1e-5   # the polynomial is not libm exp: the error is real


# ---- QK score -----------------------------------------------------------------------

def _qk_model(q, k):
    """One chain over chunks of 32 (odd pair then even pair per lane), then the
    tree s_i = l_i + l_{i+8}, t_i = s_i + s_{i+4}, (t0+t1) + (t2+t3)."""
    d = q.shape[0]
    lanes = [np.float32(0.0)] * 16
    for c in range(d // 32):
        for ln in range(16):
            i = 32 * c + 2 * ln
            a = (int(q[i + 1]) << 16) | int(q[i])
            b = (int(k[i + 1]) << 16) | int(k[i])
            lanes[ln] = _dp_model(lanes[ln], a, b)
    s = [np.float32(lanes[i] + lanes[i + 8]) for i in range(8)]
    t = [np.float32(s[i] + s[i + 4]) for i in range(4)]
    return np.float32(np.float32(t[0] + t[1]) + np.float32(t[2] + t[3]))


def test_qk_dot_against_model_and_f64():
    rng = np.random.default_rng(4)
    for d in (32, 64, 256):
        for _ in range(20):
            q = W.f32_to_bf16(rng.standard_normal(d).astype(np.float32))
            k = W.f32_to_bf16(rng.standard_normal(d).astype(np.float32))
            got = np.float32(L.oracle_qk_dot(q.ctypes.data, k.ctypes.data, d))
            assert bits(got) == bits(_qk_model(q, k))
            exact = float(W.bf16_to_f32(q).astype(np.float64) @ W.bf16_to_f32(k).astype(np.float64))
            assert abs(float(got) - exact) <= 1e-5 * (1 + abs(exact))


# ---- whole head: closed forms ----------------------------------------------------

def _head(q, k, v, n, scale):
    return oracle.head(q, k, v, n, scale)


def test_single_key_returns_v0():
    rng = np.random.default_rng(5)
    d = 256
    q = W.f32_to_bf16(rng.standard_normal(d).astype(np.float32))
    k = W.f32_to_bf16(rng.standard_normal((4, d)).astype(np.float32))
    v = W.f32_to_bf16(rng.standard_normal((4, d)).astype(np.float32))
    assert np.array_equal(_head(q, k, v, 1, 1 / 16), v[0])


@pytest.mark.parametrize("n", [1, 5, 16, 37, 100])
def test_zero_keys_give_uniform_weights_in_order(n):
    rng = np.random.default_rng(6 + n)
    d = 64
    q = W.f32_to_bf16(rng.standard_normal(d).astype(np.float32))
    k = np.zeros((n, d), dtype=np.uint16)
    v = W.f32_to_bf16(rng.standard_normal((n, d)).astype(np.float32))
    got = _head(q, k, v, n, 1 / 8)
    p = np.float32(np.float32(1.0) / np.float32(n))
    acc = np.zeros(d, dtype=np.float32)
    vf = W.bf16_to_f32(v)
    for j in range(n):
        acc = (vf[j].astype(np.float64) * np.float64(p) + acc.astype(np.float64)).astype(np.float32)
    want = np.array([L.oracle_cvtneps2bf16(float(x)) for x in acc], dtype=np.uint16)
    assert np.array_equal(got, want)


def test_constant_values_give_the_constant():
    rng = np.random.default_rng(7)
    d, n = 128, 300
    q = W.f32_to_bf16(rng.standard_normal(d).astype(np.float32))
    k = W.f32_to_bf16(rng.standard_normal((n, d)).astype(np.float32))
    c = W.f32_to_bf16(np.float32([0.7109375]))[0]
    v = np.full((n, d), c, dtype=np.uint16)
    got = _head(q, k, v, n, 1 / math.sqrt(d))
    dist = np.abs(got.astype(np.int32) - int(c))
    assert dist.max() <= 1


def test_dominant_key_returns_its_row():
    rng = np.random.default_rng(8)
    d, n, js = 256, 200, 77
    k = W.f32_to_bf16(rng.standard_normal((n, d)).astype(np.float32))
    q = W.f32_to_bf16((W.bf16_to_f32(k[js]) * 8.0).astype(np.float32))
    v = W.f32_to_bf16(rng.standard_normal((n, d)).astype(np.float32))
    got = W.bf16_to_f32(_head(q, k, v, n, 1 / 16))
    assert np.abs(got - W.bf16_to_f32(v[js])).max() <= 2 ** -7 * np.abs(W.bf16_to_f32(v)).max()


@pytest.mark.parametrize("d,n", [(32, 3), (64, 50), (256, 130)])
def test_head_against_float64_sdpa(d, n):
    rng = np.random.default_rng(9 + d)
    q = W.f32_to_bf16(rng.standard_normal(d).astype(np.float32))
    k = W.f32_to_bf16(rng.standard_normal((n, d)).astype(np.float32))
    v = W.f32_to_bf16(rng.standard_normal((n, d)).astype(np.float32))
    scale = 1 / math.sqrt(d)
    got = W.bf16_to_f32(_head(q, k, v, n, scale)).astype(np.float64)
    s = W.bf16_to_f32(k).astype(np.float64) @ W.bf16_to_f32(q).astype(np.float64) * scale
    p = np.exp(s - s.max())
    p /= p.sum()
    ref = p @ W.bf16_to_f32(v).astype(np.float64)
    # one bf16 rounding (2^-9 relative) plus the polynomial's 7e-5
    assert np.all(np.abs(got - ref) <= 2 ** -8 * np.abs(ref) + 2e-4 * np.abs(W.bf16_to_f32(v)).max())


# ---- the reference's invariants -------------------------------------------------------

@pytest.mark.parametrize("past", [0, 3, 13, 16, 40])
def test_prefill_block_equals_repeated_decode(past):
    rng = np.random.default_rng(10 + past)
    d, rows = 256, 8
    n = past + rows
    q = W.f32_to_bf16(rng.standard_normal((rows, d)).astype(np.float32))
    k = W.f32_to_bf16(rng.standard_normal((n, d)).astype(np.float32))
    v = W.f32_to_bf16(rng.standard_normal((n, d)).astype(np.float32))
    block = oracle.prefill_block(q, k, v, past, 1 / 16)
    for i in range(rows):
        assert np.array_equal(block[i], _head(q[i], k, v, past + i + 1, 1 / 16)), i


def test_gqa_mapping():
    w = W.make("gqa", heads=4, kv_heads=2, head_dim=64, rows=3, past=20, seed=12)
    w.q[:, 1] = w.q[:, 0]          # heads 0 and 1 share KV head 0
    w.q[:, 2] = w.q[:, 0]          # head 2 reads KV head 1
    out = oracle.attention(w, "scalar")
    assert np.array_equal(out[:, 0], out[:, 1])
    assert not np.array_equal(out[:, 0], out[:, 2])
    w2 = W.Workload(w.name, w.heads, w.kv_heads, w.head_dim, w.rows, w.past, w.capacity, w.q,
                    w.k.copy(), w.v.copy(), w.scale)
    w2.k[1] = 0                    # KV head 1 changed: heads 0, 1 unaffected
    out2 = oracle.attention(w2, "scalar")
    assert np.array_equal(out[:, :2], out2[:, :2])
    assert not np.array_equal(out[:, 2:], out2[:, 2:])


def test_causal_rows_ignore_future_keys():
    w = W.make("causal", heads=2, kv_heads=1, head_dim=64, rows=12, past=5, seed=13)
    out = oracle.attention(w, "scalar")
    w.k[0, 10:] = 0x4000
    w.v[0, 10:] = 0x4000
    out2 = oracle.attention(w, "scalar")
    # rows 0..4 see keys <= 9 only
    assert np.array_equal(out[:5], out2[:5])
    assert not np.array_equal(out[5:], out2[5:])


@pytest.mark.skipif(not oracle.avx512_available(), reason="host lacks AVX-512 BF16")
@pytest.mark.parametrize("case", [(8, 2, 256, 1, 0), (8, 2, 256, 1, 36), (8, 2, 256, 1, 1023), (4, 4, 64, 1, 7),
                                  (8, 2, 256, 19, 37), (6, 2, 256, 129, 0), (8, 4, 128, 300, 211),
                                  (4, 1, 32, 9, 1)])
def test_avx512_equals_scalar(case):
    h, kvh, d, rows, past = case
    w = W.make("x", heads=h, kv_heads=kvh, head_dim=d, rows=rows, past=past, seed=14)
    a = oracle.attention(w, "avx512", threads=3)
    b = oracle.attention(w, "scalar")
    assert np.array_equal(a, b)


def test_invalid_geometry_refused():
    w = W.make("bad", heads=4, kv_heads=2, head_dim=64, rows=2, past=3, seed=15)
    spec = oracle.Spec(4, 3, 64, 256, 64, 256)     # 4 heads, gqa 3
    out = np.zeros((2, 4, 64), dtype=np.uint16)
    call = oracle.Call(w.q.ctypes.data, w.k.ctypes.data, w.v.ctypes.data, out.ctypes.data, 2, 3, w.kv_stride,
                       w.scale, 0.0)
    import ctypes
    assert L.oracle_attention_scalar(ctypes.byref(spec), ctypes.byref(call)) == -1
    spec = oracle.Spec(4, 2, 48, 256, 64, 256)     # head_dim not a multiple of 32
    assert L.oracle_attention_scalar(ctypes.byref(spec), ctypes.byref(call)) == -1


# ---- golden fixtures -------------------------------------------------------------------

def _load(path):
    z = np.load(path, allow_pickle=False)
    h, kvh, d, rows, past, cap = (int(x) for x in z["geometry"])
    w = W.Workload(os.path.basename(path), h, kvh, d, rows, past, cap, z["q"], z["k"], z["v"], float(z["scale"]))
    return w, z["out"]


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))),
                         ids=lambda p: os.path.basename(p)[:-4])
def test_golden(path):
    w, want = _load(path)
    assert np.array_equal(oracle.attention(w, "scalar"), want)
    if oracle.avx512_available():
        assert np.array_equal(oracle.attention(w, "avx512", threads=2), want)


def test_golden_inputs_match_generator():
    w, _ = _load(os.path.join(GOLDEN, "prefill_r19_p37_d256.npz"))
    g = W.make("prefill_r19_p37_d256", heads=8, kv_heads=2, head_dim=256, rows=19, past=37, seed=107)
    assert np.array_equal(w.q, g.q) and np.array_equal(w.k, g.k) and np.array_equal(w.v, g.v)


# ---- the parity criterion has teeth -------------------------------------------------

def test_parity_criterion_rejects_bf16_probabilities():
    """P rounded to bf16 before P.V (a textbook flash kernel) drifts by more
    than one ulp on far more than 0.1 % of outputs: the criterion tells it
    apart from the exact-maximum hi/lo scheme the kernels use."""
    w = W.make("teeth", heads=2, kv_heads=1, head_dim=64, rows=64, past=256, seed=16)
    ref = oracle.attention(w, "scalar")
    qf = W.bf16_to_f32(w.q).astype(np.float64)
    kf = W.bf16_to_f32(w.k[0]).astype(np.float64)
    vf = W.bf16_to_f32(w.v[0]).astype(np.float64)
    bad = np.zeros_like(ref)
    good = np.zeros_like(ref)
    for r in range(w.rows):
        n = w.past + r + 1
        for h in range(w.heads):
            s = (kf[:n] @ qf[r, h] * w.scale).astype(np.float32)
            e = np.array([L.oracle_exp_poly(float(x)) for x in (s - s.max()).astype(np.float32)], dtype=np.float32)
            hi = W.bf16_to_f32(W.f32_to_bf16(e))
            lo = W.bf16_to_f32(W.f32_to_bf16((e - hi).astype(np.float32)))
            bad[r, h] = W.f32_to_bf16(((hi.astype(np.float64) @ vf[:n]) / e.sum()).astype(np.float32))
            good[r, h] = W.f32_to_bf16((((hi.astype(np.float64) + lo) @ vf[:n]) / e.sum()).astype(np.float32))
    assert compare(good, ref, w)["ulp1_share"] >= 0.999
    assert compare(bad, ref, w)["ulp1_share"] < 0.99
