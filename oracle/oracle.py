"""ctypes wrapper of liboracle_sdpa.so — TEST INFRASTRUCTURE ONLY.

The oracle is what the parity tests compare the GPU with (a CPU restatement
of the reference's emitted SDPA, see sdpa_oracle.h). Only tests/, the smoke check and the
CPU-baseline leg of bench.py load it; the product path never does.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_sdpa.so")
_lib = None


class Spec(ctypes.Structure):
    _fields_ = [("heads", ctypes.c_uint64), ("gqa", ctypes.c_uint64), ("head_dim", ctypes.c_uint64),
                ("q_row", ctypes.c_uint64), ("q_head", ctypes.c_uint64), ("out_row", ctypes.c_uint64)]


class Call(ctypes.Structure):
    _fields_ = [("q", ctypes.c_void_p), ("keys", ctypes.c_void_p), ("values", ctypes.c_void_p),
                ("output", ctypes.c_void_p), ("rows", ctypes.c_uint64), ("past", ctypes.c_uint64),
                ("kv_stride", ctypes.c_uint64), ("scale", ctypes.c_float), ("sink", ctypes.c_float)]


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        u16p = ctypes.c_void_p
        L.oracle_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_bf16_to_f32.restype = ctypes.c_float
        L.oracle_f32_to_bf16_rne.argtypes = [ctypes.c_float]
        L.oracle_f32_to_bf16_rne.restype = ctypes.c_uint16
        L.oracle_cvtneps2bf16.argtypes = [ctypes.c_float]
        L.oracle_cvtneps2bf16.restype = ctypes.c_uint16
        L.oracle_dpbf16_lane.argtypes = [ctypes.c_float, ctypes.c_uint32, ctypes.c_uint32]
        L.oracle_dpbf16_lane.restype = ctypes.c_float
        L.oracle_exp_poly.argtypes = [ctypes.c_float]
        L.oracle_exp_poly.restype = ctypes.c_float
        L.oracle_hsum16.argtypes = [ctypes.c_void_p]
        L.oracle_hsum16.restype = ctypes.c_float
        L.oracle_rms_sumsq.argtypes = [u16p, ctypes.c_int]
        L.oracle_rms_sumsq.restype = ctypes.c_float
        L.oracle_rmsnorm.argtypes = [u16p, u16p, u16p, ctypes.c_int, ctypes.c_float, ctypes.c_int]
        L.oracle_rmsnorm.restype = None
        L.oracle_rope.argtypes = [u16p, u16p, u16p, ctypes.c_int]
        L.oracle_rope.restype = None
        L.oracle_head_norm_rope.argtypes = [u16p, u16p, u16p, u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_float, ctypes.c_int]
        L.oracle_head_norm_rope.restype = None
        L.oracle_sigmoid_mul.argtypes = [u16p, u16p, u16p, ctypes.c_int]
        L.oracle_sigmoid_mul.restype = None
        L.oracle_qk_dot.argtypes = [u16p, u16p, ctypes.c_int]
        L.oracle_qk_dot.restype = ctypes.c_float
        L.oracle_sdpa_head.argtypes = [u16p, u16p, u16p, ctypes.c_void_p, u16p, ctypes.c_uint64,
                                       ctypes.c_float, ctypes.c_int]
        L.oracle_sdpa_head.restype = None
        L.oracle_sdpa_head_qk0.argtypes = L.oracle_sdpa_head.argtypes
        L.oracle_sdpa_head_qk0.restype = None
        L.oracle_sdpa_head_sink.argtypes = L.oracle_sdpa_head.argtypes + [ctypes.c_float]
        L.oracle_sdpa_head_sink.restype = None
        L.oracle_sdpa_prefill_block.argtypes = [u16p, u16p, u16p, ctypes.c_void_p, u16p, ctypes.c_uint64,
                                                ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_size_t,
                                                ctypes.c_size_t]
        L.oracle_sdpa_prefill_block.restype = None
        L.oracle_sdpa_prefill_block_sink.argtypes = L.oracle_sdpa_prefill_block.argtypes + [ctypes.c_float]
        L.oracle_sdpa_prefill_block_sink.restype = None
        L.oracle_attention_scalar.argtypes = [ctypes.POINTER(Spec), ctypes.POINTER(Call)]
        L.oracle_attention_scalar.restype = ctypes.c_int
        L.oracle_attention_avx512.argtypes = [ctypes.POINTER(Spec), ctypes.POINTER(Call), ctypes.c_int]
        L.oracle_attention_avx512.restype = ctypes.c_int
        L.oracle_avx512_available.restype = ctypes.c_int
        L.oracle_physical_cores.restype = ctypes.c_int
        L.oracle_dpbf16_selfcheck.argtypes = [ctypes.c_uint64, ctypes.c_long]
        L.oracle_dpbf16_selfcheck.restype = ctypes.c_long
        L.oracle_cvt_exp_selfcheck.argtypes = [ctypes.c_uint64, ctypes.c_long]
        L.oracle_cvt_exp_selfcheck.restype = ctypes.c_long
        L.oracle_fused_qk_dot.argtypes = [u16p, u16p, ctypes.c_int]
        L.oracle_fused_qk_dot.restype = ctypes.c_float
        L.oracle_fused_head.argtypes = [u16p, u16p, u16p, u16p, ctypes.c_uint64, ctypes.c_float, ctypes.c_int,
                                        ctypes.c_void_p]
        L.oracle_fused_head.restype = ctypes.c_int
        L.oracle_avx2_qk_dot.argtypes = [u16p, u16p, ctypes.c_int]
        L.oracle_avx2_qk_dot.restype = ctypes.c_float
        L.oracle_avx2_head.argtypes = [u16p, u16p, u16p, ctypes.c_void_p, u16p, ctypes.c_uint64, ctypes.c_float,
                                       ctypes.c_int]
        L.oracle_avx2_head.restype = ctypes.c_int
        L.oracle_avx2_head_sink.argtypes = L.oracle_avx2_head.argtypes + [ctypes.c_float]
        L.oracle_avx2_head_sink.restype = ctypes.c_int
        L.oracle_avx2_cvt_bf16.argtypes = [ctypes.c_float]
        L.oracle_avx2_cvt_bf16.restype = ctypes.c_uint16
        L.oracle_exp_poly_n.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64]
        L.oracle_exp_poly_n.restype = None
        L.oracle_attention_form.argtypes = [ctypes.POINTER(Spec), ctypes.POINTER(Call), ctypes.c_int, ctypes.c_int]
        L.oracle_attention_form.restype = ctypes.c_int
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def avx512_available() -> bool:
    return bool(lib().oracle_avx512_available())


FORMS = {"chained": 0, "fused": 1, "avx2": 2, "chained_qk0": 3, "chained_sink": 4, "avx2_sink": 5}


def attention(w, impl: str = "auto", threads: int = 0, form: str = "chained", sink: float | None = None) -> np.ndarray:
    """Run the reference attention node on workload `w`; returns out bf16 bits
    [rows][heads][head_dim]. impl: 'scalar', 'avx512' or 'auto' (AVX-512
    when the host has it, which is bit-identical to the scalar one).
    form: 'chained' (the engine's default), 'fused' (the knob's online
    softmax), 'avx2' (a host without AVX-512 BF16) or 'chained_qk0' (the
    default form with the knob sdpa_qk_group = 0: four QK chains); the other
    forms than 'chained' run the scalar emulation on `threads` threads (0:
    the host's cores, at most 16). sink: the softmax sink value with the
    sink on (SdpaShape::sink); the Fused form declines it and the engine runs
    the Chained one, the AVX2 arm has its own (forms 'chained_sink' and
    'avx2_sink' of the scalar emulation)."""
    L = lib()
    sink_value = 0.0
    if sink is not None:
        form = "avx2_sink" if form == "avx2" else "chained_sink"
        sink_value = float(sink)
    if form != "chained":
        out = np.zeros((w.rows, w.heads, w.head_dim), dtype=np.uint16)
        q = np.ascontiguousarray(w.q)
        k = np.ascontiguousarray(w.k)
        v = np.ascontiguousarray(w.v)
        spec = Spec(w.heads, w.gqa, w.head_dim, w.q_row, w.head_dim, w.out_row)
        call = Call(_ptr(q), _ptr(k), _ptr(v), _ptr(out), w.rows, w.past, w.kv_stride, w.scale, sink_value)
        rc = L.oracle_attention_form(ctypes.byref(spec), ctypes.byref(call), FORMS[form],
                                     threads or min(16, os.cpu_count() or 1))
        if rc != 0:
            raise RuntimeError(f"oracle attention ({form}) failed rc={rc}")
        return out
    out = np.zeros((w.rows, w.heads, w.head_dim), dtype=np.uint16)
    q = np.ascontiguousarray(w.q)
    k = np.ascontiguousarray(w.k)
    v = np.ascontiguousarray(w.v)
    spec = Spec(w.heads, w.gqa, w.head_dim, w.q_row, w.head_dim, w.out_row)
    call = Call(_ptr(q), _ptr(k), _ptr(v), _ptr(out), w.rows, w.past, w.kv_stride, w.scale, 0.0)
    if impl == "auto":
        impl = "avx512" if L.oracle_avx512_available() else "scalar"
    if impl == "avx512":
        rc = L.oracle_attention_avx512(ctypes.byref(spec), ctypes.byref(call), threads)
    else:
        rc = L.oracle_attention_scalar(ctypes.byref(spec), ctypes.byref(call))
    if rc != 0:
        raise RuntimeError(f"oracle attention failed rc={rc}")
    return out


def head(q: np.ndarray, k: np.ndarray, v: np.ndarray, n: int, scale: float, qk_group0: bool = False,
         sink: float | None = None) -> np.ndarray:
    """One decode head (scalar emulation): q [d], k/v [>=n][d] -> out [d] bf16 bits.
    qk_group0: the knob sdpa_qk_group = 0 (the QK in four chains); sink: the
    softmax sink value with the sink on."""
    d = q.shape[-1]
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    sc = np.zeros(((n + 15) // 16) * 16, dtype=np.float32)
    out = np.zeros(d, dtype=np.uint16)
    if sink is not None:
        assert not qk_group0
        lib().oracle_sdpa_head_sink(_ptr(q), _ptr(k), _ptr(v), _ptr(sc), _ptr(out), n, scale, d, float(sink))
        return out
    fn = lib().oracle_sdpa_head_qk0 if qk_group0 else lib().oracle_sdpa_head
    fn(_ptr(q), _ptr(k), _ptr(v), _ptr(sc), _ptr(out), n, scale, d)
    return out


def exp_poly(x: np.ndarray) -> np.ndarray:
    """The reference's exponential on every element of a float32 array."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().oracle_exp_poly_n(_ptr(x), _ptr(y), x.size)
    return y


def fused_head(q: np.ndarray, k: np.ndarray, v: np.ndarray, n: int, scale: float, acc: bool = False):
    """One Fused-form decode head: out [d] bf16 bits, and the f32 accumulators
    before the conversion when `acc`."""
    d = q.shape[-1]
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    out = np.zeros(d, dtype=np.uint16)
    a = np.zeros(d, dtype=np.float32)
    if lib().oracle_fused_head(_ptr(q), _ptr(k), _ptr(v), _ptr(out), n, scale, d, _ptr(a)) != 0:
        raise ValueError("the Fused form declines this head_dim")
    return (out, a) if acc else out


def avx2_head(q: np.ndarray, k: np.ndarray, v: np.ndarray, n: int, scale: float,
              sink: float | None = None) -> np.ndarray:
    """One AVX2-arm decode head: out [d] bf16 bits (sink: the softmax sink value
    with the sink on)."""
    d = q.shape[-1]
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    sc = np.zeros(((n + 7) // 8) * 8 + 8, dtype=np.float32)
    out = np.zeros(d, dtype=np.uint16)
    rc = (lib().oracle_avx2_head(_ptr(q), _ptr(k), _ptr(v), _ptr(sc), _ptr(out), n, scale, d) if sink is None else
          lib().oracle_avx2_head_sink(_ptr(q), _ptr(k), _ptr(v), _ptr(sc), _ptr(out), n, scale, d, float(sink)))
    if rc != 0:
        raise ValueError("the AVX2 arm declines this head_dim")
    return out


def prefill_block(q: np.ndarray, k: np.ndarray, v: np.ndarray, past: int, scale: float,
                  sink: float | None = None) -> np.ndarray:
    """The 8-row prefill block (scalar emulation): q [rows][d] -> out [rows][d]
    (sink: the softmax sink value with the sink on)."""
    rows, d = q.shape
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    N = past + rows
    sc = np.zeros(rows * ((N + 15) // 16) * 16, dtype=np.float32)
    out = np.zeros((rows, d), dtype=np.uint16)
    if sink is None:
        lib().oracle_sdpa_prefill_block(_ptr(q), _ptr(k), _ptr(v), _ptr(sc), _ptr(out), past, scale, d, rows, d, d)
    else:
        lib().oracle_sdpa_prefill_block_sink(_ptr(q), _ptr(k), _ptr(v), _ptr(sc), _ptr(out), past, scale, d, rows, d,
                                             d, float(sink))
    return out



def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float, plus_one: bool = True) -> np.ndarray:
    """ElemOp::RmsNorm[Gemma] on one vector of bf16 bits (the restatement)."""
    x = np.ascontiguousarray(x, np.uint16)
    w = np.ascontiguousarray(w, np.uint16)
    y = np.empty_like(x)
    lib().oracle_rmsnorm(_p(x), _p(w), _p(y), x.size, eps, int(plus_one))
    return y


def rms_sumsq(x: np.ndarray) -> float:
    x = np.ascontiguousarray(x, np.uint16)
    return float(lib().oracle_rms_sumsq(_p(x), x.size))


def rope(x: np.ndarray, cos_row: np.ndarray, sin_row: np.ndarray) -> np.ndarray:
    """ElemOp::Rope on one vector (returns a rotated copy)."""
    y = np.ascontiguousarray(x, np.uint16).copy()
    c = np.ascontiguousarray(cos_row, np.uint16)
    s = np.ascontiguousarray(sin_row, np.uint16)
    lib().oracle_rope(_p(y), _p(c), _p(s), y.size)
    return y


def head_norm_rope(data: np.ndarray, w: np.ndarray, cos: np.ndarray, sin: np.ndarray, rows: int, past: int,
                   heads: int, head_dim: int, head_stride: int, row_stride: int, rotary: int, eps: float,
                   plus_one: bool = True, table_row: int | None = None) -> np.ndarray:
    """The head-norm-rope node over `rows` rows of a flat bf16 buffer (copy)."""
    out = np.ascontiguousarray(data, np.uint16).copy()
    w = np.ascontiguousarray(w, np.uint16)
    tr = rotary // 2 if table_row is None else table_row
    cos = np.ascontiguousarray(cos, np.uint16).reshape(-1)
    sin = np.ascontiguousarray(sin, np.uint16).reshape(-1)
    L = lib()
    for r in range(rows):
        row = out[r * row_stride:]
        at = (past + r) * tr
        L.oracle_head_norm_rope(_p(row), _p(w), _p(cos[at:]) if rotary else None, _p(sin[at:]) if rotary else None,
                                heads, head_stride, head_dim, rotary, eps, int(plus_one))
    return out


def sigmoid_mul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """ElemOp::SigmoidMul: a / (1 + exp(min(-b, 88))) in bf16."""
    a = np.ascontiguousarray(a, np.uint16)
    b = np.ascontiguousarray(b, np.uint16)
    y = np.empty_like(a)
    lib().oracle_sigmoid_mul(_p(a), _p(b), _p(y), a.size)
    return y
