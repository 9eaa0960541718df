"""KV append (the node before the attention): the oracle pinned on a known
answer, its vectorised form against its loop form, and the C ABI's refusals.
No GPU needed; the GPU parity tests are in test_gpu_kv.py."""
import ctypes

import numpy as np
import pytest

import kv_oracle
from hsdpa import binding


def encoded_block(rows, heads, hd, tag):
    """input[(r*heads + h)*hd + d] = tag | r << 10 | h << 6 | d: every element names itself."""
    r, h, d = np.meshgrid(np.arange(rows), np.arange(heads), np.arange(hd), indexing="ij")
    return (tag | (r << 10) | (h << 6) | d).astype(np.uint16).reshape(-1)


def test_known_answer():
    heads, hd, cap, rows, past = 3, 5, 16, 4, 9
    stride = cap * hd + 7
    keys = np.full(heads * stride, 0xAAAA, np.uint16)
    values = np.full(heads * stride, 0x5555, np.uint16)
    ik, iv = encoded_block(rows, heads, hd, 0x8000), encoded_block(rows, heads, hd, 0x0000)
    kv_oracle.kv_append_tasks(keys, values, ik, iv, heads, hd, stride, rows, past)
    for h in range(heads):
        for p in range(cap):
            for d in range(hd):
                at = h * stride + p * hd + d
                if past <= p < past + rows:
                    r = p - past
                    assert keys[at] == 0x8000 | r << 10 | h << 6 | d
                    assert values[at] == r << 10 | h << 6 | d
                else:
                    assert keys[at] == 0xAAAA and values[at] == 0x5555
        # the padding between heads (stride > cap*hd) is never written
        assert np.all(keys[h * stride + cap * hd:(h + 1) * stride] == 0xAAAA)


def test_tasks_past_heads_and_empty_block_do_nothing():
    keys = np.zeros(2 * 40, np.uint16)
    values = keys.copy()
    ik = np.ones(40, np.uint16)
    kv_oracle.kv_append_tasks(keys, values, ik, ik, 2, 4, 40, 0, 3)
    assert not keys.any()
    kv_oracle.kv_append_tasks(keys, values, ik, ik, 2, 4, 40, 1, 3, tasks=5)   # tasks 2..4 are no-ops
    assert np.count_nonzero(keys) == 8


@pytest.mark.parametrize("heads,hd,cap,rows,past,pad", [(2, 256, 64, 17, 40, 0), (4, 100, 50, 50, 0, 3),
                                                       (1, 8, 10, 1, 9, 0), (3, 64, 300, 129, 100, 16)])
def test_vectorised_equals_loop(heads, hd, cap, rows, past, pad):
    rng = np.random.default_rng(heads * 1000 + hd + rows)
    stride = cap * hd + pad
    base_k = rng.integers(0, 1 << 16, heads * stride, dtype=np.uint16)
    base_v = rng.integers(0, 1 << 16, heads * stride, dtype=np.uint16)
    ik = rng.integers(0, 1 << 16, rows * heads * hd, dtype=np.uint16)
    iv = rng.integers(0, 1 << 16, rows * heads * hd, dtype=np.uint16)
    k1, v1, k2, v2 = base_k.copy(), base_v.copy(), base_k.copy(), base_v.copy()
    kv_oracle.kv_append_tasks(k1, v1, ik, iv, heads, hd, stride, rows, past)
    kv_oracle.kv_append(k2, v2, ik, iv, heads, hd, stride, rows, past)
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)


def spec(**kw):
    d = dict(heads=2, head_dim=256, stride=1024 * 256, capacity=1024, max_batch=64, r16=0, reserved=0)
    d.update(kw)
    return binding.KvSpec(**d)


@pytest.mark.parametrize("kw,code", [
    (dict(heads=0), 1), (dict(head_dim=0), 1), (dict(max_batch=0), 1),
    (dict(capacity=32), 6),                                  # capacity < max_batch
    (dict(stride=1024 * 256 - 1), 4),                        # capacity * head_dim > stride
    (dict(stride=(1 << 30)), 4),                             # stride > i32::MAX / 2
    (dict(heads=1 << 22, stride=1 << 20, capacity=1024, head_dim=1024), 4),  # heads*head_dim*2 > i32::MAX
    (dict(r16=1), 13),                                       # the AArch64 R16 layout
])
def test_kv_check_refusals(kw, code):
    s = spec(**kw)
    assert binding.library().hsdpa_kv_check(ctypes.byref(s)) == code


def test_kv_check_accepts_the_reference_geometry():
    # Qwen3.5 full-attention layers: 2 KV heads of 256, a 12 288-position reserve
    s = spec(heads=2, head_dim=256, capacity=12288, stride=12288 * 256, max_batch=4096)
    assert binding.library().hsdpa_kv_check(ctypes.byref(s)) == 0


def call_rc(s, rows, past, ptr=16):
    c = binding.KvCall(ptr, ptr, ptr, ptr, rows, past)
    return binding.library().hsdpa_kv_append(ctypes.byref(s), ctypes.byref(c), None)


def test_kv_append_call_refusals_happen_on_the_host():
    s = spec()
    assert call_rc(s, 0, 5000) == 0                          # empty block: nothing, like kv.rs:31-34
    assert call_rc(s, 65, 0) == 12                           # rows > max_batch
    assert call_rc(s, 64, 961) == 6                          # past + rows > capacity
    assert call_rc(s, 1, 1024) == 6
    assert call_rc(s, 1, 0, ptr=0) == 9                      # null pointers


def test_kv_append_without_gpu_reports_no_device():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    assert call_rc(spec(), 1, 0) == 11


# ---- head-norm-rope and output-gate refusals (host side) ----------------------

def nr_rc(**kw):
    d = dict(heads=16, head_dim=256, head_stride=256, row_stride=8192, rotary_dims=64, table_row=32,
             positions=100, plus_one=1, reserved=0)
    call_kw = {k[5:]: kw.pop(k) for k in list(kw) if k.startswith("call_")}
    d.update(kw)
    s = binding.NormRopeSpec(**d)
    c = dict(data=16, weight=16, cos=16, sin=16, rows=4, past=0, eps=1e-6, reserved=0.0)
    c.update(call_kw)
    call = binding.NormRopeCall(**c)
    return binding.library().hsdpa_head_norm_rope(ctypes.byref(s), ctypes.byref(call), None)


@pytest.mark.parametrize("kw,code", [
    (dict(heads=0), 1), (dict(head_dim=0), 1),
    (dict(head_dim=100), 2), (dict(head_dim=1024, head_stride=1024), 2),   # multiple of 32, at most 512
    (dict(rotary_dims=48), 2), (dict(rotary_dims=512), 2),                 # multiple of 32, at most head_dim
    (dict(head_stride=128), 4), (dict(row_stride=4000), 4), (dict(table_row=16), 4),
    (dict(call_past=97), 6),                                                # past + rows > table positions
    (dict(call_data=0), 9), (dict(call_cos=0), 9),
])
def test_head_norm_rope_refusals(kw, code):
    assert nr_rc(**kw) == code


def test_head_norm_rope_empty_and_device():
    import torch

    assert nr_rc(call_rows=0) == 0
    assert nr_rc(rotary_dims=0, call_cos=0, call_sin=0, call_past=10 ** 6) in (0, 11)  # no tables needed
    if not torch.cuda.is_available():
        assert nr_rc() == 11


def gate_rc(width=4096, attn_row=4096, gate_row=8192, attn=16, gate=16, rows=2):
    s = binding.GateSpec(width, attn_row, gate_row)
    c = binding.GateCall(attn, gate, rows)
    return binding.library().hsdpa_output_gate(ctypes.byref(s), ctypes.byref(c), None)


def test_output_gate_refusals():
    import torch

    assert gate_rc(width=0) == 1
    assert gate_rc(attn_row=100) == 4 and gate_rc(gate_row=100) == 4
    assert gate_rc(rows=0) == 0
    assert gate_rc(attn=0) == 9
    if not torch.cuda.is_available():
        assert gate_rc() == 11
