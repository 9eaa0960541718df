"""The attention chain of one layer (hsdpa_attention_layer), host side: every
refusal of the call happens on the host with the named status, before any
device work; a valid call without a GPU reports NO_DEVICE. GPU parity is in
test_gpu_layer.py."""
import ctypes

import pytest

import hsdpa
from hsdpa import binding

HEADS, GQA, HD, CAP = 16, 8, 256, 1000
Q_ROW = 2 * HEADS * HD                      # gated: [Q ; gate] on each row
P = 0x100000                                # a 16-byte aligned fake device address


def plan():
    return hsdpa.Plan(HEADS, GQA, HD, CAP, q_row=Q_ROW)


def layer_call(**kw):
    d = dict(q=P, k=P, v=P, keys=P, values=P, output=P, gate=P + HEADS * HD * 2, q_norm=P, k_norm=P, cos=P, sin=P,
             rows=1, past=10, kv_row=2 * HD, gate_row=Q_ROW, rotary_dims=64, table_row=32, positions=CAP,
             scale=1 / 16, eps=1e-6, plus_one=1, reserved=0, workspace=P, workspace_bytes=1 << 30)
    d.update(kw)
    return binding.LayerCall(**d)


def rc(p, **kw):
    c = layer_call(**kw)
    return binding.STATUS[hsdpa.library().hsdpa_attention_layer(p.handle, ctypes.byref(c), None)]


@pytest.mark.parametrize("kw,status", [
    (dict(rows=0, q=0), "HSDPA_OK"),                                  # the empty call: nothing, like each node
    (dict(rotary_dims=48), "HSDPA_ERR_HEAD_DIM"),                     # not a multiple of 32
    (dict(rotary_dims=288), "HSDPA_ERR_HEAD_DIM"),                    # beyond head_dim
    (dict(table_row=16), "HSDPA_ERR_STRIDE"),                         # < rotary/2
    (dict(kv_row=HD), "HSDPA_ERR_STRIDE"),                            # < kv_heads * head_dim
    (dict(positions=10), "HSDPA_ERR_CAPACITY"),                       # the tables end before the row
    (dict(rows=2, past=CAP - 1), "HSDPA_ERR_CAPACITY"),               # the cache ends before the block
    (dict(k=0), "HSDPA_ERR_NULL"),
    (dict(v=0), "HSDPA_ERR_NULL"),
    (dict(q_norm=0), "HSDPA_ERR_NULL"),
    (dict(k_norm=0), "HSDPA_ERR_NULL"),
    (dict(cos=0), "HSDPA_ERR_NULL"),
    (dict(keys=0), "HSDPA_ERR_NULL"),
    (dict(workspace=0), "HSDPA_ERR_NULL"),
    (dict(workspace_bytes=16), "HSDPA_ERR_WORKSPACE"),
    (dict(q=P + 2), "HSDPA_ERR_ALIGNMENT"),
    (dict(gate=P + 8), "HSDPA_ERR_ALIGNMENT"),                        # the gate is read 8 bytes at a time
    (dict(gate_row=Q_ROW + 4), "HSDPA_ERR_ALIGNMENT"),
    (dict(gate_row=HEADS * HD - 8), "HSDPA_ERR_STRIDE"),              # shorter than q_dim
])
def test_layer_refusals(kw, status):
    assert rc(plan(), **kw) == status


def test_layer_accepts_no_rope_and_no_gate_on_the_host():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    p = plan()
    assert rc(p) == "HSDPA_ERR_NO_DEVICE"
    assert rc(p, rotary_dims=0, cos=0, sin=0, table_row=0, positions=0) == "HSDPA_ERR_NO_DEVICE"
    assert rc(p, gate=0, gate_row=0) == "HSDPA_ERR_NO_DEVICE"
    assert hsdpa.library().hsdpa_attention_layer(None, None, None) == 9


def test_layer_refuses_a_plan_with_the_sink():
    """The layer's attention node has no sink (src/jit/schedule/scheduler.rs:111)
    and the layer call carries no sink value: a plan with the flag is refused,
    before anything else, even for an empty call."""
    p = hsdpa.Plan(HEADS, GQA, HD, CAP, q_row=Q_ROW, sink=True)
    assert rc(p) == "HSDPA_ERR_SINK_UNSUPPORTED"
    assert rc(p, rows=0, q=0) == "HSDPA_ERR_SINK_UNSUPPORTED"
