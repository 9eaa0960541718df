"""hsdpa_attention_static, the entry point that allocates nothing, against
hsdpa_attention with a caller workspace: the same kernels on the same
inputs, so the outputs must be equal bit for bit. Two calls in a row, the
second on a smaller input, so the second finds the first call's contents in
the shared static scratch."""
import ctypes

import numpy as np
import pytest
import torch

import hsdpa
from hsdpa import binding
from hsdpa import workloads as W

pytestmark = pytest.mark.gpu


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()


def _run(plan, w, static):
    """One call of workload w through the C ABI; returns the output bits."""
    q, k, v = _dev(w.q), _dev(w.k), _dev(w.v)
    out = torch.full((w.rows, w.heads, w.head_dim), -1, dtype=torch.int16, device="cuda")
    if static:
        ws_ptr, ws_bytes = 0, 0
    else:
        ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
        ws_ptr, ws_bytes = ws.data_ptr(), plan.workspace_bytes
    call = binding.Call(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), w.rows, w.past, w.scale, 0.0,
                        ws_ptr, ws_bytes)
    stream = torch.cuda.current_stream().cuda_stream
    fn = hsdpa.library().hsdpa_attention_static if static else hsdpa.library().hsdpa_attention
    rc = fn(plan.handle, ctypes.byref(call), ctypes.c_void_p(stream))
    assert rc == 0, binding.STATUS.get(rc)
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint16)


CASES = [
    # name, plan (heads, gqa, head_dim, capacity, form, max_rows), first call (rows, past), second call
    ("decode_32k_then_1k", (16, 8, 256, 32768, "chained", 1), (1, 32767), (1, 1023)),
    ("fused_decode_40k_then_5k", (16, 8, 256, 40001, "fused", 1), (1, 40000), (1, 4999)),
    ("fused_decode_3k_then_500", (16, 8, 256, 3000, "fused", 1), (1, 2999), (1, 499)),
    ("few_rows_d128_then_decode", (16, 8, 128, 20000, "chained", 4), (4, 19996), (1, 700)),
    ("split_prefill_d64_then_decode", (8, 2, 64, 4096, "chained", 0), (64, 3000), (1, 300)),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_static_matches_workspace_entry(torch_cuda, case):
    name, (h, g, d, cap, form, max_rows), first, second = case
    plan = hsdpa.Plan(h, g, d, cap, form=form, max_rows=max_rows)
    assert plan.workspace_bytes <= binding.STATIC_SCRATCH_BYTES, plan.workspace_bytes
    for i, (rows, past) in enumerate((first, second)):
        w = W.make(f"{name}_{i}", heads=h, kv_heads=h // g, head_dim=d, rows=rows, past=past, capacity=cap,
                   seed=31 + i)
        print(f"case {name} call {i}: rows {rows} past {past} route {plan.route(rows, past)['main']}", flush=True)
        got = _run(plan, w, static=True)
        want = _run(plan, w, static=False)
        assert np.array_equal(got, want), f"{name} call {i}"


def test_static_refuses_a_plan_beyond_the_scratch(torch_cuda):
    plan = hsdpa.Plan(16, 8, 256, 32768)                  # any rows: the split cells alone are 67 MB
    assert plan.workspace_bytes > binding.STATIC_SCRATCH_BYTES
    call = binding.Call(0x10000, 0x20000, 0x30000, 0x40000, 1, 100, 0.0625, 0.0, 0, 0)
    rc = hsdpa.library().hsdpa_attention_static(plan.handle, ctypes.byref(call), None)
    assert binding.STATUS[rc] == "HSDPA_ERR_STATIC_SCRATCH"


def test_static_entry_under_graph_capture(torch_cuda):
    """hsdpa_attention_static captured in a HIP graph (its address resolved at
    plan creation, so the captured call looks nothing up): each replay equals
    hsdpa_attention bit for bit, also after an eager call on other inputs has
    left its own contents in the shared scratch between the replays."""
    h, g, d, cap = 16, 8, 256, 8192
    plan = hsdpa.Plan(h, g, d, cap, max_rows=1)
    w = W.make("graph_static", heads=h, kv_heads=h // g, head_dim=d, rows=1, past=5000, capacity=cap, seed=41)
    other = W.make("graph_static_other", heads=h, kv_heads=h // g, head_dim=d, rows=1, past=700, capacity=cap,
                   seed=42)
    want = _run(plan, w, static=False)
    q, k, v = _dev(w.q), _dev(w.k), _dev(w.v)
    out = torch.full((w.rows, w.heads, w.head_dim), -1, dtype=torch.int16, device="cuda")
    call = binding.Call(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), w.rows, w.past, w.scale, 0.0,
                        0, 0)
    lib = hsdpa.library()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        rc = lib.hsdpa_attention_static(plan.handle, ctypes.byref(call), ctypes.c_void_p(side.cuda_stream))
        assert rc == 0, binding.STATUS.get(rc)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.hsdpa_attention_static(plan.handle, ctypes.byref(call),
                                        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, binding.STATUS.get(rc)
    for i in range(3):
        out.fill_(-1)
        print(f"graph replay {i}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint16), want), f"replay {i}"
        _run(plan, other, static=True)          # eager, other contents in the scratch
