"""hsdpa_attention_frame: a decode step whose rows and past the kernels read
from device memory, as the reference's tasks read them through AttentionCall's
pointers (src/jit/execution/abi.rs:156-180). One HIP graph is captured once
and replayed at successive past values (the cache growing by a token, then by
thousands), each replay's output checked against the oracle at that past; the
run-time values that compute nothing (rows 0) or are refused (rows 2, past at
the capacity) leave the output untouched and report through the status word."""
import ctypes

import numpy as np
import pytest
import torch

import hsdpa
import oracle
from hsdpa import binding
from hsdpa import workloads as W
from parity import assert_parity

pytestmark = pytest.mark.gpu

CASES = [
    # name, heads, kv_heads, head_dim, capacity, form, successive past values
    ("frame_d256_g8", 16, 2, 256, 40000, "chained", [1023, 1024, 1025, 5000, 32767]),
    ("frame_d256_g8_fused", 16, 2, 256, 40000, "fused", [0, 300, 20000]),
    ("frame_d256_g16_two_blocks", 32, 2, 256, 9000, "chained", [100, 8999]),
    # 16 columns at D = 256 over a long capacity: pass 2 in chunked runs
    ("frame_d256_g16_runs", 32, 2, 256, 40000, "chained", [4000, 39999]),
    ("frame_d128_g8", 32, 4, 128, 70000, "chained", [2047, 2048, 65000]),
    ("frame_d64_g24_two_groups", 48, 2, 64, 6000, "fused", [5, 5999]),
]


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_frame_graph_replays_successive_steps(torch_cuda, case):
    name, h, kvh, d, cap, form, pasts = case
    plan = hsdpa.Plan(h, h // kvh, d, cap, form=form, max_rows=1)
    w = W.make(name, heads=h, kv_heads=kvh, head_dim=d, rows=1, past=max(pasts), capacity=cap, seed=23)
    q, k, v = _dev(w.q), _dev(w.k), _dev(w.v)
    out = torch.full((1, h, d), -1, dtype=torch.int16, device="cuda")
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    vals = torch.zeros(2, dtype=torch.int64, device="cuda")            # rows, past
    status = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    call = binding.FrameCall(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), vals.data_ptr(),
                             vals.data_ptr() + 8, w.scale, 0.0, ws.data_ptr(), plan.workspace_bytes,
                             status.data_ptr())
    lib = hsdpa.library()
    # one eager call (rows 0) loads the kernels before the capture
    rc = lib.hsdpa_attention_frame(plan.handle, ctypes.byref(call),
                                   ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, binding.STATUS.get(rc)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.hsdpa_attention_frame(plan.handle, ctypes.byref(call),
                                       ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, binding.STATUS.get(rc)
    for past in pasts:
        print(f"case {name} replay at past {past}", flush=True)
        vals.copy_(torch.tensor([1, past], dtype=torch.int64))
        out.fill_(-1)
        status.fill_(-1)
        graph.replay()
        torch.cuda.synchronize()
        assert int(status.item()) == 0, binding.STATUS.get(int(status.item()))
        got = out.cpu().numpy().view(np.uint16)
        ws_view = W.Workload(name, h, kvh, d, 1, past, cap, w.q, w.k, w.v, w.scale)
        assert_parity(got, oracle.attention(ws_view, form=form), ws_view, f"{name} past {past}")
    # run-time values with nothing to compute: the output keeps its sentinel
    for rows, past, want in [(0, 100, "HSDPA_OK"), (2, 100, "HSDPA_ERR_BATCH"), (1, cap, "HSDPA_ERR_CAPACITY")]:
        print(f"case {name} replay with rows {rows} past {past}", flush=True)
        vals.copy_(torch.tensor([rows, past], dtype=torch.int64))
        out.fill_(-1)
        status.fill_(-1)
        graph.replay()
        torch.cuda.synchronize()
        assert binding.STATUS.get(int(status.item())) == want, (rows, past)
        assert (out.cpu().numpy() == -1).all(), (rows, past)
