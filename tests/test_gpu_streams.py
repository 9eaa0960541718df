"""Stream and graph behaviour through the C ABI: one plan serving calls on two
streams at once (each with its own workspace), and calls captured into a HIP
graph and replayed several times with other work, on the same workspace, in
between. Every result must equal, bit for bit, the same call run alone and
eagerly. The kernels use no memset nodes, so nothing in a replay depends on
state a previous replay left behind."""
import numpy as np
import pytest

from hsdpa import workloads as W

import hsdpa

pytestmark = pytest.mark.gpu


def dev_tensors(torch, w):
    dev = torch.device("cuda")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)
    out = torch.full((w.rows, w.heads, w.head_dim), -1, dtype=torch.int16, device=dev)
    return t(w.q), t(w.k), t(w.v), out


def alone(torch, plan, w):
    q, k, v, out = dev_tensors(torch, w)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    hsdpa.attention_torch(plan, q, k, v, out, w.rows, w.past, w.scale, ws)
    torch.cuda.synchronize()
    return out.cpu()


def test_two_streams_two_workspaces(torch_cuda):
    torch = torch_cuda
    # one plan; a decode and a short chunk after a long cache (the split causal kernel)
    cap = 9000
    wd = W.make("streams_decode", heads=16, kv_heads=2, head_dim=256, rows=1, past=8191, capacity=cap, seed=21)
    wp = W.make("streams_prefill", heads=16, kv_heads=2, head_dim=256, rows=300, past=8000, capacity=cap, seed=22)
    plan = hsdpa.Plan(16, 8, 256, cap)
    want_d, want_p = alone(torch, plan, wd), alone(torch, plan, wp)
    bd, bp = dev_tensors(torch, wd), dev_tensors(torch, wp)
    wsd = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    wsp = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    for _ in range(5):
        hsdpa.attention_torch(plan, *bd[:3], bd[3], wd.rows, wd.past, wd.scale, wsd, s1)
        hsdpa.attention_torch(plan, *bp[:3], bp[3], wp.rows, wp.past, wp.scale, wsp, s2)
    torch.cuda.synchronize()
    assert torch.equal(bd[3].cpu(), want_d)
    assert torch.equal(bp[3].cpu(), want_p)


def test_graph_replays_with_work_between(torch_cuda):
    torch = torch_cuda
    cap = 6000
    wd = W.make("graph_decode", heads=16, kv_heads=2, head_dim=128, rows=1, past=5000, capacity=cap, seed=31)
    wp = W.make("graph_prefill", heads=16, kv_heads=2, head_dim=128, rows=100, past=5000, capacity=cap, seed=32)
    other = W.make("graph_other", heads=16, kv_heads=2, head_dim=128, rows=200, past=3000, capacity=cap, seed=33)
    plan = hsdpa.Plan(16, 8, 128, cap)
    want_d, want_p, want_o = alone(torch, plan, wd), alone(torch, plan, wp), alone(torch, plan, other)
    bd, bp, bo = dev_tensors(torch, wd), dev_tensors(torch, wp), dev_tensors(torch, other)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())

    def step():
        hsdpa.attention_torch(plan, *bd[:3], bd[3], wd.rows, wd.past, wd.scale, ws, st)
        hsdpa.attention_torch(plan, *bp[:3], bp[3], wp.rows, wp.past, wp.scale, ws, st)

    with torch.cuda.stream(st):
        step()                                      # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        step()
    torch.cuda.synchronize()
    for replay in range(3):
        bd[3].fill_(-1)
        bp[3].fill_(-1)
        torch.cuda.synchronize()
        with torch.cuda.stream(st):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(bd[3].cpu(), want_d), f"replay {replay}: decode"
        assert torch.equal(bp[3].cpu(), want_p), f"replay {replay}: prefill"
        # eager work on the same workspace between replays
        bo[3].fill_(-1)
        st.wait_stream(torch.cuda.current_stream())
        hsdpa.attention_torch(plan, *bo[:3], bo[3], other.rows, other.past, other.scale, ws, st)
        torch.cuda.synchronize()
        assert torch.equal(bo[3].cpu(), want_o), f"after replay {replay}: eager call"


def test_graph_replays_prefill_forms(torch_cuda):
    """The prefill forms that launch several kernels or keep state in their
    workspace, captured in one graph on one workspace: the paired form (maxima,
    P.V, combine), the split form, and a short chunk of 29 key tiles (its P
    operands two rounds at a time). Each replay, with an eager call on the
    same workspace in between, equals the calls run alone."""
    torch = torch_cuda
    cap = 3000
    ws_ = [W.make("graph_paired", heads=16, kv_heads=2, head_dim=128, rows=3000, past=0, capacity=cap, seed=41),
           W.make("graph_split", heads=16, kv_heads=2, head_dim=128, rows=64, past=2000, capacity=cap, seed=42),
           W.make("graph_short", heads=16, kv_heads=2, head_dim=128, rows=512, past=400, capacity=cap, seed=43)]
    plan = hsdpa.Plan(16, 8, 128, cap)
    assert [plan.route(w.rows, w.past)["main"] for w in ws_] == ["causal_paired", "causal_split", "causal_short"]
    want = [alone(torch, plan, w) for w in ws_]
    bufs = [dev_tensors(torch, w) for w in ws_]
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())

    def step():
        for w, b in zip(ws_, bufs):
            hsdpa.attention_torch(plan, *b[:3], b[3], w.rows, w.past, w.scale, ws, st)

    with torch.cuda.stream(st):
        step()                                      # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        step()
    torch.cuda.synchronize()
    for replay in range(3):
        for b in bufs:
            b[3].fill_(-1)
        torch.cuda.synchronize()
        with torch.cuda.stream(st):
            graph.replay()
        torch.cuda.synchronize()
        for w, b, x in zip(ws_, bufs, want):
            assert torch.equal(b[3].cpu(), x), f"replay {replay}: {w.name}"
        # the paired call again, eagerly, on the same workspace
        b = bufs[0]
        b[3].fill_(-1)
        st.wait_stream(torch.cuda.current_stream())
        hsdpa.attention_torch(plan, *b[:3], b[3], ws_[0].rows, ws_[0].past, ws_[0].scale, ws, st)
        torch.cuda.synchronize()
        assert torch.equal(b[3].cpu(), want[0]), f"after replay {replay}: eager paired call"
