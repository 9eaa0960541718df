"""GPU parity of the softmax sink (SdpaShape::sink, src/jit/ir.rs:55-60)
through the C ABI: a plan with the sink flag, the call's sink value. The
reference's softmax with the sink (src/jit/target/x86/emit_sdpa/x86/decode.rs:
239-290) takes the maximum as vmaxss(hmax, sink), adds P(sink - M) to the sum
and multiplies by the sum's reciprocal; the oracle restates it (form
'chained_sink', pinned in test_sink_oracle.py). Every kernel family the
Chained form runs is covered: the decode passes (two passes and the combine,
pass 2 over every key, pass 2 over all groups, runs of keys per workgroup,
padded groups, the other head dimensions), the few-rows kernels, and the
causal prefill with the sink (one workgroup, split with the narrow and the
wide combine, paired). Sinks at and above the largest scores take a visible
share of each row (checked: the outputs then differ from the plain softmax's
by far more than the bar); a sink far below the scores leaves the plain
outputs. A Fused plan with the sink runs the Chained form, as the engine does
when the Fused form declines it (src/jit/emit_sdpa.rs:468-470)."""
import ctypes

import numpy as np
import pytest
import torch

import hsdpa
import oracle
from hsdpa import binding
from hsdpa import workloads as W
from parity import assert_parity, compare

from gpu_util import run_hsdpa

pytestmark = pytest.mark.gpu

# Scores of these workloads are about N(0, 1): the largest of n is about
# sqrt(2 ln n), and the sum of the exponentials about 1.65 n. A sink s takes
# the share e^s / (e^s + 1.65 n) of each row.
CASES = [
    # name, heads, kv_heads, head_dim, rows, past, sink, main kernels, sink dominant
    ("sink_decode_d256_n1", 8, 2, 256, 1, 0, 0.5, "decode", True),
    ("sink_decode_d256_n300_direct", 16, 2, 256, 1, 299, 6.0, "decode", True),
    ("sink_decode_d256_n20001_runs", 16, 2, 256, 1, 20000, 10.0, "decode", True),
    ("sink_decode_d128_n5000_g4", 16, 4, 128, 1, 4999, 9.0, "decode", True),
    ("sink_decode_d64_n777_g1", 4, 4, 64, 1, 776, 7.0, "decode", True),
    ("sink_decode_d256_g24_two_groups", 48, 2, 256, 1, 33000, 10.0, "decode", True),
    # between 8K and 16K keys pass 2 takes all groups of a KV head per workgroup
    ("sink_decode_d256_g24_all_groups", 48, 2, 256, 1, 12000, 10.0, "decode", True),
    ("sink_decode_d128_g17_padded", 17, 1, 128, 1, 900, 7.0, "decode", True),
    ("sink_decode_d96_n1000", 8, 2, 96, 1, 999, 7.0, "decode", True),
    ("sink_decode_d288_n300", 4, 2, 288, 1, 299, 6.0, "decode", True),
    ("sink_decode_moderate_d256_n4000", 16, 2, 256, 1, 3999, 2.0, "decode", False),
    ("sink_few_r3_d256_p37", 16, 2, 256, 3, 37, 4.0, "few_rows", True),
    ("sink_few_r5_d128_p900", 16, 2, 128, 5, 900, 7.0, "few_rows", True),
    # pass 2 walking a run for all groups: the sink term in workgroup 0's sums
    ("sink_few_r6_d256_p40000_all_chunked", 16, 2, 256, 6, 40000, 9.0, "few_rows", True),
    ("sink_prefill_r70_p5_d128_g1", 8, 8, 128, 70, 5, 4.0, "causal", True),
    ("sink_prefill_r40_p10_d96", 8, 2, 96, 40, 10, 4.0, "causal", True),
    ("sink_prefill_r20_p50_d384", 4, 1, 384, 20, 50, 4.0, "causal", True),
    ("sink_prefill_r512_d256_split4", 16, 4, 256, 512, 0, 5.0, "causal_split", True),
    ("sink_prefill_r100_p9000_d256_wide_combine", 8, 2, 256, 100, 9000, 9.0, "causal_split", True),
    ("sink_prefill_r64_p3000_d64_split", 8, 2, 64, 64, 3000, 8.0, "causal_split", True),
    ("sink_prefill_r4099_d128_paired", 8, 2, 128, 4099, 0, 6.0, "causal_paired", True),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_sink(torch_cuda, case):
    name, h, kvh, d, rows, past, sink, main, dominant = case
    w = W.make(name, heads=h, kv_heads=kvh, head_dim=d, rows=rows, past=past, seed=17)
    plan = hsdpa.Plan(w.heads, w.gqa, w.head_dim, w.capacity, sink=True)
    r = plan.route(rows, past)
    assert (r["main"], r["main_form"]) == (main, "chained"), r
    print(f"case {name} sink {sink}", flush=True)
    q = torch.from_numpy(np.ascontiguousarray(w.q).view(np.int16)).cuda()
    k = torch.from_numpy(np.ascontiguousarray(w.k).view(np.int16)).cuda()
    v = torch.from_numpy(np.ascontiguousarray(w.v).view(np.int16)).cuda()
    out = torch.full((w.rows, w.heads, w.head_dim), -1, dtype=torch.int16, device="cuda")
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    hsdpa.attention_torch(plan, q, k, v, out, w.rows, w.past, w.scale, ws, sink=sink)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    ref = oracle.attention(w, sink=sink)
    res = assert_parity(got, ref, w, name)
    print(name, res, flush=True)
    if dominant:
        # the sink's share moves the outputs well past the bar
        plain = compare(got, oracle.attention(w), w)
        assert plain["ulp1_share"] < 0.9, plain


def test_sink_far_below_the_scores_is_the_plain_softmax(torch_cuda):
    """A sink far below every score adds an exponential of about 1e-38: the
    outputs are the plain softmax's within the bar (decode and prefill)."""
    for rows, past in ((1, 3000), (48, 200)):
        w = W.make("sink_far", heads=16, kv_heads=2, head_dim=256, rows=rows, past=past, seed=5)
        plan = hsdpa.Plan(w.heads, w.gqa, w.head_dim, w.capacity, sink=True)
        q = torch.from_numpy(np.ascontiguousarray(w.q).view(np.int16)).cuda()
        k = torch.from_numpy(np.ascontiguousarray(w.k).view(np.int16)).cuda()
        v = torch.from_numpy(np.ascontiguousarray(w.v).view(np.int16)).cuda()
        out = torch.full((w.rows, w.heads, w.head_dim), -1, dtype=torch.int16, device="cuda")
        ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
        hsdpa.attention_torch(plan, q, k, v, out, w.rows, w.past, w.scale, ws, sink=-1e4)
        torch.cuda.synchronize()
        got = out.cpu().numpy().view(np.uint16)
        assert_parity(got, oracle.attention(w), w, f"sink far below, rows {rows}")


def test_sink_value_ignored_without_the_flag(torch_cuda):
    """Without the plan's sink flag the call's sink value is not read, as the
    reference's kernels without the sink ignore their sink argument: the
    outputs equal a call with sink 0, bit for bit."""
    w = W.make("sink_off", heads=16, kv_heads=2, head_dim=256, rows=1, past=2000, seed=6)
    plan = hsdpa.Plan(w.heads, w.gqa, w.head_dim, w.capacity)
    base = run_hsdpa(w, plan)
    q = torch.from_numpy(np.ascontiguousarray(w.q).view(np.int16)).cuda()
    k = torch.from_numpy(np.ascontiguousarray(w.k).view(np.int16)).cuda()
    v = torch.from_numpy(np.ascontiguousarray(w.v).view(np.int16)).cuda()
    out = torch.full((w.rows, w.heads, w.head_dim), -1, dtype=torch.int16, device="cuda")
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    hsdpa.attention_torch(plan, q, k, v, out, w.rows, w.past, w.scale, ws, sink=50.0)
    torch.cuda.synchronize()
    assert (out.cpu().numpy().view(np.uint16) == base).all()


def test_sink_fused_plan_runs_chained(torch_cuda):
    """A Fused plan with the sink computes the Chained form with the sink."""
    w = W.make("sink_fused", heads=16, kv_heads=2, head_dim=256, rows=1, past=5000, seed=8)
    fused = hsdpa.Plan(w.heads, w.gqa, w.head_dim, w.capacity, sink=True, form="fused")
    chained = hsdpa.Plan(w.heads, w.gqa, w.head_dim, w.capacity, sink=True)
    outs = []
    for plan in (fused, chained):
        q = torch.from_numpy(np.ascontiguousarray(w.q).view(np.int16)).cuda()
        k = torch.from_numpy(np.ascontiguousarray(w.k).view(np.int16)).cuda()
        v = torch.from_numpy(np.ascontiguousarray(w.v).view(np.int16)).cuda()
        out = torch.full((w.rows, w.heads, w.head_dim), -1, dtype=torch.int16, device="cuda")
        ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
        hsdpa.attention_torch(plan, q, k, v, out, w.rows, w.past, w.scale, ws, sink=8.0)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy().view(np.uint16))
    assert (outs[0] == outs[1]).all()
    assert_parity(outs[0], oracle.attention(w, sink=8.0), w, "sink fused plan")


def test_sink_frame_call_graph_replays(torch_cuda):
    """The frame call with the sink, captured once and replayed at successive
    pasts (rows and past read on the device), against the oracle."""
    h, kvh, d, cap, sink = 16, 2, 256, 40000, 9.0
    plan = hsdpa.Plan(h, h // kvh, d, cap, sink=True, max_rows=1)
    w = W.make("sink_frame", heads=h, kv_heads=kvh, head_dim=d, rows=1, past=32767, capacity=cap, seed=23)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()  # noqa: E731
    q, k, v = dev(w.q), dev(w.k), dev(w.v)
    out = torch.full((1, h, d), -1, dtype=torch.int16, device="cuda")
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    vals = torch.zeros(2, dtype=torch.int64, device="cuda")
    status = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    call = binding.FrameCall(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), vals.data_ptr(),
                             vals.data_ptr() + 8, w.scale, sink, ws.data_ptr(), plan.workspace_bytes,
                             status.data_ptr())
    lib = hsdpa.library()
    rc = lib.hsdpa_attention_frame(plan.handle, ctypes.byref(call),
                                   ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, binding.STATUS.get(rc)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.hsdpa_attention_frame(plan.handle, ctypes.byref(call),
                                       ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, binding.STATUS.get(rc)
    for past in (0, 1023, 5000, 32767):
        print(f"sink frame replay at past {past}", flush=True)
        vals.copy_(torch.tensor([1, past], dtype=torch.int64))
        out.fill_(-1)
        status.fill_(-1)
        graph.replay()
        torch.cuda.synchronize()
        assert int(status.item()) == 0, binding.STATUS.get(int(status.item()))
        got = out.cpu().numpy().view(np.uint16)
        wv = W.Workload("sink_frame", h, kvh, d, 1, past, cap, w.q, w.k, w.v, w.scale)
        assert_parity(got, oracle.attention(wv, sink=sink), wv, f"sink frame past {past}")


def test_sink_static_entry_matches(torch_cuda):
    """hsdpa_attention_static with the sink equals hsdpa_attention bit for bit."""
    plan = hsdpa.Plan(16, 8, 256, 8192, sink=True, max_rows=1)
    w = W.make("sink_static", heads=16, kv_heads=2, head_dim=256, rows=1, past=8000, capacity=8192, seed=9)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()  # noqa: E731
    q, k, v = dev(w.q), dev(w.k), dev(w.v)
    outs = []
    for static in (False, True):
        out = torch.full((1, 16, 256), -1, dtype=torch.int16, device="cuda")
        ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
        call = binding.Call(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), 1, w.past, w.scale, 7.5,
                            0 if static else ws.data_ptr(), 0 if static else plan.workspace_bytes)
        fn = hsdpa.library().hsdpa_attention_static if static else hsdpa.library().hsdpa_attention
        rc = fn(plan.handle, ctypes.byref(call), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert rc == 0, binding.STATUS.get(rc)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy().view(np.uint16))
    assert (outs[0] == outs[1]).all()
    assert_parity(outs[0], oracle.attention(w, sink=7.5), w, "sink static")


# A seeded sweep with the sink on: group shapes, head dimensions (tuned and
# not), rows and cached positions drawn at random (fixed seed), a Chained or a
# Fused plan (the latter runs the Chained form with the sink), and sink values
# from far below the scores to dominant.
SWEEP_GROUPS = [(8, 2), (16, 2), (16, 4), (12, 1), (6, 3), (34, 2), (24, 2), (4, 4), (10, 2), (64, 4)]
SWEEP_DIMS = [64, 128, 256, 256, 128, 32, 96, 160, 384]
SWEEP_ROWS = [1, 1, 1, 2, 3, 5, 8, 9, 16, 33, 64, 100, 257]
SWEEP_SINKS = [-40.0, -2.0, 0.0, 1.5, 3.0, 5.0, 8.0, 12.0]
SWEEP_SEED = 20261203
SWEEP_COUNT = 32
SWEEP_MAX_WORK = 1.5e8          # rows x keys x heads x head_dim: the oracle's sink form is scalar


def _sweep_draw():
    rng = np.random.default_rng(SWEEP_SEED)
    out = []
    while len(out) < SWEEP_COUNT:
        h, kvh = SWEEP_GROUPS[rng.integers(len(SWEEP_GROUPS))]
        d = int(SWEEP_DIMS[rng.integers(len(SWEEP_DIMS))])
        rows = int(SWEEP_ROWS[rng.integers(len(SWEEP_ROWS))])
        past = int([0, rng.integers(1, 64), rng.integers(64, 1100), rng.integers(1100, 12000)][rng.integers(4)])
        form = "fused" if rng.random() < 0.3 else "chained"
        sink = float(SWEEP_SINKS[rng.integers(len(SWEEP_SINKS))])
        if rows * (past + rows) * h * d > SWEEP_MAX_WORK:
            continue
        out.append((f"k{len(out):02d}_h{h}k{kvh}_d{d}_r{rows}_p{past}_{form}_s{sink:g}", h, kvh, d, rows, past, form,
                    sink))
    return out


SWEEP = _sweep_draw()

# the kernel families the draw reaches (main kernels, tail kernels, split over keys)
SWEEP_REACHED = {
    ("causal", "none", False),
    ("causal_split", "none", True),
    ("decode", "none", False),
    ("few_rows", "none", False),
}


def _sweep_plan(h, kvh, d, rows, past, form):
    return hsdpa.Plan(h, h // kvh, d, past + rows, form=form, sink=True)


def test_sink_sweep_reaches_the_kernel_families():
    """The draw reaches the decode, few-rows and causal kernels, split and
    not, every part on the Chained form (checked on the host, before the
    parity sweep)."""
    seen = set()
    for _, h, kvh, d, rows, past, form, _s in SWEEP:
        r = _sweep_plan(h, kvh, d, rows, past, form).route(rows, past)
        assert r["main_form"] == "chained" and r["tail_form"] == "chained", r
        seen.add((r["main"], r["tail"], r["splits"] > 1))
    assert SWEEP_REACHED <= seen, sorted(SWEEP_REACHED - seen)


def test_sink_sweep_parity(torch_cuda):
    """Each call against the oracle's sink form: no NaN, the per-row bound,
    a call of at least 4096 outputs at least 99.9 % of them within one ulp, a
    smaller one at most max(2, 1 %) past one ulp; pooled, at least 99.9 %."""
    from parity import ABS_FACTOR, ULP_SHARE

    within = total = 0
    for i, (name, h, kvh, d, rows, past, form, sink) in enumerate(SWEEP):
        w = W.make(name, heads=h, kv_heads=kvh, head_dim=d, rows=rows, past=past, seed=400 + i)
        plan = _sweep_plan(h, kvh, d, rows, past, form)
        print(f"case {name}", flush=True)
        q = torch.from_numpy(np.ascontiguousarray(w.q).view(np.int16)).cuda()
        k = torch.from_numpy(np.ascontiguousarray(w.k).view(np.int16)).cuda()
        v = torch.from_numpy(np.ascontiguousarray(w.v).view(np.int16)).cuda()
        out = torch.full((w.rows, w.heads, w.head_dim), -1, dtype=torch.int16, device="cuda")
        ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
        hsdpa.attention_torch(plan, q, k, v, out, w.rows, w.past, w.scale, ws, sink=sink)
        torch.cuda.synchronize()
        got = out.cpu().numpy().view(np.uint16)
        r = compare(got, oracle.attention(w, sink=sink), w)
        assert not r["nan"], (name, r)
        assert r["max_abs_over_vmax"] <= ABS_FACTOR, (name, r)
        n = got.size
        off = int(round((1.0 - r["ulp1_share"]) * n))
        if n >= 4096:
            assert r["ulp1_share"] >= ULP_SHARE, (name, r)
        else:
            assert off <= max(2, n // 100), (name, r)
        within += n - off
        total += n
    assert within / total >= ULP_SHARE, (within, total)
