"""GPU parity with the strides of AttentionSpec away from their dense values
(abi.rs:136-180): q heads q_head apart inside rows q_row apart, output rows
out_row apart, KV heads kv_stride apart in the cache (room between heads). The
same seeded workload is laid out densely for the oracle and padded for the
GPU; the padding of the output must stay untouched."""
import numpy as np
import pytest

import oracle
from hsdpa import workloads as W
from parity import assert_parity

import hsdpa

pytestmark = pytest.mark.gpu

CASES = [
    # name, heads, kv_heads, head_dim, rows, past
    ("decode_d256", 16, 2, 256, 1, 5000),
    ("decode_d128_g16", 16, 1, 128, 1, 900),
    ("prefill_d256", 16, 2, 256, 80, 200),
    ("prefill_d128_split", 16, 4, 128, 40, 3000),      # the split causal kernel
    ("prefill_d96_more", 8, 2, 96, 70, 100),           # the other head dims' unit
    ("few_rows_d256_r3", 16, 2, 256, 3, 900),          # (row, head) columns on the decode kernels
]

SENTINEL = np.uint16(0x7E5A)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_padded_strides(torch_cuda, case):
    torch = torch_cuda
    name, h, kvh, d, rows, past = case
    print(f"case {name}", flush=True)
    w = W.make(name, heads=h, kv_heads=kvh, head_dim=d, rows=rows, past=past, seed=d + rows)
    q_head, q_row = d + 32, h * (d + 32) + 64               # multiples of 8 elements
    out_row = h * d + 128
    cap = w.capacity
    kv_stride = (cap + 37) * d
    qp = np.full((rows, q_row), 0x3F80, np.uint16)          # padding reads as 1.0: must not matter
    for hh in range(h):
        qp[:, hh * q_head:hh * q_head + d] = w.q[:, hh, :]
    kp = np.full((kvh, kv_stride), 0x7FC0, np.uint16)       # NaN between heads: must never be read
    vp = np.full((kvh, kv_stride), 0x7FC0, np.uint16)
    for g in range(kvh):
        kp[g, :cap * d] = w.k[g].reshape(-1)
        vp[g, :cap * d] = w.v[g].reshape(-1)
    dev = torch.device("cuda")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)
    out = t(np.full((rows, out_row), SENTINEL, np.uint16))
    plan = hsdpa.Plan(h, h // kvh, d, cap, q_row=q_row, q_head=q_head, out_row=out_row, kv_stride=kv_stride)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=dev)
    hsdpa.attention_torch(plan, t(qp), t(kp), t(vp), out, rows, past, w.scale, ws)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    assert (got[:, h * d:] == SENTINEL).all(), "output padding written"
    ref = oracle.attention(w)
    r = assert_parity(got[:, :h * d].reshape(rows, h, d), ref, w, name)
    print(name, r, flush=True)
