"""GPU parity of the element nodes around the attention, through the C ABI,
against the oracle's restatements: head RMS norm + RoPE (in place on q and k)
and the output gate. Bit-exact: the kernels follow the emitted operation
order, so every output bf16 must equal the oracle's."""
import numpy as np
import pytest

import oracle
from hsdpa import workloads as W

import hsdpa

pytestmark = pytest.mark.gpu


def bf(x):
    return W.f32_to_bf16(np.asarray(x, np.float32))


def rope_tables(positions, rotary, theta=1e7):
    half = rotary // 2
    inv = theta ** (-np.arange(half, dtype=np.float64) * 2.0 / rotary)
    ang = np.arange(positions, dtype=np.float64)[:, None] * inv[None, :]
    return bf(np.cos(ang)), bf(np.sin(ang))


def special_rows(rng, hd):
    """Rows that stress the edges: zeros, denormals (zero in the sum of
    squares, not in the product), huge values, a NaN, one dominant element."""
    z = np.zeros(hd, np.uint16)
    den = rng.integers(1, 0x7F, hd).astype(np.uint16) | (rng.integers(0, 2, hd).astype(np.uint16) << 15)
    huge = bf(rng.normal(0, 1e30, hd))
    nan = bf(rng.normal(0, 1, hd)); nan[5] = 0x7FC0
    dom = np.full(hd, bf([1.0])[0], np.uint16); dom[0] = bf([4096.0])[0]
    return [z, den, huge, nan, dom]


NR_CASES = [
    # name, heads, head_dim, head_stride, row_stride, rotary, rows, past, plus_one
    ("q_prefill_gated", 16, 256, 256, 2 * 16 * 256, 64, 4096, 8192, 1),
    ("k_prefill", 2, 256, 256, 2 * 256, 64, 4096, 8192, 1),
    ("q_decode_gated", 16, 256, 256, 2 * 16 * 256, 64, 1, 32767, 1),
    ("full_rope_d128", 4, 128, 160, 4 * 160 + 32, 128, 37, 3, 1),
    ("no_rope_d64_plain_w", 3, 64, 64, 192, 0, 20, 0, 0),
    ("d96_three_blocks", 2, 96, 96, 192, 32, 9, 100, 1),
]


@pytest.mark.parametrize("case", NR_CASES, ids=[c[0] for c in NR_CASES])
def test_head_norm_rope_bit_exact(torch_cuda, case):
    torch = torch_cuda
    name, heads, hd, hs, rs, rot, rows, past, plus = case
    print(f"norm-rope case {name}", flush=True)
    rng = np.random.default_rng(len(name) * 7 + rows)
    data = bf(rng.normal(0, rng.uniform(0.5, 8), rows * rs))
    if rows >= 8:   # a few special rows, first head of rows 1..5
        for i, srow in enumerate(special_rows(rng, hd)):
            data[(i + 1) * rs:(i + 1) * rs + hd] = srow
    w = bf(rng.normal(0, 0.1, hd))
    positions = past + rows + 5
    cos, sin = rope_tables(positions, rot) if rot else (np.zeros(1, np.uint16), np.zeros(1, np.uint16))
    ref = oracle.head_norm_rope(data, w, cos, sin, rows, past, heads, hd, hs, rs, rot, 1e-6, bool(plus))
    dev = torch.device("cuda")
    t = torch.from_numpy(data.view(np.int16)).to(dev)
    tw = torch.from_numpy(w.view(np.int16)).to(dev)
    tc = torch.from_numpy(np.ascontiguousarray(cos).reshape(-1).view(np.int16)).to(dev)
    ts = torch.from_numpy(np.ascontiguousarray(sin).reshape(-1).view(np.int16)).to(dev)
    hsdpa.head_norm_rope_torch(t, tw, tc, ts, heads, hd, hs, rs, rot, rows, past, 1e-6, bool(plus),
                               table_row=max(rot // 2, 1), positions=positions)
    torch.cuda.synchronize()
    got = t.cpu().numpy().view(np.uint16)
    diff = np.flatnonzero(got != ref)
    assert diff.size == 0, f"{name}: {diff.size} differ, first at {diff[:6]}: {got[diff[:6]]} vs {ref[diff[:6]]}"


@pytest.mark.parametrize("rows,width,attn_row,gate_row", [(4096, 4096, 4096, 8192), (1, 4096, 4096, 8192),
                                                          (33, 100, 128, 300)])
def test_output_gate_bit_exact(torch_cuda, rows, width, attn_row, gate_row):
    torch = torch_cuda
    print(f"gate case rows {rows} width {width}", flush=True)
    rng = np.random.default_rng(rows + width)
    attn = bf(rng.normal(0, 2, rows * attn_row))
    q = bf(rng.normal(0, 4, rows * gate_row + width))
    gate_off = gate_row - width if gate_row >= 2 * width else 0
    specials = bf([0.0, -0.0, 88.5, -88.5, 100.0, -100.0, np.inf, -np.inf, np.nan, 1e-40, 3.0e38])
    q[gate_off:gate_off + specials.size] = specials
    attn[:specials.size] = bf([1.0] * specials.size)
    ref = attn.copy()
    for r in range(rows):
        a = attn[r * attn_row:r * attn_row + width]
        g = q[gate_off + r * gate_row:gate_off + r * gate_row + width]
        ref[r * attn_row:r * attn_row + width] = oracle.sigmoid_mul(a, g)
    dev = torch.device("cuda")
    ta = torch.from_numpy(attn.view(np.int16)).to(dev)
    tq = torch.from_numpy(q.view(np.int16)).to(dev)
    hsdpa.output_gate_torch(ta, tq[gate_off:], width, attn_row, gate_row, rows)
    torch.cuda.synchronize()
    got = ta.cpu().numpy().view(np.uint16)
    diff = np.flatnonzero(got != ref)
    assert diff.size == 0, f"{diff.size} differ, first at {diff[:6]}: {got[diff[:6]]} vs {ref[diff[:6]]}"
