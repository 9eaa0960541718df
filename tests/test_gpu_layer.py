"""GPU parity of the attention chain of one layer (hsdpa_attention_layer):
bit-exact against the same chain run as separate nodes through the C ABI
(head-norm-rope on q, on k, kv-append, attention, output gate), on every
buffer it writes; and, composed, against the oracle's restatements of those
nodes (norms, append and gate bit for bit, the attention within the parity
bar)."""
import numpy as np
import pytest

import kv_oracle
import oracle
from hsdpa import workloads as W
from parity import assert_parity

import hsdpa

pytestmark = pytest.mark.gpu


def bf(x):
    return W.f32_to_bf16(np.asarray(x, np.float32))


def rope_tables(positions, rotary, theta=1e7):
    half = max(rotary // 2, 1)
    inv = theta ** (-np.arange(half, dtype=np.float64) * 2.0 / max(rotary, 2))
    ang = np.arange(positions, dtype=np.float64)[:, None] * inv[None, :]
    return bf(np.cos(ang)), bf(np.sin(ang))


class Chain:
    """Seeded host buffers of one layer call: q [rows][q_row] (Q, then the gate
    when gated), k and v [rows][kv_heads*hd], the cache (positions < past hold
    earlier keys, the rest stale bytes), the norm weights and RoPE tables."""

    def __init__(self, heads, kvh, hd, rows, past, cap, gated, rotary, seed, kv_offset=0):
        rng = np.random.default_rng(seed)
        self.heads, self.kvh, self.hd, self.rows, self.past, self.cap = heads, kvh, hd, rows, past, cap
        self.gated, self.rotary, self.kv_offset = gated, rotary, kv_offset
        self.q_dim = heads * hd
        self.q_row = 2 * self.q_dim if gated else self.q_dim
        self.kv_row = kvh * hd
        self.q = bf(rng.normal(0, 2, rows * self.q_row))
        self.k = bf(rng.normal(0, 2, rows * self.kv_row))
        self.v = bf(rng.normal(0, 1, rows * self.kv_row))
        self.keys = bf(rng.normal(0, 1, kvh * cap * hd))
        self.values = bf(rng.normal(0, 1, kvh * cap * hd))
        self.q_norm = bf(rng.normal(0, 0.1, hd))
        self.k_norm = bf(rng.normal(0, 0.1, hd))
        self.cos, self.sin = rope_tables(cap, rotary)
        self.scale = float(np.float32(1.0 / np.sqrt(hd)))
        self.eps = 1e-6

    def device(self, torch):
        dev = torch.device("cuda")
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)
        o = self.kv_offset   # k and v may start o elements into their allocation
        pad = lambda a: t(np.concatenate([np.zeros(o, np.uint16), a]))[o:]
        return dict(q=t(self.q), k=pad(self.k), v=pad(self.v), keys=t(self.keys), values=t(self.values),
                    q_norm=t(self.q_norm), k_norm=t(self.k_norm), cos=t(self.cos), sin=t(self.sin),
                    out=torch.full((self.rows * self.q_dim,), -1, dtype=torch.int16, device=dev))

    def plan(self):
        return hsdpa.Plan(self.heads, self.heads // self.kvh, self.hd, self.cap, q_row=self.q_row)


def run_fused(torch, c, gated=None):
    gated = c.gated if gated is None else gated
    b = c.device(torch)
    plan = c.plan()
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    gate = b["q"][c.q_dim:] if gated else None
    hsdpa.attention_layer_torch(plan, b["q"], b["k"], b["v"], b["keys"], b["values"], b["out"], b["q_norm"],
                                b["k_norm"], b["cos"] if c.rotary else None, b["sin"] if c.rotary else None,
                                c.rows, c.past, c.scale, c.eps, ws, c.kv_row, c.rotary, gate=gate,
                                gate_row=c.q_row if gated else 0, positions=c.cap)
    torch.cuda.synchronize()
    return {n: b[n].cpu().numpy().view(np.uint16) for n in ("q", "k", "keys", "values", "out")}


def run_nodes(torch, c):
    b = c.device(torch)
    plan = c.plan()
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    cos = b["cos"] if c.rotary else None
    sin = b["sin"] if c.rotary else None
    hsdpa.head_norm_rope_torch(b["q"], b["q_norm"], cos, sin, c.heads, c.hd, c.hd, c.q_row, c.rotary, c.rows, c.past,
                               c.eps, positions=c.cap, table_row=c.rotary // 2)
    hsdpa.head_norm_rope_torch(b["k"], b["k_norm"], cos, sin, c.kvh, c.hd, c.hd, c.kv_row, c.rotary, c.rows, c.past,
                               c.eps, positions=c.cap, table_row=c.rotary // 2)
    spec = hsdpa.kv_spec(c.kvh, c.hd, c.cap, c.rows)
    hsdpa.kv_append_torch(spec, b["keys"], b["values"], b["k"], b["v"], c.rows, c.past)
    hsdpa.attention_torch(plan, b["q"], b["keys"], b["values"], b["out"], c.rows, c.past, c.scale, ws)
    if c.gated:
        hsdpa.output_gate_torch(b["out"], b["q"][c.q_dim:], c.q_dim, c.q_dim, c.q_row, c.rows)
    torch.cuda.synchronize()
    return {n: b[n].cpu().numpy().view(np.uint16) for n in ("q", "k", "keys", "values", "out")}


CASES = [
    # name, heads, kv_heads, head_dim, rows, past, capacity, gated, rotary
    ("decode_qwen_8k", 16, 2, 256, 1, 8191, 8192, True, 64),
    ("prefill_qwen_512_after_1000", 16, 2, 256, 512, 1000, 1600, True, 64),
    ("prefill_short_gated_96_after_160", 16, 2, 256, 96, 160, 300, True, 64),
    ("decode_ungated_d128_g4", 8, 2, 128, 1, 300, 400, False, 128),
    ("decode_direct_gated_qwen_1k", 16, 2, 256, 1, 1023, 1100, True, 64),       # pass 2 gates the outputs
    ("prefill_ragged_d64_g2", 8, 4, 64, 70, 33, 200, True, 32),
    ("decode_g16_no_rope", 16, 1, 256, 1, 5000, 5100, True, 0),
    ("decode_g32_two_groups", 32, 1, 128, 1, 700, 800, True, 64),
    ("decode_g17_through_prefill", 17, 1, 128, 1, 700, 800, True, 64),
    # a few rows after a cache: the decode kernels, gate rows gate_row apart
    ("few_rows_qwen_4_after_3000", 16, 2, 256, 4, 3000, 3100, True, 64),
    ("few_rows_d128_3_after_50", 8, 2, 128, 3, 50, 80, True, 128),
    # k and v 2 bytes off: the decode takes the separate element launch
    ("decode_unaligned_kv", 16, 2, 256, 1, 1000, 1100, True, 64, 1),
    # head dimensions outside 64/128/256: the generic norm path and the other
    # attention instantiations
    ("decode_d160_gated", 8, 2, 160, 1, 900, 1000, True, 32),
    ("prefill_d96_r40_after_60", 8, 4, 96, 40, 60, 120, True, 64),
    ("decode_d512_ungated", 4, 1, 512, 1, 300, 400, False, 128),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_layer_equals_the_nodes(torch_cuda, case):
    name, heads, kvh, hd, rows, past, cap, gated, rotary = case[:9]
    print(f"layer case {name}", flush=True)
    c = Chain(heads, kvh, hd, rows, past, cap, gated, rotary, seed=len(name), kv_offset=case[9] if len(case) > 9 else 0)
    fused = run_fused(torch_cuda, c)
    nodes = run_nodes(torch_cuda, c)
    for n in ("q", "k", "keys", "values", "out"):
        assert np.array_equal(fused[n], nodes[n]), f"{name}: {n} differs at {np.flatnonzero(fused[n] != nodes[n])[:8]}"


@pytest.mark.parametrize("rows,past", [(1, 2047), (96, 500)])
def test_layer_against_the_oracle(torch_cuda, rows, past):
    """The chain composed from the oracle's nodes: q and k normalised and
    rotated, the append, the attention on the result, the gate."""
    c = Chain(16, 2, 256, rows, past, past + rows + 16, True, 64, seed=rows + past)
    ungated = run_fused(torch_cuda, c, gated=False)
    gated = run_fused(torch_cuda, c)
    q_o = oracle.head_norm_rope(c.q, c.q_norm, c.cos, c.sin, rows, past, c.heads, c.hd, c.hd, c.q_row, c.rotary,
                                c.eps)
    k_o = oracle.head_norm_rope(c.k, c.k_norm, c.cos, c.sin, rows, past, c.kvh, c.hd, c.hd, c.kv_row, c.rotary,
                                c.eps)
    keys_o, values_o = c.keys.copy(), c.values.copy()
    kv_oracle.kv_append(keys_o, values_o, k_o, c.v, c.kvh, c.hd, c.cap * c.hd, rows, past)
    for got in (ungated, gated):
        assert np.array_equal(got["q"], q_o) and np.array_equal(got["k"], k_o)
        assert np.array_equal(got["keys"], keys_o) and np.array_equal(got["values"], values_o)
    qa = q_o.reshape(rows, c.q_row)[:, :c.q_dim].reshape(rows, c.heads, c.hd)
    w = W.Workload("layer", c.heads, c.kvh, c.hd, rows, past, c.cap, np.ascontiguousarray(qa),
                   keys_o.reshape(c.kvh, c.cap, c.hd), values_o.reshape(c.kvh, c.cap, c.hd), c.scale)
    ref = oracle.attention(w)
    r = assert_parity(ungated["out"].reshape(rows, c.heads, c.hd), ref, w, "layer")
    print("layer", rows, past, r, flush=True)
    gate = c.q.reshape(rows, c.q_row)[:, c.q_dim:]
    want = oracle.sigmoid_mul(ungated["out"].reshape(rows, c.q_dim), np.ascontiguousarray(gate))
    assert np.array_equal(gated["out"].reshape(rows, c.q_dim), want)
