"""GPU parity of the KV append (hsdpa_kv_append through the C ABI) against the
oracle's restatement of the reference's append: bit-exact copies, nothing
outside the block's positions touched, both the vector and the scalar path,
and the append feeding the attention."""
import numpy as np
import pytest

import kv_oracle
import oracle
from hsdpa import workloads as W
from parity import assert_parity

import hsdpa

pytestmark = pytest.mark.gpu

CASES = [
    # name, heads, head_dim, capacity, pad (stride - capacity*head_dim), rows, past, offset (elements)
    ("prefill_4096_after_8192", 2, 256, 12288 + 64, 0, 4096, 8192, 0),
    ("decode_row", 2, 256, 32768, 0, 1, 32767, 0),
    ("ragged_head_dim", 3, 100, 300, 7, 57, 200, 0),          # scalar path: head_dim % 8 != 0
    ("unaligned_input", 4, 128, 512, 0, 33, 17, 1),           # scalar path: inputs 2 bytes off
    ("padded_stride", 2, 64, 1000, 40, 999, 1, 0),            # vector path, stride > capacity*head_dim
]


def run_case(torch, heads, hd, cap, pad, rows, past, off, seed):
    rng = np.random.default_rng(seed)
    stride = cap * hd + pad
    keys0 = rng.integers(0, 1 << 16, heads * stride, dtype=np.uint16)
    values0 = rng.integers(0, 1 << 16, heads * stride, dtype=np.uint16)
    ik = rng.integers(0, 1 << 16, rows * heads * hd, dtype=np.uint16)
    iv = rng.integers(0, 1 << 16, rows * heads * hd, dtype=np.uint16)
    dev = torch.device("cuda")
    tk = torch.from_numpy(keys0.view(np.int16)).to(dev)
    tv = torch.from_numpy(values0.view(np.int16)).to(dev)
    # inputs at an element offset `off` inside a larger buffer
    tik = torch.from_numpy(np.concatenate([np.zeros(off, np.uint16), ik]).view(np.int16)).to(dev)[off:]
    tiv = torch.from_numpy(np.concatenate([np.zeros(off, np.uint16), iv]).view(np.int16)).to(dev)[off:]
    spec = hsdpa.kv_spec(heads, hd, cap, max(rows, 1), stride=stride)
    hsdpa.kv_append_torch(spec, tk, tv, tik, tiv, rows, past)
    torch.cuda.synchronize()
    k_ref, v_ref = keys0.copy(), values0.copy()
    kv_oracle.kv_append(k_ref, v_ref, ik, iv, heads, hd, stride, rows, past)
    return tk.cpu().numpy().view(np.uint16), tv.cpu().numpy().view(np.uint16), k_ref, v_ref


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_kv_append_bit_exact(torch_cuda, case):
    name, heads, hd, cap, pad, rows, past, off = case
    print(f"kv case {name}", flush=True)
    k, v, k_ref, v_ref = run_case(torch_cuda, heads, hd, cap, pad, rows, past, off, seed=len(name))
    assert np.array_equal(k, k_ref), f"{name}: keys differ at {np.flatnonzero(k != k_ref)[:8]}"
    assert np.array_equal(v, v_ref), f"{name}: values differ at {np.flatnonzero(v != v_ref)[:8]}"


def test_kv_append_empty_block_touches_nothing(torch_cuda):
    k, v, k_ref, v_ref = run_case(torch_cuda, 2, 64, 128, 0, 0, 5, 0, seed=3)
    assert np.array_equal(k, k_ref) and np.array_equal(v, v_ref)


def test_append_then_attention(torch_cuda):
    """The node order of the reference (kv-append, then attention): a 96-row
    block appended after 160 cached positions, then the causal prefill over
    the cache, equals the oracle's attention on the oracle-appended cache."""
    torch = torch_cuda
    w = W.make("append_then_attend", heads=16, kv_heads=2, head_dim=256, rows=96, past=160, seed=31)
    hd, kvh, cap = w.head_dim, w.kv_heads, w.capacity
    stride = cap * hd
    rng = np.random.default_rng(5)
    # the block's new K/V rows, token-major, taken from the workload's own cache rows
    k_cache = np.ascontiguousarray(w.k).reshape(-1).copy()
    v_cache = np.ascontiguousarray(w.v).reshape(-1).copy()
    ik = np.stack([k_cache.reshape(kvh, cap, hd)[:, w.past + r, :] for r in range(w.rows)]).reshape(-1).copy()
    iv = np.stack([v_cache.reshape(kvh, cap, hd)[:, w.past + r, :] for r in range(w.rows)]).reshape(-1).copy()
    # the device cache starts with garbage at the block's positions
    k_dev0 = k_cache.copy().reshape(kvh, cap, hd)
    v_dev0 = v_cache.copy().reshape(kvh, cap, hd)
    k_dev0[:, w.past:w.past + w.rows, :] = rng.integers(0, 1 << 16, (kvh, w.rows, hd), dtype=np.uint16)
    v_dev0[:, w.past:w.past + w.rows, :] = rng.integers(0, 1 << 16, (kvh, w.rows, hd), dtype=np.uint16)
    dev = torch.device("cuda")
    tk = torch.from_numpy(k_dev0.reshape(-1).view(np.int16)).to(dev)
    tv = torch.from_numpy(v_dev0.reshape(-1).view(np.int16)).to(dev)
    spec = hsdpa.kv_spec(kvh, hd, cap, w.rows)
    hsdpa.kv_append_torch(spec, tk, tv, torch.from_numpy(ik.view(np.int16)).to(dev),
                          torch.from_numpy(iv.view(np.int16)).to(dev), w.rows, w.past)
    plan = hsdpa.Plan(w.heads, w.gqa, hd, cap)
    q = torch.from_numpy(np.ascontiguousarray(w.q).view(np.int16)).to(dev)
    out = torch.full((w.rows, w.heads, hd), -1, dtype=torch.int16, device=dev)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=dev)
    hsdpa.attention_torch(plan, q, tk, tv, out, w.rows, w.past, w.scale, ws)
    torch.cuda.synchronize()
    assert np.array_equal(tk.cpu().numpy().view(np.uint16), k_cache)
    ref = oracle.attention(w)
    r = assert_parity(out.cpu().numpy().view(np.uint16), ref, w, "append_then_attend")
    print("append_then_attend", r, flush=True)
