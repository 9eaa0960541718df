"""GPU parity of the KV snapshot copies (hsdpa_kv_take / hsdpa_kv_restore
through the C ABI, driven by KvCache) against the oracle's restatement of the
reference's snapshot_take / restore_from loops: bit-exact, nothing outside the
copied positions touched, through the byte format and back, from pinned and
pageable slots, and a restored cache feeding the attention."""
import io

import numpy as np
import pytest

import kv_oracle
import oracle
from hsdpa import workloads as W
from hsdpa.snapshot import Instantaneous, KvCache, read_chat, write_chat
from parity import assert_parity

import hsdpa

pytestmark = pytest.mark.gpu

# n_kv_heads, kv_reserve_tokens, per-layer head_dim (0 = a layer without cache), max_positions, pos
CASES = [
    ("mixed_layers", 2, 300, [128, 0, 256, 64], 280, 257),
    ("one_position", 4, 64, [256], 64, 1),
    ("full_reserve", 1, 512, [100, 256], 512, 512),          # head_dim 100: odd row pitch in bytes / 16
    ("qwen_like", 2, 8192 + 128, [256, 0, 0, 0, 256], 8192 + 64, 8192 + 3),
]


def fill(torch, cache, rng):
    host = rng.integers(0, 1 << 16, cache.kv.numel(), dtype=np.uint16)
    cache.kv.copy_(torch.from_numpy(host.view(np.int16)))
    return host


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_take_and_restore_bit_exact(torch_cuda, case):
    torch = torch_cuda
    name, nkv, reserve, dims, maxp, pos = case
    print(f"snapshot case {name}", flush=True)
    rng = np.random.default_rng(len(name))
    cache = KvCache(nkv, reserve, dims, dn_conv_len=6, logits_len=5)
    live = fill(torch, cache, rng)
    cache.pos = pos
    cache.dn_conv[:] = rng.standard_normal(6)
    cache.logits[:] = rng.integers(0, 1 << 16, 5)
    s = cache.snapshot_reserve(maxp)
    s.kv[:] = rng.integers(0, 1 << 16, s.kv.size, dtype=np.uint16)   # stale bytes beyond pos must stay
    want = s.kv.copy()
    kv_oracle.snapshot_take(live, cache.kv_offsets, cache.kv_strides, reserve, nkv, want, s.snap_offsets,
                            s.snap_positions, pos)
    cache.snapshot_take(s)
    assert s.is_filled() and s.pos() == pos
    assert np.array_equal(s.kv, want), f"{name}: take differs at {np.flatnonzero(s.kv != want)[:8]}"
    assert np.array_equal(s.dn_conv, cache.dn_conv) and np.array_equal(s.logits, cache.logits)

    # restore a shorter prefix into a cache of other bytes
    p = max(pos // 2, 1)
    garbage = fill(torch, cache, np.random.default_rng(99))
    cache.pos = 0
    want_live = garbage.copy()
    kv_oracle.restore_from(want_live, cache.kv_offsets, cache.kv_strides, reserve, nkv, s.kv, s.snap_offsets,
                           s.snap_positions, p)
    cache.restore_from(s, p)
    got = cache.kv.cpu().numpy().view(np.uint16)
    assert cache.pos == p
    assert np.array_equal(got, want_live), f"{name}: restore differs at {np.flatnonzero(got != want_live)[:8]}"


def test_restore_through_the_byte_format_and_pinned_slots(torch_cuda):
    torch = torch_cuda
    rng = np.random.default_rng(4)
    cache = KvCache(2, 1024, [256, 128], logits_len=7)
    live = fill(torch, cache, rng)
    cache.pos = 1000
    for pinned in (False, True):
        s = cache.snapshot_reserve(1024, pinned=pinned)
        cache.snapshot_take(s)
        t = Instantaneous.from_bytes(s.to_bytes())
        fresh = KvCache(2, 1024, [256, 128], logits_len=7)
        fresh.restore_from(t, t.pos())
        got = fresh.kv.cpu().numpy().view(np.uint16)
        want = np.zeros_like(live)
        kv_oracle.restore_from(want, cache.kv_offsets, cache.kv_strides, 1024, 2, t.kv, t.snap_offsets,
                               t.snap_positions, 1000)
        assert np.array_equal(got, want), f"pinned={pinned}"
        # and the restored prefix is the original cache's
        for l in range(2):
            k0, k1 = cache.keys(l)[:, :1000 * cache.layer_head_dim(l)], fresh.keys(l)[:, :1000 * cache.layer_head_dim(l)]
            assert torch.equal(k0, k1)


def test_chat_file_restores_into_a_cache(torch_cuda):
    torch = torch_cuda
    cache = KvCache(1, 64, [128], logits_len=3)
    fill(torch, cache, np.random.default_rng(8))
    cache.pos = 40
    s = cache.snapshot_reserve(64)
    cache.snapshot_take(s)
    b = io.BytesIO()
    write_chat(b, "qwen3_5", 248320, list(range(40)), False, True, s)
    fresh = KvCache(1, 64, [128], logits_len=3)
    c = read_chat(io.BytesIO(b.getvalue()), "qwen3_5", 248320, cache=fresh)
    assert fresh.pos == 40 and c.ledger.tolist() == list(range(40))
    assert torch.equal(fresh.keys(0)[:, :40 * 128], cache.keys(0)[:, :40 * 128])
    assert torch.equal(fresh.values(0)[:, :40 * 128], cache.values(0)[:, :40 * 128])


@pytest.mark.parametrize("rows,past", [(1, 8191), (64, 4032)])
def test_restored_cache_feeds_the_attention(torch_cuda, rows, past):
    """A cache saved as a snapshot file (8 192 positions of a 2-KV-head, head_dim
    256 layer), read back and restored into the device cache, then the
    attention over it: equal to the oracle's attention on the original K/V."""
    torch = torch_cuda
    w = W.make("restore_then_attend", heads=16, kv_heads=2, head_dim=256, rows=rows, past=past, seed=rows)
    hd, kvh, cap = w.head_dim, w.kv_heads, w.capacity
    n = past + rows
    # the snapshot of a one-layer cache reserved at `cap` positions, filled to n
    snap_kv = np.concatenate([np.ascontiguousarray(w.k).reshape(-1), np.ascontiguousarray(w.v).reshape(-1)])
    s = Instantaneous([0, 2 * kvh * cap * hd], [0, 2 * kvh * cap * hd], [cap], snap_kv.astype(np.uint16),
                      np.zeros(0, np.float32), np.zeros(0, np.float32), np.zeros(0, np.uint16), n, True)
    t = Instantaneous.from_bytes(s.to_bytes())
    cache = KvCache(kvh, cap, [hd])
    cache.kv.fill_(0x7FC0)                         # NaN bf16 everywhere before the restore
    cache.restore_from(t, n)
    plan = hsdpa.Plan(w.heads, w.gqa, hd, cap)
    dev = torch.device("cuda")
    q = torch.from_numpy(np.ascontiguousarray(w.q).view(np.int16)).to(dev)
    out = torch.full((w.rows, w.heads, hd), -1, dtype=torch.int16, device=dev)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=dev)
    hsdpa.attention_torch(plan, q, cache.keys(0).reshape(-1), cache.values(0).reshape(-1), out, w.rows, w.past,
                          w.scale, ws)
    torch.cuda.synchronize()
    ref = oracle.attention(w)
    r = assert_parity(out.cpu().numpy().view(np.uint16), ref, w, "restore_then_attend")
    print("restore_then_attend", rows, past, r, flush=True)
