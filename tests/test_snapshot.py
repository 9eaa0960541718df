"""KV snapshot format and copies, host side: the byte format pinned on a
hand-written vector, round trips, every refusal of the reader (version,
truncation, the 64 GiB block ceiling), the conversation file around it, the
oracle's take/restore loops pinned on a self-naming cache, the Runner-level
refusals of KvCache, and the C ABI's refusals of hsdpa_kv_take /
hsdpa_kv_restore. No GPU needed; GPU parity is in test_gpu_snapshot.py."""
import ctypes
import io

import numpy as np
import pytest

import kv_oracle
from hsdpa import binding
from hsdpa.snapshot import (MAX_BLOCK_SNAPSHOT, Instantaneous, KvCache, SnapshotError, read_chat,
                            write_chat)

# A one-layer snapshot (1 KV head, 2 reserved positions, head_dim 2), written
# out field by field from the format's definition (model.rs:273-290).
TINY_HEX = (
    "01000000"                                                   # SNAPSHOT_FORMAT = 1, u32 LE
    "0200000000000000" "0000000000000000" "0800000000000000"     # kv_offsets = [0, 8]
    "0200000000000000" "0000000000000000" "0800000000000000"     # snap_offsets = [0, 8]
    "0100000000000000" "0200000000000000"                        # snap_positions = [2]
    "0800000000000000" "010a020b030c040d050e060f07100811"        # kv = 0x0a01, 0x0b02, ..., 0x1108
    "0100000000000000" "803f"                                    # logits = [0x3f80]
    "0000000000000000"                                           # dn_conv = []
    "0100000000000000" "0000c03f"                                # dn_recurrent = [1.5f]
    "0200000000000000"                                           # pos = 2
)
TINY_KV = [0x0A01, 0x0B02, 0x0C03, 0x0D04, 0x0E05, 0x0F06, 0x1007, 0x1108]


def tiny(filled=True):
    return Instantaneous([0, 8], [0, 8], [2], np.array(TINY_KV, np.uint16), np.zeros(0, np.float32),
                         np.array([1.5], np.float32), np.array([0x3F80], np.uint16), 2, filled)


def test_known_answer_bytes():
    assert tiny().to_bytes().hex() == TINY_HEX


def test_known_answer_read():
    s = Instantaneous.from_bytes(bytes.fromhex(TINY_HEX))
    assert s.kv_offsets == [0, 8] and s.snap_offsets == [0, 8] and s.snap_positions == [2]
    assert s.kv.dtype == np.uint16 and s.kv.tolist() == TINY_KV
    assert s.logits.tolist() == [0x3F80] and s.dn_conv.size == 0 and s.dn_recurrent.tolist() == [1.5]
    assert s.pos() == 2 and s.is_filled()
    keys, values = s.layer_kv(0, 1)
    assert keys.tolist() == [[[0x0A01, 0x0B02], [0x0C03, 0x0D04]]]
    assert values.tolist() == [[[0x0E05, 0x0F06], [0x1007, 0x1108]]]


def random_slot(rng, layers=(3, 0, 5), nkv=2, positions=7, conv=5, rec=4, logits=9, pos=6):
    offs, snap_offs, snap_pos, total, live = [0], [0], [], 0, 0
    for hd in layers:
        live += 2 * nkv * 16 * hd
        offs.append(live)
        cap = positions if hd else 0
        snap_pos.append(cap)
        total += 2 * nkv * cap * hd
        snap_offs.append(total)
    f32 = lambda n: rng.integers(0, 1 << 32, n, dtype=np.uint32).view(np.float32)  # any bits, NaNs included
    return Instantaneous(offs, snap_offs, snap_pos, rng.integers(0, 1 << 16, total, dtype=np.uint16), f32(conv),
                         f32(rec), rng.integers(0, 1 << 16, logits, dtype=np.uint16), pos, True)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_round_trip_is_bit_exact(seed):
    rng = np.random.default_rng(seed)
    s = random_slot(rng, conv=[0, 5, 17][seed], rec=[4, 0, 3][seed])
    data = s.to_bytes()
    assert len(data) == 4 + 3 * 8 + 8 * (len(s.kv_offsets) + len(s.snap_offsets) + len(s.snap_positions)) \
        + 4 * 8 + s.byte_size() + 8
    t = Instantaneous.from_bytes(data)
    assert (t.kv_offsets, t.snap_offsets, t.snap_positions, t.pos()) == \
        (s.kv_offsets, s.snap_offsets, s.snap_positions, s.pos())
    assert np.array_equal(t.kv, s.kv) and np.array_equal(t.logits, s.logits)
    assert np.array_equal(t.dn_conv.view(np.uint32), s.dn_conv.view(np.uint32))
    assert np.array_equal(t.dn_recurrent.view(np.uint32), s.dn_recurrent.view(np.uint32))
    assert t.to_bytes() == data


def test_file_round_trip(tmp_path):
    s = random_slot(np.random.default_rng(7))
    path = tmp_path / "slot.bin"
    with open(path, "wb") as f:
        s.write_to(f)
    with open(path, "rb") as f:
        t = Instantaneous.read(f)
        assert f.read() == b""                      # read consumes exactly the snapshot
    assert t.to_bytes() == s.to_bytes()


def test_empty_snapshot_write_is_refused_and_writes_nothing():
    b = io.BytesIO()
    with pytest.raises(SnapshotError) as e:
        tiny(filled=False).write_to(b)
    assert e.value.kind == "InvalidInput" and b.getvalue() == b""


@pytest.mark.parametrize("version", [0, 2, 0xFFFFFFFF])
def test_other_format_version_is_refused(version):
    data = version.to_bytes(4, "little") + bytes.fromhex(TINY_HEX)[4:]
    with pytest.raises(SnapshotError) as e:
        Instantaneous.from_bytes(data)
    assert e.value.kind == "InvalidData"


def test_every_truncation_is_an_unexpected_eof():
    data = bytes.fromhex(TINY_HEX)
    for n in range(len(data)):
        with pytest.raises(SnapshotError) as e:
            Instantaneous.from_bytes(data[:n])
        assert e.value.kind == "UnexpectedEof", n


class Unseekable:
    """A stream that can only read (a pipe): the reader must not allocate a
    claimed block before the bytes arrive."""

    def __init__(self, data):
        self.b = io.BytesIO(data)

    def read(self, n=-1):
        return self.b.read(n)


VERSION = (1).to_bytes(4, "little")
EMPTY_USIZES = (0).to_bytes(8, "little")


@pytest.mark.parametrize("stream", [io.BytesIO, Unseekable])
@pytest.mark.parametrize("field,count,kind", [
    ("usizes", (MAX_BLOCK_SNAPSHOT // 8) + 1, "InvalidData"),       # one element beyond the ceiling
    ("usizes", (1 << 64) - 1, "InvalidData"),                         # saturating product
    ("usizes", MAX_BLOCK_SNAPSHOT // 8, "UnexpectedEof"),             # exactly at the ceiling: accepted, then short
    ("kv", (MAX_BLOCK_SNAPSHOT // 2) + 1, "InvalidData"),
    ("kv", MAX_BLOCK_SNAPSHOT // 2, "UnexpectedEof"),
    ("f32", (MAX_BLOCK_SNAPSHOT // 4) + 1, "InvalidData"),
    ("f32", MAX_BLOCK_SNAPSHOT // 4, "UnexpectedEof"),
])
def test_block_ceiling(stream, field, count, kind):
    n = count.to_bytes(8, "little")
    if field == "usizes":
        data = VERSION + n
    elif field == "kv":
        data = VERSION + EMPTY_USIZES * 3 + n
    else:
        data = VERSION + EMPTY_USIZES * 3 + EMPTY_USIZES * 2 + n       # kv, logits empty; dn_conv huge
    with pytest.raises(SnapshotError) as e:
        Instantaneous.read(stream(data + b"\x00" * 64))
    assert e.value.kind == kind


def test_restorable_at():
    s = tiny()                           # dn_recurrent non-empty: only the exact position
    assert s.restorable_at(2) and not s.restorable_at(1) and not s.restorable_at(3)
    s.dn_recurrent = np.zeros(0, np.float32)
    assert s.restorable_at(0) and s.restorable_at(1) and s.restorable_at(2) and not s.restorable_at(3)
    s.clear()
    assert not s.restorable_at(0) and s.pos() == 0 and not s.is_filled()


def test_byte_accounting():
    s = tiny()
    assert s.byte_size() == 8 * 2 + 0 * 4 + 1 * 4 + 1 * 2
    assert s.bytes() == 2 * (8 + 1) + 4 * (0 + 1) + 8 * (2 + 2 + 1)
    assert "B)" in repr(s) and "2561" not in repr(s)


# ---- the conversation file ---------------------------------------------------

def test_chat_known_answer_and_round_trip():
    s = tiny()
    b = io.BytesIO()
    write_chat(b, "qwen3_5", 248320, [7, 0x01020304], True, False, s)
    data = b.getvalue()
    head = b"HERBERT-BF16-CHAT-1\nqwen3_5\n248320\n2\n1\n0\n"
    assert data[:len(head)] == head
    assert data[len(head):len(head) + 8] == bytes.fromhex("07000000" "04030201")
    assert data[len(head) + 8:] == bytes.fromhex(TINY_HEX)
    c = read_chat(io.BytesIO(data), "qwen3_5", 248320)
    assert (c.model_type, c.vocab_size, c.ledger.tolist(), c.assistant_open, c.tools_announced) == \
        ("qwen3_5", 248320, [7, 0x01020304], True, False)
    assert c.slot.to_bytes() == s.to_bytes()


def chat_bytes(header: bytes, ledger, slot=None):
    return header + np.asarray(ledger, "<u4").tobytes() + (slot or tiny()).to_bytes()


@pytest.mark.parametrize("header,expect", [
    (b"HERBERT-BF16-CHAT-2\nq\n10\n2\n0\n0\n", "not a saved conversation"),
    (b"HERBERT-BF16-CHAT-1\nq\nten\n2\n0\n0\n", "not a saved conversation"),
    (b"HERBERT-BF16-CHAT-1\nq\n10\n-2\n0\n0\n", "not a saved conversation"),
    (b"HERBERT-BF16-CHAT-1\nother\n10\n2\n0\n0\n", "saved from another model"),
    (b"HERBERT-BF16-CHAT-1\nq\n11\n2\n0\n0\n", "saved from another model"),
])
def test_chat_refusals(header, expect):
    with pytest.raises(SnapshotError) as e:
        read_chat(io.BytesIO(chat_bytes(header, [1, 2])), "q", 10)
    assert e.value.kind == "Backend" and expect in str(e.value)


def test_chat_header_parsing_follows_the_reference():
    # "+2" parses as a usize, "\r\n" ends a line like "\n", a flag other than "1" reads as false
    c = read_chat(io.BytesIO(chat_bytes(b"HERBERT-BF16-CHAT-1\r\nq\n10\n+2\r\nyes\n1\n", [1, 2])), "q", 10)
    assert c.ledger.tolist() == [1, 2] and not c.assistant_open and c.tools_announced


def test_chat_ledger_must_match_the_state():
    with pytest.raises(SnapshotError) as e:
        read_chat(io.BytesIO(chat_bytes(b"HERBERT-BF16-CHAT-1\nq\n10\n3\n0\n0\n", [1, 2, 3])))
    assert "the state holds 2 positions but the ledger 3 tokens" in str(e.value)


def test_chat_truncated():
    data = chat_bytes(b"HERBERT-BF16-CHAT-1\nq\n10\n2\n0\n0\n", [1, 2])
    for n in (0, 5, 30, 40, len(data) - 1):
        with pytest.raises(SnapshotError) as e:
            read_chat(io.BytesIO(data[:n]))
        assert e.value.kind == "UnexpectedEof"


# ---- the oracle's copy loops, pinned ----------------------------------------

def named_cache(nkv, reserve, dims):
    """A live cache whose every element names itself:
    l << 13 | half << 12 | h << 10 | p << 4 | d."""
    strides = [reserve * d for d in dims]
    offs = [0]
    for st in strides:
        offs.append(offs[-1] + 2 * nkv * st)
    kv = np.zeros(offs[-1], np.uint16)
    for l, d in enumerate(dims):
        for half in range(2):
            for h in range(nkv):
                for p in range(reserve):
                    for x in range(d):
                        kv[offs[l] + half * nkv * strides[l] + h * strides[l] + p * d + x] = \
                            l << 13 | half << 12 | h << 10 | p << 4 | x
    return kv, offs, strides


def test_oracle_take_known_answer():
    nkv, reserve, dims, cap, pos = 2, 8, [3, 0, 5], 6, 4
    kv, offs, strides = named_cache(nkv, reserve, dims)
    snap_pos = [cap if d else 0 for d in dims]
    snap_offs = [0]
    for l, d in enumerate(dims):
        snap_offs.append(snap_offs[-1] + 2 * nkv * snap_pos[l] * d)
    snap = np.full(snap_offs[-1], 0xFFFF, np.uint16)
    kv_oracle.snapshot_take(kv, offs, strides, reserve, nkv, snap, snap_offs, snap_pos, pos)
    for l, d in enumerate(dims):
        for half in range(2):
            for h in range(nkv):
                for p in range(snap_pos[l]):
                    for x in range(d):
                        got = snap[snap_offs[l] + half * nkv * cap * d + h * cap * d + p * d + x]
                        assert got == ((l << 13 | half << 12 | h << 10 | p << 4 | x) if p < pos else 0xFFFF)
    with pytest.raises(ValueError):
        kv_oracle.snapshot_take(kv, offs, strides, reserve, nkv, snap, snap_offs, snap_pos, cap + 1)


def test_oracle_restore_known_answer_and_take_restore_identity():
    nkv, reserve, dims, cap = 2, 8, [4, 0, 2], 7
    src, offs, strides = named_cache(nkv, reserve, dims)
    snap_pos = [cap if d else 0 for d in dims]
    snap_offs = [0]
    for l, d in enumerate(dims):
        snap_offs.append(snap_offs[-1] + 2 * nkv * snap_pos[l] * d)
    snap = np.zeros(snap_offs[-1], np.uint16)
    kv_oracle.snapshot_take(src, offs, strides, reserve, nkv, snap, snap_offs, snap_pos, 6)
    for p in (0, 1, 3, 6):
        live = np.full_like(src, 0xBEEF)
        # rows the live cache already holds are skipped (first_different_row) with the same end state
        live[offs[0]:offs[0] + 2 * dims[0]] = src[offs[0]:offs[0] + 2 * dims[0]]
        kv_oracle.restore_from(live, offs, strides, reserve, nkv, snap, snap_offs, snap_pos, p)
        for l, d in enumerate(dims):
            for half in range(2):
                for h in range(nkv):
                    a = offs[l] + half * nkv * strides[l] + h * strides[l]
                    assert np.array_equal(live[a:a + p * d], src[a:a + p * d])
                    tail = live[a + max(p, 2 if (l, half, h) == (0, 0, 0) else 0) * d:a + strides[l]]
                    assert np.all(tail == 0xBEEF), (p, l, half, h)


def test_first_different_row():
    a = np.arange(12, dtype=np.uint16)
    b = a.copy()
    assert kv_oracle.first_different_row(a, b, 3) == 4
    b[7] ^= 1
    assert kv_oracle.first_different_row(a, b, 3) == 2
    b[0] ^= 1
    assert kv_oracle.first_different_row(a, b, 3) == 0


# ---- KvCache on the host: geometry and refusals ------------------------------

def cpu_cache(**kw):
    d = dict(n_kv_heads=2, kv_reserve_tokens=8, layer_head_dims=[4, 0, 8], logits_len=3, device="cpu")
    d.update(kw)
    return KvCache(**d)


def test_cache_geometry_and_reserve():
    c = cpu_cache()
    assert c.kv_strides == [32, 0, 64] and c.kv_offsets == [0, 128, 128, 384] and c.kv.numel() == 384
    assert [c.layer_head_dim(l) for l in range(3)] == [4, 0, 8]
    s = c.snapshot_reserve(5)
    assert s.snap_positions == [5, 0, 5] and s.snap_offsets == [0, 80, 80, 240] and s.kv.size == 240
    assert s.kv_offsets == c.kv_offsets and not s.is_filled() and s.logits.size == 3
    assert c.snapshot_reserve(100).snap_positions == [8, 0, 8]   # min(reserve, max_positions)


def test_restore_refusals():
    c = cpu_cache()
    s = c.snapshot_reserve(8)
    with pytest.raises(SnapshotError, match="snapshot is empty"):
        c.restore_from(s, 0)
    s._is_filled, s._pos = True, 4
    with pytest.raises(SnapshotError, match="beyond snapshot"):
        c.restore_from(s, 5)
    other = cpu_cache(layer_head_dims=[4, 0, 16])
    with pytest.raises(SnapshotError, match="different Runner"):
        other.restore_from(s, 1)
    rec = cpu_cache(dn_recurrent_len=4)
    s2 = rec.snapshot_reserve(8)
    s2._is_filled, s2._pos = True, 4
    with pytest.raises(SnapshotError, match="only an EXACT prefix"):
        rec.restore_from(s2, 3)
    short = Instantaneous(s.kv_offsets, s.snap_offsets, s.snap_positions, s.kv[:-1], s.dn_conv, s.dn_recurrent,
                          s.logits, 4, True)
    with pytest.raises(SnapshotError, match="outside its KV block"):
        c.restore_from(short, 1)


def test_take_refusal_leaves_the_slot_empty():
    c = cpu_cache()
    s = c.snapshot_reserve(3)
    s._is_filled, s._pos = True, 2
    c.pos = 4
    with pytest.raises(SnapshotError, match="layer 0 holds 4 positions, the slot buffer holds 3"):
        c.snapshot_take(s)
    assert not s.is_filled()


# ---- the C ABI's refusals (host side) ---------------------------------------

def kv_spec_raw(heads=2, hd=128, cap=1024, r16=0):
    return binding.KvSpec(heads, hd, cap * hd, cap, 1, r16, 0)


def take_rc(spec, snap_positions, positions, ptr=16):
    return binding.library().hsdpa_kv_take(ctypes.byref(spec) if spec is not None else None, ptr, ptr, ptr,
                                           snap_positions, positions, None)


def restore_rc(spec, snap_positions, positions, ptr=16):
    return binding.library().hsdpa_kv_restore(ctypes.byref(spec) if spec is not None else None, ptr,
                                              snap_positions, ptr, ptr, positions, None)


@pytest.mark.parametrize("rc", [take_rc, restore_rc])
def test_snapshot_copy_refusals(rc):
    s = kv_spec_raw()
    ceiling = MAX_BLOCK_SNAPSHOT // (4 * 2 * 128)
    assert rc(s, 10, 11) == 6                    # more positions than the snapshot layer holds
    assert rc(s, 2000, 1025) == 6                # more positions than the live cache holds
    assert rc(s, ceiling + 1, 0) == 6            # a layer block beyond 64 GiB
    assert rc(s, ceiling, 0) == 0                # at the ceiling, nothing to copy
    assert rc(s, 10, 0, ptr=0) == 0              # nothing to copy: pointers unused
    assert rc(s, 10, 5, ptr=0) == 9
    assert rc(None, 10, 5) == 9
    assert rc(kv_spec_raw(r16=1), 10, 5) == 13
    assert rc(kv_spec_raw(heads=0), 10, 5) == 1


@pytest.mark.parametrize("rc", [take_rc, restore_rc])
def test_snapshot_copy_without_gpu_reports_no_device(rc):
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    assert rc(kv_spec_raw(), 10, 5) == 11
