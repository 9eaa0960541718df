"""The KV snapshot: the on-disk format of a frozen KV cache, and its copies
between host memory and the device cache.

`Instantaneous` is the reference's snapshot slot (src/jit/model.rs:186-326):
the geometry it was reserved for, the per-layer KV at the snapshot's
capacities, the two DeltaNet states, the last token's logits and the position.
Its byte format (write_to / read, model.rs:268-319) is, little-endian:

    u32 SNAPSHOT_FORMAT (= 1)
    u64 n, n x u64      kv_offsets      (write_usizes, model.rs:123-129)
    u64 n, n x u64      snap_offsets
    u64 n, n x u64      snap_positions
    u64 n, n x u16      kv              (write_u16s, model.rs:142-150)
    u64 n, n x u16      logits
    u64 n, n x f32      dn_conv         (write_f32s, model.rs:162-169)
    u64 n, n x f32      dn_recurrent
    u64                 pos

Every length is written, never inferred, and on reading each block is bounded
by MAX_BLOCK_SNAPSHOT (64 GiB, length() at model.rs:110-121) before anything
is allocated. Layer l's KV block sits at snap_offsets[l]:
K[n_kv_heads][snap_positions[l]][head_dim_l] then V in the same layout
(snapshot_reserve, model.rs:675-697).

`KvCache` is the KV part of the reference's Runner on the device (the layout
of model.rs:340-366 and 545-559: all layers in one buffer, layer l at
kv_offsets[l], keys then values, head h at h * kv_strides[l]) with its
snapshot API: snapshot_reserve, snapshot_take, restore_from
(model.rs:675-857). The per-layer KV copies run through the C ABI
(hsdpa_kv_take / hsdpa_kv_restore); the DeltaNet states and logits the format
carries are host arrays here, since the kernels that own them are not part of
this library.

`write_chat` / `read_chat` are the conversation file around a snapshot
(Chat::save / Chat::restore, src/chat/session.rs:320-391).
"""
from __future__ import annotations

import ctypes
import io
import re

import numpy as np

from .binding import kv_restore_raw, kv_spec, kv_take_raw

SNAPSHOT_FORMAT = 1            # model.rs:100-103
MAX_BLOCK_SNAPSHOT = 64 << 30  # model.rs:105-108
CHAT_MAGIC = "HERBERT-BF16-CHAT-1"  # session.rs:323
_CHUNK = 1 << 26


class SnapshotError(Exception):
    """A refused snapshot operation. `kind` is the reference's error kind:
    "InvalidData", "InvalidInput" or "UnexpectedEof" (std::io::ErrorKind of the
    format functions) or "Backend" (HerbertError::Backend of the Runner and
    Chat refusals)."""

    def __init__(self, kind: str, message: str):
        self.kind = kind
        super().__init__(f"{kind}: {message}")


# ---- primitive blocks -------------------------------------------------------

def _read_exact(r, n: int) -> bytes:
    """std::io::Read::read_exact: n bytes or UnexpectedEof."""
    parts = []
    left = n
    while left:
        b = r.read(min(left, _CHUNK))
        if not b:
            raise SnapshotError("UnexpectedEof", "failed to fill whole buffer")
        parts.append(b)
        left -= len(b)
    return b"".join(parts)


def _u64(r) -> int:
    return int.from_bytes(_read_exact(r, 8), "little")


def _length(r, element_size: int) -> int:
    """length(), model.rs:110-121: a u64 count whose block must stay within
    MAX_BLOCK_SNAPSHOT."""
    n = _u64(r)
    if n * element_size > MAX_BLOCK_SNAPSHOT:
        raise SnapshotError("InvalidData", f"block of {n} elements: beyond the ceiling")
    return n


def _remaining(r) -> int | None:
    """Bytes left in a seekable stream, None when it cannot say."""
    try:
        if not r.seekable():
            return None
        here = r.tell()
        end = r.seek(0, io.SEEK_END)
        r.seek(here, io.SEEK_SET)
        return end - here
    except (AttributeError, OSError, ValueError):
        return None


def _read_array(r, n: int, dtype: str) -> np.ndarray:
    """n little-endian elements into a fresh array. A seekable stream too short
    for the block is refused before allocating; otherwise the block is read in
    bounded chunks, so a corrupt length costs no more memory than the data
    that is really there."""
    item = np.dtype(dtype).itemsize
    nbytes = n * item
    left = _remaining(r)
    if left is not None and left < nbytes:
        raise SnapshotError("UnexpectedEof", "failed to fill whole buffer")
    if left is not None and hasattr(r, "readinto"):
        out = np.empty(n, dtype=dtype)
        view = memoryview(out).cast("B")
        got = 0
        while got < nbytes:
            k = r.readinto(view[got:min(nbytes, got + _CHUNK)])
            if not k:
                raise SnapshotError("UnexpectedEof", "failed to fill whole buffer")
            got += k
    else:
        out = np.frombuffer(bytearray(_read_exact(r, nbytes)), dtype=dtype)
    return out.astype(np.dtype(dtype).newbyteorder("="), copy=False)


def _read_usizes(r) -> list[int]:
    n = _length(r, 8)
    return [int(x) for x in _read_array(r, n, "<u8")]


def _write_usizes(w, v) -> None:
    w.write(len(v).to_bytes(8, "little"))
    w.write(np.asarray(v, dtype="<u8").tobytes())


def _write_block(w, v: np.ndarray, dtype: str) -> None:
    w.write(int(v.size).to_bytes(8, "little"))
    w.write(np.ascontiguousarray(v, dtype=dtype).tobytes())


# ---- the snapshot slot ------------------------------------------------------

class Instantaneous:
    """A frozen KV state at a position (model.rs:186-212). Filled by
    KvCache.snapshot_take, replayed by KvCache.restore_from, stored by
    write_to / read. The tokens that identify the state live with the caller."""

    def __init__(self, kv_offsets, snap_offsets, snap_positions, kv, dn_conv, dn_recurrent, logits, pos=0,
                 is_filled=False, pinned=None):
        self.kv_offsets = [int(x) for x in kv_offsets]
        self.snap_offsets = [int(x) for x in snap_offsets]
        self.snap_positions = [int(x) for x in snap_positions]
        self.kv = kv
        self.dn_conv = dn_conv
        self.dn_recurrent = dn_recurrent
        self.logits = logits
        self._pos = int(pos)
        self._is_filled = bool(is_filled)
        self._pinned = pinned  # the pinned torch tensor behind `kv`, kept alive

    def byte_size(self) -> int:
        """KV, DeltaNet conv and recurrent states, logits (model.rs:215-217)."""
        return self.kv.size * 2 + (self.dn_conv.size + self.dn_recurrent.size) * 4 + self.logits.size * 2

    def bytes(self) -> int:
        """Bytes reserved by the slot, geometry included (model.rs:247-253)."""
        return (2 * (self.kv.size + self.logits.size) + 4 * (self.dn_conv.size + self.dn_recurrent.size)
                + 8 * (len(self.kv_offsets) + len(self.snap_offsets) + len(self.snap_positions)))

    def pos(self) -> int:
        return self._pos

    def is_filled(self) -> bool:
        return self._is_filled

    def clear(self) -> None:
        """An empty slot again; the buffers stay reserved (model.rs:230-234)."""
        self._is_filled = False
        self._pos = 0

    def restorable_at(self, p: int) -> bool:
        """model.rs:321-325: any earlier position on a pure-attention state, only
        the exact one once a recurrent state is part of it."""
        return self._is_filled and p <= self._pos and (p == self._pos or self.dn_recurrent.size == 0)

    def layer_kv(self, l: int, n_kv_heads: int):
        """(keys, values) views of layer l's block, [n_kv_heads][snap_positions][head_dim]."""
        sp = self.snap_positions[l]
        a, b = self.snap_offsets[l], self.snap_offsets[l + 1]
        if sp == 0:
            return None, None
        hd = (b - a) // (2 * n_kv_heads * sp)
        block = self.kv[a:a + 2 * n_kv_heads * sp * hd]
        return block[:n_kv_heads * sp * hd].reshape(n_kv_heads, sp, hd), \
            block[n_kv_heads * sp * hd:].reshape(n_kv_heads, sp, hd)

    def __repr__(self) -> str:  # never the KV bytes (model.rs:176-187)
        return f"Instantaneous(pos={self._pos} filled={self._is_filled} {self.bytes()} B)"

    # ---- serialization (model.rs:268-319) ----

    def write_to(self, w) -> None:
        if not self._is_filled:
            raise SnapshotError("InvalidInput", "empty snapshot: nothing to write")
        w.write(SNAPSHOT_FORMAT.to_bytes(4, "little"))
        _write_usizes(w, self.kv_offsets)
        _write_usizes(w, self.snap_offsets)
        _write_usizes(w, self.snap_positions)
        _write_block(w, self.kv, "<u2")
        _write_block(w, self.logits, "<u2")
        _write_block(w, self.dn_conv, "<f4")
        _write_block(w, self.dn_recurrent, "<f4")
        w.write(self._pos.to_bytes(8, "little"))

    @classmethod
    def read(cls, r) -> "Instantaneous":
        if int.from_bytes(_read_exact(r, 4), "little") != SNAPSHOT_FORMAT:
            raise SnapshotError("InvalidData", "snapshot of another version of format")
        kv_offsets = _read_usizes(r)
        snap_offsets = _read_usizes(r)
        snap_positions = _read_usizes(r)
        kv = _read_array(r, _length(r, 2), "<u2")
        logits = _read_array(r, _length(r, 2), "<u2")
        dn_conv = _read_array(r, _length(r, 4), "<f4")
        dn_recurrent = _read_array(r, _length(r, 4), "<f4")
        pos = _u64(r)
        return cls(kv_offsets, snap_offsets, snap_positions, kv, dn_conv, dn_recurrent, logits, pos, True)

    def to_bytes(self) -> bytes:
        b = io.BytesIO()
        self.write_to(b)
        return b.getvalue()

    @classmethod
    def from_bytes(cls, data: bytes) -> "Instantaneous":
        return cls.read(io.BytesIO(data))


# ---- the live cache ---------------------------------------------------------

class KvCache:
    """The KV of every layer on the device, in the Runner's layout
    (model.rs:340-366, 545-559): one buffer of sum_l 2 * n_kv_heads *
    kv_strides[l] bf16, layer l at kv_offsets[l], keys then values, head h of
    a half at h * kv_strides[l], kv_strides[l] = kv_reserve_tokens *
    head_dim_l (0 for a layer without cache). `pos` is the number of
    positions held. dn_conv, dn_recurrent and logits are the other state a
    snapshot carries, host arrays of the given lengths."""

    def __init__(self, n_kv_heads: int, kv_reserve_tokens: int, layer_head_dims, dn_conv_len: int = 0,
                 dn_recurrent_len: int = 0, logits_len: int = 0, device="cuda"):
        import torch

        if n_kv_heads <= 0 or kv_reserve_tokens <= 0:
            raise ValueError("n_kv_heads and kv_reserve_tokens must be positive")
        self.n_kv_heads = int(n_kv_heads)
        self.kv_reserve_tokens = int(kv_reserve_tokens)
        self.kv_strides = [self.kv_reserve_tokens * int(h) for h in layer_head_dims]
        self.kv_offsets = [0]
        for st in self.kv_strides:
            self.kv_offsets.append(self.kv_offsets[-1] + 2 * self.n_kv_heads * st)
        self.n_layers = len(self.kv_strides)
        self.kv = torch.zeros(self.kv_offsets[-1], dtype=torch.int16, device=device)
        self.dn_conv = np.zeros(dn_conv_len, np.float32)
        self.dn_recurrent = np.zeros(dn_recurrent_len, np.float32)
        self.logits = np.zeros(logits_len, np.uint16)
        self.pos = 0

    def layer_head_dim(self, l: int) -> int:
        """model.rs:700-703."""
        return 0 if self.kv_strides[l] == 0 else self.kv_strides[l] // self.kv_reserve_tokens

    def keys(self, l: int):
        """Layer l's keys, [n_kv_heads][kv_reserve_tokens * head_dim] (a view)."""
        a, st = self.kv_offsets[l], self.kv_strides[l]
        return self.kv[a:a + self.n_kv_heads * st].view(self.n_kv_heads, st)

    def values(self, l: int):
        a, st = self.kv_offsets[l], self.kv_strides[l]
        return self.kv[a + self.n_kv_heads * st:a + 2 * self.n_kv_heads * st].view(self.n_kv_heads, st)

    def layer_spec(self, l: int):
        """The layer's KvSpec (heads, head_dim, stride, capacity), validated by the library."""
        return kv_spec(self.n_kv_heads, self.layer_head_dim(l), self.kv_reserve_tokens, 1, self.kv_strides[l])

    # ---- snapshots (model.rs:668-857) ----

    def snapshot_reserve(self, max_positions: int, pinned: bool = False) -> Instantaneous:
        """The only allocation of a snapshot slot (model.rs:675-697): each
        layer with a cache holds min(kv_reserve_tokens, max_positions)
        positions. `pinned` backs the KV with page-locked host memory."""
        snap_offsets, snap_positions, total = [0], [], 0
        for l in range(self.n_layers):
            cap = 0 if self.kv_strides[l] == 0 else min(self.kv_reserve_tokens, int(max_positions))
            snap_positions.append(cap)
            total += 2 * self.n_kv_heads * cap * self.layer_head_dim(l)
            snap_offsets.append(total)
        pin = None
        if pinned:
            import torch

            pin = torch.zeros(total, dtype=torch.int16, pin_memory=True)
            kv = pin.numpy().view(np.uint16)
        else:
            kv = np.zeros(total, np.uint16)
        return Instantaneous(list(self.kv_offsets), snap_offsets, snap_positions, kv,
                             np.zeros_like(self.dn_conv), np.zeros_like(self.dn_recurrent),
                             np.zeros_like(self.logits), 0, False, pin)

    def _compatible(self, s: Instantaneous) -> None:
        """compatible_snapshot, model.rs:705-725, plus the block bounds a
        snapshot read from a file must meet (the reference's slices would
        panic on them, model.rs:756-765, 830-833)."""
        if (s.kv_offsets != self.kv_offsets or s.dn_conv.size != self.dn_conv.size
                or s.dn_recurrent.size != self.dn_recurrent.size or s.logits.size != self.logits.size):
            raise SnapshotError("Backend", "the snapshot has been reserved for a different Runner geometry "
                                           "(KV cache, pass, or model differ) -- reclaim it after any reconstruction")
        if len(s.snap_positions) != self.n_layers or len(s.snap_offsets) != self.n_layers + 1:
            raise SnapshotError("Backend", "snapshot geometry does not cover the layers of this cache")
        for l in range(self.n_layers):
            need = 2 * self.n_kv_heads * s.snap_positions[l] * self.layer_head_dim(l)
            if s.snap_offsets[l] + need > s.kv.size:
                raise SnapshotError("Backend", f"snapshot layer {l} lies outside its KV block")

    @staticmethod
    def _host_ptr(a: np.ndarray) -> int:
        if not a.flags["C_CONTIGUOUS"] or a.dtype != np.uint16:
            raise ValueError("snapshot KV must be a contiguous uint16 array")
        return a.ctypes.data_as(ctypes.c_void_p).value or 0

    def _stream(self, stream):
        import torch

        if not self.kv.is_cuda:
            raise ValueError("the live cache must be a device tensor")
        return torch.cuda.current_stream(self.kv.device) if stream is None else stream

    def snapshot_take(self, s: Instantaneous, stream=None) -> None:
        """Copy the current state into `s` (model.rs:728-773): the first `pos`
        positions of every layer with a cache, then the other state. The slot
        is marked empty before the first copy, so a refusal half-way leaves it
        empty, never half old and half new."""
        self._compatible(s)
        base = self._host_ptr(s.kv)
        s._is_filled = False
        st = None
        for l in range(self.n_layers):
            if self.kv_strides[l] == 0:
                continue
            if self.pos > s.snap_positions[l]:
                raise SnapshotError("Backend", f"snapshot rejected -- layer {l} holds {self.pos} positions, the "
                                               f"slot buffer holds {s.snap_positions[l]} (increase positions_max)")
            st = st or self._stream(stream)
            kv_take_raw(self.layer_spec(l), self.keys(l).data_ptr(), self.values(l).data_ptr(),
                        base + 2 * s.snap_offsets[l], s.snap_positions[l], self.pos, st.cuda_stream)
        if st is not None:
            st.synchronize()
        s.dn_conv[...] = self.dn_conv
        s.dn_recurrent[...] = self.dn_recurrent
        s.logits[...] = self.logits
        s._pos = self.pos
        s._is_filled = True

    def restore_from(self, s: Instantaneous, p: int, stream=None) -> None:
        """Replace the current state by `s` truncated to `p` positions
        (model.rs:786-857). Refused: a snapshot of another geometry, an empty
        one, p beyond it, and p short of it once a recurrent state is part of
        it. Only the first p positions of each layer are copied."""
        self._compatible(s)
        if not s.is_filled():
            raise SnapshotError("Backend", "restoration refused -- snapshot is empty")
        if p > s.pos():
            raise SnapshotError("Backend", f"restoration refused -- p={p} beyond snapshot ({s.pos()} positions)")
        if p < s.pos() and self.dn_recurrent.size:
            raise SnapshotError("Backend", f"restoration refused -- the recurrent state (DeltaNet) is at position "
                                           f"{s.pos()}, it does not revert to p={p}; only an EXACT prefix is "
                                           f"restorable on this model")
        st = self._stream(stream)
        base = self._host_ptr(s.kv)
        for l in range(self.n_layers):
            if self.kv_strides[l] == 0:
                continue
            kv_restore_raw(self.layer_spec(l), base + 2 * s.snap_offsets[l], s.snap_positions[l],
                           self.keys(l).data_ptr(), self.values(l).data_ptr(), p, st.cuda_stream)
        st.synchronize()
        self.dn_conv[...] = s.dn_conv
        self.dn_recurrent[...] = s.dn_recurrent
        self.logits[...] = s.logits
        self.pos = int(p)


# ---- the conversation file (session.rs:320-391) -----------------------------

_USIZE = re.compile(r"\+?[0-9]+\Z")


def _parse_usize(s: str | None) -> int | None:
    """str::parse::<usize>: an optional '+', decimal digits, at most 2^64 - 1."""
    if s is None or not _USIZE.match(s):
        return None
    v = int(s)
    return v if v < (1 << 64) else None


def write_chat(w, model_type: str, vocab_size: int, ledger, assistant_open: bool, tools_announced: bool,
               slot: Instantaneous) -> None:
    """Chat::save (session.rs:320-341): a magic line, five header lines, the
    ledger as u32 little-endian tokens, then the snapshot."""
    if not slot.is_filled():
        raise SnapshotError("InvalidInput", "empty snapshot: nothing to write")
    w.write((CHAT_MAGIC + "\n").encode())
    w.write(f"{model_type}\n{vocab_size}\n{len(ledger)}\n{int(bool(assistant_open))}\n"
            f"{int(bool(tools_announced))}\n".encode())
    w.write(np.asarray(ledger, dtype="<u4").tobytes())
    slot.write_to(w)


class ChatFile:
    def __init__(self, model_type, vocab_size, ledger, assistant_open, tools_announced, slot):
        self.model_type = model_type
        self.vocab_size = vocab_size
        self.ledger = ledger
        self.assistant_open = assistant_open
        self.tools_announced = tools_announced
        self.slot = slot


def read_chat(r, model_type: str | None = None, vocab_size: int | None = None, name: str = "<stream>",
              cache: KvCache | None = None) -> ChatFile:
    """Chat::restore (session.rs:346-391): the six header lines read byte by
    byte, the saving model checked against (model_type, vocab_size) when
    given, the ledger, the snapshot, and a state whose position must equal
    the ledger's length. With `cache`, the snapshot is restored into it at its
    own position first, as the reference restores its engine."""
    raw = bytearray()
    newlines = 0
    while newlines < 6:
        b = _read_exact(r, 1)
        raw += b
        if b == b"\n":
            newlines += 1
    text = raw.decode("latin-1")
    fields = iter([x[:-1] if x.endswith("\r") else x for x in text.split("\n")[:-1]])

    def bad():
        return SnapshotError("Backend", f"{name}: not a saved conversation")

    if next(fields, None) != CHAT_MAGIC:
        raise bad()
    mt = next(fields, None)
    vocab = _parse_usize(next(fields, None))
    if mt is None or vocab is None:
        raise bad()
    if (model_type is not None and mt != model_type) or (vocab_size is not None and vocab != vocab_size):
        raise SnapshotError("Backend", f"{name}: saved from another model ({mt}, vocab {vocab})")
    count = _parse_usize(next(fields, None))
    if count is None:
        raise bad()
    assistant_open = next(fields, None) == "1"
    tools_announced = next(fields, None) == "1"
    ledger = _read_array(r, count, "<u4")
    slot = Instantaneous.read(r)
    if cache is not None:
        cache.restore_from(slot, slot.pos())
        held = cache.pos
    else:
        held = slot.pos()
    if held != count:
        raise SnapshotError("Backend", f"{name}: the state holds {held} positions but the ledger {count} tokens")
    return ChatFile(mt, vocab, ledger, assistant_open, tools_announced, slot)
