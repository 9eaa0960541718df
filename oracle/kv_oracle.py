"""CPU restatement of the reference's KV append and snapshot copies — TEST
INFRASTRUCTURE ONLY.

Only tests/ use it: the oracle that hsdpa_kv_append, hsdpa_kv_take and
hsdpa_kv_restore are compared with; the product path never does. The snapshot copies
(snapshot_take / restore_from, below) restate model.rs:732-857 and are pinned
by the tests against a hand-placed known-answer cache and by take-then-restore
identity. It restates src/jit/target/x86/execution/kv.rs:15-69: one task per KV
head (tasks at or past `heads` return at once, kv.rs:29-30), nothing for an
empty block (kv.rs:31-34), and for each row r of the block a byte copy of
head_dim bf16 from the token-major source (row r, head h at
(r*heads + h)*head_dim, kv.rs:40-43) to the head-major cache (position past + r
of head h at h*stride + (past + r)*head_dim, kv.rs:44-48), keys then values
(kv.rs:49-59). `kv_append_tasks` follows that loop nest literally and is
pinned by the tests against a known-answer block; `kv_append` is the
vectorised form used on large blocks, checked equal to the loop form.
"""
from __future__ import annotations

import numpy as np


def kv_append_tasks(keys: np.ndarray, values: np.ndarray, input_keys: np.ndarray, input_values: np.ndarray,
                    heads: int, head_dim: int, stride: int, rows: int, past: int, tasks: int | None = None) -> None:
    """In place on flat uint16 arrays, task by task and row by row."""
    for task in range(heads if tasks is None else tasks):
        if task >= heads or rows == 0:
            continue
        for r in range(rows):
            src = (r * heads + task) * head_dim
            dst = task * stride + (past + r) * head_dim
            keys[dst:dst + head_dim] = input_keys[src:src + head_dim]
            values[dst:dst + head_dim] = input_values[src:src + head_dim]


def kv_append(keys: np.ndarray, values: np.ndarray, input_keys: np.ndarray, input_values: np.ndarray,
              heads: int, head_dim: int, stride: int, rows: int, past: int) -> None:
    """The same copy, one slice per head."""
    if rows == 0:
        return
    ik = input_keys[:rows * heads * head_dim].reshape(rows, heads, head_dim)
    iv = input_values[:rows * heads * head_dim].reshape(rows, heads, head_dim)
    for h in range(heads):
        dst = h * stride + past * head_dim
        keys[dst:dst + rows * head_dim] = ik[:, h, :].reshape(-1)
        values[dst:dst + rows * head_dim] = iv[:, h, :].reshape(-1)


# ---- snapshot copies -------------------------------------------------------
# Restatement of the KV loops of Runner::snapshot_take (src/jit/model.rs:732-773)
# and Runner::restore_from (model.rs:786-857) over flat uint16 arrays: the live
# cache `kv` holds layer l at kv_offsets[l], keys then values, head h of a half
# at h * kv_strides[l]; the snapshot `snap` holds layer l at snap_offsets[l],
# head h of a half at h * snap_positions[l] * head_dim_l. head_dim_l is
# kv_strides[l] // kv_reserve_tokens (model.rs:700-703).

def first_different_row(live: np.ndarray, snap: np.ndarray, hd: int) -> int:
    """model.rs:861-865: the first row of hd elements where the two differ, or
    their length in rows."""
    rows = live.size // hd
    for r in range(rows):
        if not np.array_equal(live[r * hd:(r + 1) * hd], snap[r * hd:(r + 1) * hd]):
            return r
    return rows


def snapshot_take(kv: np.ndarray, kv_offsets, kv_strides, kv_reserve_tokens: int, n_kv_heads: int,
                  snap: np.ndarray, snap_offsets, snap_positions, pos: int) -> None:
    """model.rs:741-767. Raises ValueError where the reference refuses a layer
    that holds more positions than the slot."""
    for l, st in enumerate(kv_strides):
        if st == 0:
            continue
        hd = st // kv_reserve_tokens
        used = pos
        if used > snap_positions[l]:
            raise ValueError(f"layer {l} holds {used} positions, the slot {snap_positions[l]}")
        snap_st = snap_positions[l] * hd
        src_at, dst_at = kv_offsets[l], snap_offsets[l]
        for half in range(2):
            src0 = src_at + half * n_kv_heads * st
            dst0 = dst_at + half * n_kv_heads * snap_st
            for h in range(n_kv_heads):
                n = used * hd
                snap[dst0 + h * snap_st:dst0 + h * snap_st + n] = kv[src0 + h * st:src0 + h * st + n]


def restore_from(kv: np.ndarray, kv_offsets, kv_strides, kv_reserve_tokens: int, n_kv_heads: int,
                 snap: np.ndarray, snap_offsets, snap_positions, p: int) -> None:
    """model.rs:820-852 without the R16 copies (an AArch64 layout): from the
    first differing row of each head, the snapshot's rows replace the live ones."""
    for l, st in enumerate(kv_strides):
        if st == 0:
            continue
        hd = st // kv_reserve_tokens
        used = p
        snap_st = snap_positions[l] * hd
        dst_at, src_at = kv_offsets[l], snap_offsets[l]
        for half in range(2):
            dst0 = dst_at + half * n_kv_heads * st
            src0 = src_at + half * n_kv_heads * snap_st
            for h in range(n_kv_heads):
                n = used * hd
                s = snap[src0 + h * snap_st:src0 + h * snap_st + n]
                live = kv[dst0 + h * st:dst0 + h * st + n]
                start = first_different_row(live, s, hd)
                if start == used:
                    continue
                live[start * hd:] = s[start * hd:]
