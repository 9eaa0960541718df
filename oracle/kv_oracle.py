"""CPU restatement of the reference's KV append — TEST INFRASTRUCTURE ONLY.

Only tests/ use it, as the checker of hsdpa_kv_append; the product path never
does. It restates src/jit/target/x86/execution/kv.rs:15-69: one task per KV
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
