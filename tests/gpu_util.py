"""Run one workload through libhsdpa.so on the current GPU (test helper)."""
from __future__ import annotations

import numpy as np


def run_hsdpa(w, plan=None, stream=None) -> np.ndarray:
    import torch
    import hsdpa

    dev = torch.device("cuda")
    if plan is None:
        plan = hsdpa.Plan(w.heads, w.gqa, w.head_dim, w.capacity)
    q = torch.from_numpy(np.ascontiguousarray(w.q).view(np.int16)).to(dev)
    k = torch.from_numpy(np.ascontiguousarray(w.k).view(np.int16)).to(dev)
    v = torch.from_numpy(np.ascontiguousarray(w.v).view(np.int16)).to(dev)
    out = torch.full((w.rows, w.heads, w.head_dim), -1, dtype=torch.int16, device=dev)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=dev)
    hsdpa.attention_torch(plan, q, k, v, out, w.rows, w.past, w.scale, ws, stream)
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint16)
