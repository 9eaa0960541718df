#!/usr/bin/env python3
"""Benchmark of the attention step on one MI355X.

Headline: decode SDPA at 32K context in GB/s (fraction of the 8 TB/s HBM
peak): 1 query row, 16 query heads on 2 KV heads, head_dim 256, 32768 cached
keys, bf16 with f32 accumulation. Alongside it, in the same JSON line: the
causal prefill of a 4096-row chunk after 8192 cached keys (16/2 heads,
head_dim 256) in TFLOP/s against the dense bf16 MFMA peak, and the CPU
baseline (the AVX-512 BF16 restatement of the reference's emitted SDPA) on
this host's cores.

A step is one attention call over one synthetic batch. Inputs are resident
in HBM before timing. Decode rotates 16 distinct 64 MiB caches (1 GiB) so that
the 256 MB Infinity Cache cannot hold the working set. The K timed steps
are captured once into a HIP graph and replayed, so the figure is GPU time,
not Python launch time; the replay's output is checked against an eager call.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-prefill]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "herbert-jit-bf16_amd"))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
MFMA_BF16_PEAK_TFS = 2500.0  # MI355X dense bf16 MFMA, TFLOP/s

# Memory traffic per call, from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs
# of this script (KiB per dispatch, summed over the kernels of one call).
# FETCH_SIZE is scaled by 2 and WRITE_SIZE by 1: a 256 MiB device copy reads
# 131 086 KiB and writes 262 144 KiB on these counters. FETCH_SIZE counts
# every L2 fill from the memory fabric, so Infinity Cache hits are included.
# Summary and commands: profiles/pmc_traffic_decode32k_prefill4096.md
TRAFFIC_BYTES = {
    "decode_32k": (2 * (16452.3 + 17547.9 + 1087.9) + (2176.4 + 2056.0 + 8.0)) * 1024,
    "prefill_4096_after_8192": (2 * 1267085.2 + 35840.0) * 1024,
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def device_buffers(torch, w, copies=1):
    import numpy as np

    dev = torch.device("cuda")
    q = torch.from_numpy(np.ascontiguousarray(w.q).view(np.int16)).to(dev)
    k0 = torch.from_numpy(np.ascontiguousarray(w.k).view(np.int16)).to(dev)
    v0 = torch.from_numpy(np.ascontiguousarray(w.v).view(np.int16)).to(dev)
    ks = [k0] + [k0.clone() for _ in range(copies - 1)]
    vs = [v0] + [v0.clone() for _ in range(copies - 1)]
    out = torch.zeros((w.rows, w.heads, w.head_dim), dtype=torch.int16, device=dev)
    return q, ks, vs, out


def time_steps(torch, plan, w, q, ks, vs, out, ws, steps, warmup):
    """Warm up eagerly, capture `steps` calls into a graph, replay it once
    after a synchronize, return (ms per step, eager output, graph output)."""
    stream = torch.cuda.Stream()
    nb = ws.numel()

    def call(i):
        plan.attention_raw(q.data_ptr(), ks[i % len(ks)].data_ptr(), vs[i % len(vs)].data_ptr(), out.data_ptr(),
                           w.rows, w.past, w.scale, ws.data_ptr(), nb, stream.cuda_stream)

    with torch.cuda.stream(stream):
        for i in range(warmup):
            call(i)
    torch.cuda.synchronize()
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(steps):
            call(i)
    torch.cuda.synchronize()
    out.zero_()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):  # replay() runs on the current stream: time it there
        start.record(stream)
        graph.replay()
        end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end) / steps
    return ms, wall, eager, out.clone()


def host_description():
    """CPU model, sockets and logical CPUs of this host (from /proc/cpuinfo)."""
    model, sockets = "?", set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, val = line.partition(":")
                key = key.strip()
                if key == "model name" and model == "?":
                    model = val.strip()
                elif key == "physical id":
                    sockets.add(val.strip())
    except OSError:
        pass
    return f"{model}, {max(len(sockets), 1)} socket(s), {os.cpu_count()} logical CPUs"


def median_time(fn, warm, runs):
    ts = []
    for i in range(warm + runs):
        t0 = time.perf_counter()
        fn()
        if i >= warm:
            ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2]


def cpu_baseline(w_decode, decode_gbs_gpu):
    """Time the AVX-512 BF16 restatement of the reference on this host: the
    reference's decode node has Hq tasks, so it uses min(cores, Hq) threads;
    a 1-thread figure is reported beside it."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    if not oracle.avx512_available():
        return None, "host lacks AVX-512 BF16"
    cores = oracle.lib().oracle_physical_cores()
    used = min(cores, w_decode.heads)
    med = median_time(lambda: oracle.attention(w_decode, "avx512", threads=used), 3, 20)
    med1 = median_time(lambda: oracle.attention(w_decode, "avx512", threads=1), 1, 5)
    nbytes = w_decode.decode_bytes()
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": used,
            "kind": "port",
            "sample": f"decode 32K (same inputs), 20 runs after 3 warm-ups, median {med*1e3:.2f} ms, "
                      f"{used} of {cores} physical cores, pinned",
            "host": host_description(),
            "one_thread": {"value": round(nbytes / med1 / 1e9, 3), "unit": "GB/s",
                           "sample": f"5 runs after 1 warm-up, median {med1*1e3:.2f} ms"}}, None


def cpu_prefill_sample(wp, threads):
    """Bounded sample of the prefill on the CPU: the chunk's last 256-row pass."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    from hsdpa import workloads as W

    rows = 256
    past = wp.past + wp.rows - rows
    ws = W.Workload("prefill_sample", wp.heads, wp.kv_heads, wp.head_dim, rows, past, wp.capacity,
                    wp.q[-rows:], wp.k, wp.v, wp.scale)
    med = median_time(lambda: oracle.attention(ws, "avx512", threads=threads), 1, 3)
    return {"value": round(ws.prefill_flops() / med / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"last 256-row pass of the 4096-row chunk (past {past}), 3 runs after 1 warm-up, "
                      f"median {med*1e3:.1f} ms"}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--prefill-steps", type=int, default=0, help="timed prefill steps (default: --steps, max 20)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the attention step here is built and timed on a single MI355X; "
              f"--gpus {args.gpus} is not supported (multi-GPU sharding is a design note only).", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import hsdpa
    from hsdpa import workloads as W

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    hsdpa.library()  # fails loudly if libhsdpa.so is missing
    props = torch.cuda.get_device_properties(0)
    log(f"device {props.name} gcn {getattr(props, 'gcnArchName', '?')} CUs {props.multi_processor_count}")

    # ---- decode, 32K context ------------------------------------------------
    wd = W.config("decode_32k", seed=0)
    q, ks, vs, out = device_buffers(torch, wd, copies=16)
    plan = hsdpa.Plan(wd.heads, wd.gqa, wd.head_dim, wd.capacity)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    ms, wall, eager, replay = time_steps(torch, plan, wd, q, ks, vs, out, ws, args.steps, args.warmup)
    if not torch.equal(eager, replay):
        print("graph replay differs from the eager call", file=sys.stderr)
        sys.exit(3)
    dec_bytes = wd.decode_bytes()
    gbs = dec_bytes / (ms * 1e-3) / 1e9
    log(f"decode_32k: {ms*1e3:.2f} us/step, {gbs:.1f} GB/s ({gbs/HBM_PEAK_GBS:.1%} of HBM peak), wall {wall*1e3:.2f} ms")
    del ks, vs
    torch.cuda.empty_cache()

    result = {
        "metric": "decode SDPA GB/s (% HBM peak) @32K ctx; prefill TFLOP/s (% MFMA peak)",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "decode_32k: 1 query row, 16 query heads on 2 KV heads (GQA 8:1), head_dim 256, "
                               "32768 cached keys, bf16 q/K/V/out, f32 accumulation, scale 1/16",
                   "algorithmic_bytes": dec_bytes, "kv_caches_rotated": 16, "timing": "HIP graph of the timed steps"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": round(TRAFFIC_BYTES["decode_32k"]),
                     "kernel": "decode step (decode_qk + decode_pv + decode_combine)"},
    }

    # ---- prefill, 4096 rows after 8192 ------------------------------------------
    if not args.no_prefill:
        wp = W.config("prefill_4096_after_8192", seed=0)
        q, ks, vs, out = device_buffers(torch, wp, copies=1)
        plan_p = hsdpa.Plan(wp.heads, wp.gqa, wp.head_dim, wp.capacity)
        ws_p = torch.empty(plan_p.workspace_bytes, dtype=torch.uint8, device="cuda")
        psteps = args.prefill_steps or min(args.steps, 20)
        pms, pwall, eager, replay = time_steps(torch, plan_p, wp, q, ks, vs, out, ws_p, psteps, min(args.warmup, 3))
        if not torch.equal(eager, replay):
            print("prefill graph replay differs from the eager call", file=sys.stderr)
            sys.exit(3)
        flops = wp.prefill_flops()
        tfs = flops / (pms * 1e-3) / 1e12
        log(f"prefill_4096_after_8192: {pms:.3f} ms/step, {tfs:.1f} TFLOP/s ({tfs/MFMA_BF16_PEAK_TFS:.1%} of MFMA peak)")
        result["prefill"] = {
            "value": round(tfs, 2), "unit": "TFLOP/s", "ms_per_step": round(pms, 4), "steps": psteps,
            "config": {"workload": "prefill_4096_after_8192: causal chunk of 4096 rows after 8192 cached keys, "
                                   "16 query heads on 2 KV heads, head_dim 256, scale 1/16",
                       "algorithmic_flops": flops},
            "roofline": {"bound": "mfma", "achieved": round(tfs, 2), "peak": MFMA_BF16_PEAK_TFS, "unit": "TFLOP/s",
                         "frac": round(tfs / MFMA_BF16_PEAK_TFS, 4),
                         "traffic": round(TRAFFIC_BYTES["prefill_4096_after_8192"]),
                         "kernel": "prefill_attn"},
        }
        del ks, vs, q, out
        torch.cuda.empty_cache()
        wp_cpu = wp
    else:
        wp_cpu = None

    # ---- CPU baseline ------------------------------------------------------------
    if not args.no_cpu:
        cb, why = cpu_baseline(wd, gbs)
        if cb is None:
            result["cpu_baseline"] = {"value": None, "unit": "GB/s", "cores": 0, "kind": "port", "sample": why}
        else:
            result["cpu_baseline"] = cb
            if wp_cpu is not None:
                import oracle

                result["prefill"]["cpu_baseline"] = cpu_prefill_sample(wp_cpu, oracle.lib().oracle_physical_cores())
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
