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

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-prefill] [--no-layer] [--no-sweep]
                    [--only CONFIG ...]

Every configuration of the benchmark is timed and reported under "configs"
with its own value, time and roofline fraction: decode at 1K keys (8/2
heads), decode at 32K (the headline), the 512-row causal chunk into an empty
cache (16/4 heads), the 4096-row chunk after 8192 keys, and decode at 128K
keys with outlier keys and values. The three decode configurations are also
timed under the reference's Fused form ("configs_fused").

Also timed: the whole attention chain of a gated Qwen3.5 layer (q/k norm and
RoPE, KV append, attention, output gate) fused into one call against the same
nodes called one by one; the decode at 1K, 8K, 32K and 128K keys; and 2, 4, 8
and 16 rows after the 32K cache (`--no-sweep` skips these two).
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
# 131 087 KiB and writes 262 144 KiB on these counters. FETCH_SIZE counts
# every L2 fill from the memory fabric, so Infinity Cache hits are included.
# Summary and commands: profiles/pmc_traffic_bench_configs.md
TRAFFIC_BYTES = {
    "chained": {
        "decode_1k": (2 * (559.9 + 2242.9) + (34.0 + 4.0)) * 1024,
        "decode_32k": (2 * (16465.3 + 17501.5 + 1091.5) + (2112.0 + 2056.0 + 8.0)) * 1024,
        "prefill_512": (2 * 8603.5 + 4096.0) * 1024,
        "prefill_4096_after_8192": (2 * (78085.9 + 141420.1 + 31024.3) + (512.0 + 81790.3 + 15360.0)) * 1024,
        "decode_128k_outliers": (2 * (65624.7 + 69768.4 + 1091.5) + (8320.1 + 2056.0 + 8.0)) * 1024,
    },
    "fused": {
        "decode_1k": (2 * (568.3 + 2269.5) + (36.0 + 4.0)) * 1024,
        "decode_32k": (2 * (16464.5 + 17528.4 + 1143.5) + (2112.0 + 2064.0 + 8.0)) * 1024,
        "decode_128k_outliers": (2 * (65622.1 + 69804.4 + 1143.5) + (8320.1 + 2064.0 + 8.0)) * 1024,
    },
}

PREFILL_KERNELS = {"prefill_512": "prefill_kd (one workgroup per 32-row block; its keys split among 8 waves)",
                   "prefill_4096_after_8192": "prefill_split_max + prefill_split_pv + prefill_split_combine "
                                              "(row groups paired: the longest with the shortest)"}


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
    # the buffers were filled on the current stream (copies, clones, zeros)
    stream.wait_stream(torch.cuda.current_stream())
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


def layer_buffers(torch, w, copies, seed=7):
    """Device buffers of a gated layer chain on workload w's cache: q rows of
    [Q ; gate] (2*q_dim), the block's k and v projections, norm weights, RoPE
    tables over the capacity (rotary 64 of head_dim, the Qwen3.5 layout)."""
    import numpy as np
    from hsdpa import workloads as W

    rng = np.random.default_rng(seed)
    dev = torch.device("cuda")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)
    bf = lambda a: W.f32_to_bf16(np.asarray(a, np.float32))
    q_dim, kv_row, rot = w.heads * w.head_dim, w.kv_heads * w.head_dim, 64
    ang = np.arange(w.capacity, dtype=np.float64)[:, None] * (1e7 ** (-np.arange(rot // 2) * 2.0 / rot))[None, :]
    b = dict(q=t(bf(rng.normal(0, 2, w.rows * 2 * q_dim))), k=t(bf(rng.normal(0, 2, w.rows * kv_row))),
             v=t(bf(rng.normal(0, 1, w.rows * kv_row))), q_norm=t(bf(rng.normal(0, 0.1, w.head_dim))),
             k_norm=t(bf(rng.normal(0, 0.1, w.head_dim))), cos=t(bf(np.cos(ang))), sin=t(bf(np.sin(ang))),
             out=torch.zeros(w.rows * q_dim, dtype=torch.int16, device=dev))
    k0 = t(w.k)
    v0 = t(w.v)
    b["keys"] = [k0] + [k0.clone() for _ in range(copies - 1)]
    b["values"] = [v0] + [v0.clone() for _ in range(copies - 1)]
    return b, q_dim, kv_row, rot


def layer_step(hsdpa, plan, w, b, i, ws, fused, stream):
    """One layer step: the fused call, or the five nodes in order."""
    q_dim, kv_row, rot = w.heads * w.head_dim, w.kv_heads * w.head_dim, 64
    keys, values = b["keys"][i % len(b["keys"])], b["values"][i % len(b["values"])]
    gate = b["q"][q_dim:]
    if fused:
        hsdpa.attention_layer_torch(plan, b["q"], b["k"], b["v"], keys, values, b["out"], b["q_norm"], b["k_norm"],
                                    b["cos"], b["sin"], w.rows, w.past, w.scale, 1e-6, ws, kv_row, rot, gate=gate,
                                    gate_row=2 * q_dim, positions=w.capacity, stream=stream)
        return
    hsdpa.head_norm_rope_torch(b["q"], b["q_norm"], b["cos"], b["sin"], w.heads, w.head_dim, w.head_dim, 2 * q_dim,
                               rot, w.rows, w.past, 1e-6, positions=w.capacity, stream=stream)
    hsdpa.head_norm_rope_torch(b["k"], b["k_norm"], b["cos"], b["sin"], w.kv_heads, w.head_dim, w.head_dim, kv_row,
                               rot, w.rows, w.past, 1e-6, positions=w.capacity, stream=stream)
    spec = hsdpa.kv_spec(w.kv_heads, w.head_dim, w.capacity, w.rows)
    hsdpa.kv_append_torch(spec, keys, values, b["k"], b["v"], w.rows, w.past, stream=stream)
    hsdpa.attention_torch(plan, b["q"], keys, values, b["out"], w.rows, w.past, w.scale, ws, stream)
    hsdpa.output_gate_torch(b["out"], gate, q_dim, q_dim, 2 * q_dim, w.rows, stream=stream)


def time_layer(torch, hsdpa, w, copies, steps, warmup):
    """The gated layer chain (norms, append, attention, gate) on workload w:
    ms per step fused (hsdpa_attention_layer) and as separate nodes, each a
    HIP graph of `steps` steps. First checks one eager step of each on fresh
    buffers for equal outputs, cache and q/k."""
    plan = hsdpa.Plan(w.heads, w.gqa, w.head_dim, w.capacity, q_row=2 * w.heads * w.head_dim)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.Stream()
    results = {}
    check = []
    for fused in (True, False):
        b = layer_buffers(torch, w, copies)[0]
        stream.wait_stream(torch.cuda.current_stream())   # filled there: copies, clones, zeros
        with torch.cuda.stream(stream):
            layer_step(hsdpa, plan, w, b, 0, ws, fused, stream)
        torch.cuda.synchronize()
        check.append([b[n].clone() for n in ("q", "k", "out")] + [b["keys"][0].clone(), b["values"][0].clone()])
        # the clones run on the current stream; the warm-up steps rewrite q, k
        # and the cache in place on `stream`
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            for i in range(warmup):
                layer_step(hsdpa, plan, w, b, i, ws, fused, stream)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(steps):
                layer_step(hsdpa, plan, w, b, i, ws, fused, stream)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            start.record(stream)
            graph.replay()
            end.record(stream)
        torch.cuda.synchronize()
        results["fused" if fused else "nodes"] = start.elapsed_time(end) / steps
        del b, graph
        torch.cuda.empty_cache()
    same = all(torch.equal(x, y) for x, y in zip(check[0], check[1]))
    return results["fused"], results["nodes"], same


CONFIG_ORDER = ["decode_1k", "decode_32k", "prefill_512", "prefill_4096_after_8192", "decode_128k_outliers"]
CONFIG_TEXT = {
    "decode_1k": "1 query row, 8 query heads on 2 KV heads (GQA 4:1), head_dim 256, 1024 cached keys",
    "decode_32k": "1 query row, 16 query heads on 2 KV heads (GQA 8:1), head_dim 256, 32768 cached keys",
    "prefill_512": "causal chunk of 512 rows into an empty cache, 16 query heads on 4 KV heads, head_dim 256",
    "prefill_4096_after_8192": "causal chunk of 4096 rows after 8192 cached keys, 16 query heads on 2 KV heads, "
                               "head_dim 256",
    "decode_128k_outliers": "1 query row, 16 query heads on 2 KV heads, head_dim 256, 131072 cached keys; 4 key "
                            "channels per KV head x20, 1% of value rows x8",
}
DECODE_KERNELS = "decode step (decode_qk + decode_pv + decode_combine)"
# up to 1024 keys (one row, one group): pass 2 writes the outputs itself
DECODE_DIRECT = "decode step (decode_qk + decode_direct, no combine launch)"


def bench_config(torch, hsdpa, W, name, kind, steps, warmup, form="chained"):
    """Time one configuration as a HIP graph of `steps` calls. Decode rotates
    distinct caches totalling at least 1 GiB (the Infinity Cache is 256 MB);
    a prefill reads a 24 MiB or smaller cache and runs long enough per call
    that one copy is representative. Returns the configuration's record."""
    w = W.config(name, seed=0)
    per_cache = 2 * w.kv_heads * w.capacity * w.head_dim * 2
    copies = max(4, -(-(1 << 30) // per_cache)) if kind == "decode" else 1
    q, ks, vs, out = device_buffers(torch, w, copies=copies)
    plan = hsdpa.Plan(w.heads, w.gqa, w.head_dim, w.capacity, **({"form": form} if form != "chained" else {}))
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    ms, wall, eager, replay = time_steps(torch, plan, w, q, ks, vs, out, ws, steps, warmup)
    if not torch.equal(eager, replay):
        print(f"{name}: graph replay differs from the eager call", file=sys.stderr)
        sys.exit(3)
    launches = plan.route(w.rows, w.past)["launches"]
    del q, ks, vs, out, ws
    torch.cuda.empty_cache()
    text = f"{name}: {CONFIG_TEXT[name]}, bf16 q/K/V/out, f32 accumulation, scale 1/16"
    if form != "chained":
        text += f", decode form {form}"
    if kind == "decode":
        nbytes = w.decode_bytes()
        val = nbytes / (ms * 1e-3) / 1e9
        log(f"{name} ({form}): {ms*1e3:.2f} us/step, {val:.1f} GB/s ({val/HBM_PEAK_GBS:.1%} of HBM peak), "
            f"wall {wall*1e3:.2f} ms")
        tr = TRAFFIC_BYTES.get(form, {}).get(name)
        return {"value": round(val, 2), "unit": "GB/s", "ms_per_step": round(ms, 5), "steps": steps,
                "config": {"workload": text, "algorithmic_bytes": nbytes, "kv_caches_rotated": copies},
                "roofline": {"bound": "hbm", "achieved": round(val, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(val / HBM_PEAK_GBS, 4), "traffic": round(tr) if tr else None,
                             "kernel": DECODE_DIRECT if launches == 2 else DECODE_KERNELS}}
    flops = w.prefill_flops()
    val = flops / (ms * 1e-3) / 1e12
    log(f"{name}: {ms*1e3:.2f} us/step, {val:.1f} TFLOP/s ({val/MFMA_BF16_PEAK_TFS:.1%} of MFMA peak)")
    tr = TRAFFIC_BYTES["chained"].get(name)
    return {"value": round(val, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 5), "steps": steps,
            "config": {"workload": text, "algorithmic_flops": flops},
            "roofline": {"bound": "mfma", "achieved": round(val, 2), "peak": MFMA_BF16_PEAK_TFS, "unit": "TFLOP/s",
                         "frac": round(val / MFMA_BF16_PEAK_TFS, 4), "traffic": round(tr) if tr else None,
                         "kernel": PREFILL_KERNELS[name]}}


def bench_prefill_passes(torch, hsdpa, W, name, steps, warmup, rows_per_pass=256):
    """The chunk as the reference engine sends it to the attention node:
    passes of at most 256 rows (prefill_pass, src/jit/schedule.rs:290-298,
    bounded by max_batch, src/jit/model/mounted.rs:185-187), each a call
    after the rows before it (4096 rows after 8192 keys: 16 calls after 8192,
    8448, ..., 12032 keys), one plan with max_rows = 256. `steps` chunks are
    captured into one HIP graph. Returns the record (TFLOP/s over the chunk)."""
    w = W.config(name, seed=0)
    q, ks, vs, out = device_buffers(torch, w, copies=1)
    plan = hsdpa.Plan(w.heads, w.gqa, w.head_dim, w.capacity, max_rows=rows_per_pass)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    passes = [(r0, min(rows_per_pass, w.rows - r0)) for r0 in range(0, w.rows, rows_per_pass)]
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    qrow_b, orow_b = 2 * w.q_row, 2 * w.out_row

    def chunk():
        for r0, rows in passes:
            plan.attention_raw(q.data_ptr() + r0 * qrow_b, ks[0].data_ptr(), vs[0].data_ptr(),
                               out.data_ptr() + r0 * orow_b, rows, w.past + r0, w.scale, ws.data_ptr(), ws.numel(),
                               stream.cuda_stream)

    with torch.cuda.stream(stream):
        for _ in range(warmup):
            chunk()
    torch.cuda.synchronize()
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for _ in range(steps):
            chunk()
    torch.cuda.synchronize()
    out.zero_()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start.record(stream)
        graph.replay()
        end.record(stream)
    torch.cuda.synchronize()
    if not torch.equal(eager, out):
        print(f"{name} in passes: graph replay differs from the eager calls", file=sys.stderr)
        sys.exit(3)
    ms = start.elapsed_time(end) / steps
    kernels = sorted({plan.route(rows, w.past + r0)["main"] for r0, rows in passes})
    launches = sum(plan.route(rows, w.past + r0)["launches"] for r0, rows in passes)
    flops = w.prefill_flops()
    val = flops / (ms * 1e-3) / 1e12
    log(f"{name} in {len(passes)} passes of {rows_per_pass} rows: {ms*1e3:.2f} us/chunk, {val:.1f} TFLOP/s "
        f"({val/MFMA_BF16_PEAK_TFS:.1%} of MFMA peak), kernels {kernels}, {launches} launches")
    del q, ks, vs, out, ws
    torch.cuda.empty_cache()
    return {"value": round(val, 2), "unit": "TFLOP/s", "ms_per_chunk": round(ms, 5), "steps": steps,
            "passes": len(passes), "rows_per_pass": rows_per_pass, "kernels": kernels, "launches": launches,
            "frac": round(val / MFMA_BF16_PEAK_TFS, 4),
            "workload": f"the {w.rows}-row chunk as {len(passes)} sequential hsdpa_attention calls of "
                        f"{rows_per_pass} rows after {w.past}, {w.past + rows_per_pass}, ... keys (the reference "
                        f"engine's prefill passes), one HIP graph of {steps} chunks"}


def bench_frame(torch, hsdpa, W, name, steps, warmup):
    """Decode through hsdpa_attention_frame (rows and past read from device
    memory by the kernels): a HIP graph of `steps` frame calls over distinct
    caches (at least 1 GiB), as the other decode timings rotate theirs."""
    w = W.config(name, seed=0)
    per_cache = 2 * w.kv_heads * w.capacity * w.head_dim * 2
    copies = max(4, -(-(1 << 30) // per_cache))
    q, ks, vs, out = device_buffers(torch, w, copies=copies)
    plan = hsdpa.Plan(w.heads, w.gqa, w.head_dim, w.capacity, max_rows=1)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    vals = torch.tensor([1, w.past], dtype=torch.int64, device="cuda")
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())

    def call(i):
        plan.attention_frame_raw(q.data_ptr(), ks[i % copies].data_ptr(), vs[i % copies].data_ptr(), out.data_ptr(),
                                 vals.data_ptr(), vals.data_ptr() + 8, w.scale, ws.data_ptr(), ws.numel(),
                                 status.data_ptr(), stream.cuda_stream)

    with torch.cuda.stream(stream):
        for i in range(warmup):
            call(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(steps):
            call(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start.record(stream)
        graph.replay()
        end.record(stream)
    torch.cuda.synchronize()
    if int(status.item()) != 0:
        print(f"{name} frame: status {int(status.item())}", file=sys.stderr)
        sys.exit(3)
    ms = start.elapsed_time(end) / steps
    val = w.decode_bytes() / (ms * 1e-3) / 1e9
    log(f"{name} frame call: {ms*1e3:.2f} us/step, {val:.1f} GB/s")
    del q, ks, vs, out, ws
    torch.cuda.empty_cache()
    return {"us": round(ms * 1e3, 2), "GB/s": round(val, 1), "frac": round(val / HBM_PEAK_GBS, 4)}


def cpu_config_baseline(w, kind, threads, runs=5):
    """The AVX-512 BF16 restatement on this host for one configuration, the
    whole call (a decode uses min(threads, Hq) workers: the reference's decode
    node has Hq tasks). Median of `runs` after one warm-up."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    used = min(threads, w.heads) if kind == "decode" else threads
    med = median_time(lambda: oracle.attention(w, "avx512", threads=used), 1, runs)
    if kind == "decode":
        val, unit = w.decode_bytes() / med / 1e9, "GB/s"
    else:
        val, unit = w.prefill_flops() / med / 1e12, "TFLOP/s"
    return {"value": round(val, 4), "unit": unit, "cores": used, "kind": "port",
            "sample": f"the whole call, {runs} runs after 1 warm-up, median {med*1e3:.2f} ms"}


def cpu_baseline(w_decode):
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
    ap.add_argument("--no-layer", action="store_true", help="skip the fused layer chain timing")
    ap.add_argument("--no-sweep", action="store_true", help="skip the decode length sweep and the few-rows timings")
    ap.add_argument("--prefill-steps", type=int, default=0, help="timed prefill steps (default: --steps, max 20)")
    ap.add_argument("--no-fused", action="store_true", help="skip the decode timings under the Fused form")
    ap.add_argument("--only", nargs="*", default=None, choices=CONFIG_ORDER,
                    help="time only these configurations (the headline line then lacks the others)")
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

    # ---- the five configurations -------------------------------------------------
    # decode_32k is the headline (`value`); prefill_4096_after_8192 is also
    # repeated as `prefill`. Each configuration carries its own time, value and
    # roofline fraction under "configs".
    psteps = args.prefill_steps or min(args.steps, 20)
    configs = {}
    for name in CONFIG_ORDER:
        if args.only and name not in args.only:
            continue
        kind = "prefill" if name.startswith("prefill") else "decode"
        if kind == "prefill" and args.no_prefill:
            continue
        configs[name] = bench_config(torch, hsdpa, W, name, kind, psteps if kind == "prefill" else args.steps,
                                     min(args.warmup, 3) if kind == "prefill" else args.warmup)
    head = configs.get("decode_32k")
    result = {
        "metric": "decode SDPA GB/s (% HBM peak) @32K ctx; prefill TFLOP/s (% MFMA peak)",
        "value": head["value"] if head else None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"] if head else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "decode_32k: 1 query row, 16 query heads on 2 KV heads (GQA 8:1), head_dim 256, "
                               "32768 cached keys, bf16 q/K/V/out, f32 accumulation, scale 1/16",
                   "algorithmic_bytes": head["config"]["algorithmic_bytes"] if head else None,
                   "kv_caches_rotated": head["config"]["kv_caches_rotated"] if head else None,
                   "timing": "HIP graph of the timed steps"},
        "roofline": head["roofline"] if head else None,
    }
    if "prefill_4096_after_8192" in configs:
        result["prefill"] = configs["prefill_4096_after_8192"]
        # the same chunk as the reference engine sends it: passes of 256 rows
        configs["prefill_4096_after_8192"]["engine_passes"] = bench_prefill_passes(
            torch, hsdpa, W, "prefill_4096_after_8192", psteps, min(args.warmup, 3))
    result["configs"] = configs
    # the headline decode through the frame entry (rows and past read on the device)
    if not args.only or "decode_32k" in args.only:
        result["frame"] = {"decode_32k": bench_frame(torch, hsdpa, W, "decode_32k", args.steps, args.warmup),
                           "entry": "hsdpa_attention_frame: the kernels read rows and past from device memory "
                                    "and derive their key partition from them; graph of the timed steps"}
    # the decode configurations under the reference's Fused form (plan form =
    # HSDPA_FORM_FUSED), beside the Chained default above
    if not args.no_fused:
        fused = {}
        for name in ("decode_1k", "decode_32k", "decode_128k_outliers"):
            if args.only and name not in args.only:
                continue
            fused[name] = bench_config(torch, hsdpa, W, name, "decode", args.steps, args.warmup, form="fused")
        if fused:
            result["configs_fused"] = fused
    wd = W.config("decode_32k", seed=0) if not args.no_cpu else None
    wp_cpu = W.config("prefill_4096_after_8192", seed=0) if ("prefill" in result and not args.no_cpu) else None

    # ---- decode at other lengths (same heads): fixed latency vs stream ---------
    if not args.no_sweep:
        sweep = {}
        for n in (1024, 8192, 32768, 131072):
            wn = W.make(f"decode_{n}", heads=16, kv_heads=2, head_dim=256, rows=1, past=n - 1, seed=3)
            copies = max(4, -(-(1 << 30) // (2 * 2 * n * 256 * 2)))       # at least 1 GiB of distinct caches
            q, ks, vs, out = device_buffers(torch, wn, copies=copies)
            plan_n = hsdpa.Plan(wn.heads, wn.gqa, wn.head_dim, wn.capacity)
            ws_n = torch.empty(plan_n.workspace_bytes, dtype=torch.uint8, device="cuda")
            n_ms, _, eager, replay = time_steps(torch, plan_n, wn, q, ks, vs, out, ws_n, 20, 3)
            if not torch.equal(eager, replay):
                print(f"decode {n}: graph replay differs from the eager call", file=sys.stderr)
                sys.exit(3)
            n_gbs = wn.decode_bytes() / (n_ms * 1e-3) / 1e9
            sweep[str(n)] = {"us": round(n_ms * 1e3, 2), "GB/s": round(n_gbs, 1), "frac": round(n_gbs / HBM_PEAK_GBS, 4)}
            log(f"decode {n:6d} keys: {n_ms*1e3:7.2f} us, {n_gbs:7.1f} GB/s ({n_gbs/HBM_PEAK_GBS:.1%})")
            del q, ks, vs, out, ws_n
            torch.cuda.empty_cache()
        result["decode_sweep"] = {"keys": sweep, "config": "16 query heads on 2 KV heads, head_dim 256, 1 row; "
                                                           "caches rotated over at least 1 GiB; 20 graph steps"}
        # a few rows after the 32K cache (speculative verification): (row, head)
        # columns on the decode kernels
        few = {}
        for rows in (2, 4, 8, 16):
            wf = W.make(f"few_{rows}", heads=16, kv_heads=2, head_dim=256, rows=rows, past=32768 - rows, seed=3)
            q, ks, vs, out = device_buffers(torch, wf, copies=16)
            plan_f = hsdpa.Plan(wf.heads, wf.gqa, wf.head_dim, wf.capacity)
            ws_f = torch.empty(plan_f.workspace_bytes, dtype=torch.uint8, device="cuda")
            f_ms, _, eager, replay = time_steps(torch, plan_f, wf, q, ks, vs, out, ws_f, 20, 3)
            if not torch.equal(eager, replay):
                print(f"{rows} rows: graph replay differs from the eager call", file=sys.stderr)
                sys.exit(3)
            few[str(rows)] = {"us": round(f_ms * 1e3, 2)}
            log(f"{rows} rows after {32768 - rows} keys: {f_ms*1e3:7.2f} us")
            del q, ks, vs, out, ws_f
            torch.cuda.empty_cache()
        result["few_rows"] = {"rows": few, "config": "16 query heads on 2 KV heads, head_dim 256, rows after "
                                                     "32768 - rows cached keys; 16 rotating caches; 20 graph steps"}

    # ---- the layer chain: norms, append, attention, gate -------------------------
    if not args.no_layer:
        wl = W.config("decode_32k", seed=1)
        f_ms, n_ms, same = time_layer(torch, hsdpa, wl, 16, args.steps, args.warmup)
        if not same:
            print("fused layer chain differs from the separate nodes", file=sys.stderr)
            sys.exit(3)
        layer = {"decode_32k": {"fused_us": round(f_ms * 1e3, 2), "nodes_us": round(n_ms * 1e3, 2),
                                "launches": {"fused": 4, "nodes": 7}}}
        log(f"layer decode_32k: fused {f_ms*1e3:.2f} us, nodes {n_ms*1e3:.2f} us")
        del wl
        if not args.no_prefill:
            wl = W.config("prefill_4096_after_8192", seed=1)
            psteps = args.prefill_steps or min(args.steps, 20)
            f_ms, n_ms, same = time_layer(torch, hsdpa, wl, 1, psteps, min(args.warmup, 3))
            if not same:
                print("fused layer chain differs from the separate nodes", file=sys.stderr)
                sys.exit(3)
            layer["prefill_4096_after_8192"] = {"fused_ms": round(f_ms, 4), "nodes_ms": round(n_ms, 4),
                                                "launches": {"fused": 2, "nodes": 5}}
            log(f"layer prefill: fused {f_ms:.3f} ms, nodes {n_ms:.3f} ms")
            del wl
        result["layer"] = dict(layer, workload="gated Qwen3.5 attention layer: q and k RMS-norm (1+w) + RoPE 64 of 256, "
                                               "KV append, attention, output gate; fused = hsdpa_attention_layer, "
                                               "nodes = the five calls in order; bit-identical results checked",
                               timing="HIP graph of the timed steps")
        torch.cuda.empty_cache()

    # ---- CPU baseline ------------------------------------------------------------
    if not args.no_cpu:
        cb, why = cpu_baseline(wd)
        if cb is None:
            result["cpu_baseline"] = {"value": None, "unit": "GB/s", "cores": 0, "kind": "port", "sample": why}
        else:
            import oracle

            result["cpu_baseline"] = cb
            cores = oracle.lib().oracle_physical_cores()
            if wp_cpu is not None:
                result["prefill"]["cpu_baseline"] = cpu_prefill_sample(wp_cpu, cores)
            # every configuration's own CPU figure beside its GPU one (the
            # 4096-row chunk: the bounded sample above; the headline: above)
            for name, rec in configs.items():
                if name == "decode_32k":
                    rec["cpu_baseline"] = {k: cb[k] for k in ("value", "unit", "cores", "kind", "sample")}
                elif name == "prefill_4096_after_8192":
                    rec["cpu_baseline"] = result["prefill"]["cpu_baseline"]
                else:
                    kind = "prefill" if name.startswith("prefill") else "decode"
                    rec["cpu_baseline"] = cpu_config_baseline(W.config(name, seed=0), kind, cores)
                log(f"{name} cpu: {rec['cpu_baseline']['value']} {rec['cpu_baseline']['unit']}")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
