"""CPU tests of the C ABI of libhsdpa.so: it loads, exports every entry point
include/hsdpa.h declares, and refuses every invalid plan or call on the host
with the named status, before any device work."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import hsdpa
from hsdpa import binding
from hsdpa import workloads as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hsdpa.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*[a-z_ 0-9*]*?\b(hsdpa_[a-z_]+)\s*\(", text, re.M)))


def test_header_declares_the_abi():
    assert declared_functions() == sorted(binding.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = hsdpa.library()
    for name in declared_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", hsdpa.library_path()], capture_output=True, text=True).stdout
    for name in declared_functions():
        assert re.search(rf"\bT {name}$", out, re.M), name


def test_library_has_gfx950_code():
    """The fat binary embedded in libhsdpa.so carries a gfx950 code object."""
    out = subprocess.run(["objdump", "-h", hsdpa.library_path()], capture_output=True, text=True).stdout
    assert ".hip_fatbin" in out
    data = open(hsdpa.library_path(), "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in data


def test_status_strings_and_version():
    lib = hsdpa.library()
    for code in range(17):
        assert lib.hsdpa_status_string(code) != b"unknown status", code
    assert lib.hsdpa_version() >= 200


@pytest.mark.parametrize("kw,code", [
    (dict(heads=16, gqa=3, head_dim=256, kv_capacity=10), "HSDPA_ERR_GQA"),
    (dict(heads=16, gqa=8, head_dim=48, kv_capacity=10), "HSDPA_ERR_HEAD_DIM"),
    (dict(heads=16, gqa=8, head_dim=16, kv_capacity=10), "HSDPA_ERR_HEAD_DIM"),
    (dict(heads=16, gqa=8, head_dim=544, kv_capacity=10), "HSDPA_ERR_HEAD_DIM"),
    (dict(heads=16, gqa=8, head_dim=1024, kv_capacity=10), "HSDPA_ERR_HEAD_DIM"),
    (dict(heads=16, gqa=8, head_dim=256, kv_capacity=10, sink=2), "HSDPA_ERR_SINK_UNSUPPORTED"),
    (dict(heads=0, gqa=1, head_dim=256, kv_capacity=1), "HSDPA_ERR_EMPTY"),
    (dict(heads=16, gqa=8, head_dim=0, kv_capacity=1), "HSDPA_ERR_EMPTY"),
    (dict(heads=16, gqa=8, head_dim=256, kv_capacity=10, q_head=128), "HSDPA_ERR_STRIDE"),
    (dict(heads=16, gqa=8, head_dim=256, kv_capacity=10, q_row=1024), "HSDPA_ERR_STRIDE"),
    (dict(heads=16, gqa=8, head_dim=256, kv_capacity=10, out_row=256), "HSDPA_ERR_STRIDE"),
    (dict(heads=16, gqa=8, head_dim=256, kv_capacity=10, kv_stride=2000), "HSDPA_ERR_STRIDE"),
    (dict(heads=16, gqa=8, head_dim=256, kv_capacity=0), "HSDPA_ERR_CAPACITY"),
    (dict(heads=16, gqa=8, head_dim=256, kv_capacity=10, q_row=16 * 256 + 4), "HSDPA_ERR_ALIGNMENT"),
    (dict(heads=16, gqa=8, head_dim=256, kv_capacity=10, form=2), "HSDPA_ERR_FORM"),
    (dict(heads=16, gqa=8, head_dim=256, kv_capacity=10, max_rows=11), "HSDPA_ERR_CAPACITY"),
])
def test_plan_refusals(kw, code):
    with pytest.raises(hsdpa.HsdpaError) as e:
        hsdpa.Plan(**kw)
    assert e.value.name == code


def test_plan_accepts_engine_geometries():
    # the gated layout: q rows carry Q then the gate, 2*q_dim apart
    p = hsdpa.Plan(16, 8, 256, 8192, q_row=2 * 16 * 256, out_row=16 * 256, grouped=True)
    assert p.workspace_bytes > 0
    # every head dimension the reference's SdpaShape::check accepts: multiples
    # of 32 up to 512 (ir.rs:130-162)
    for d in range(32, 513, 32):
        hsdpa.Plan(8, 2, d, 1024)


def test_workspace_grows_with_capacity():
    a = hsdpa.Plan(16, 8, 256, 1024).workspace_bytes
    b = hsdpa.Plan(16, 8, 256, 32768).workspace_bytes
    assert b > a and b % 256 == 0


def test_workspace_follows_max_rows_and_form():
    """A plan sized for what it serves: a decode-only plan (max_rows 1) needs
    the scores, the pass-1 maxima and one round of pass-2 partials, a few MiB
    at 32K keys; any rows adds the few-rows columns and the split causal
    kernel's cells; the Fused form adds the 16-key block maxima and the
    partials' correction products."""
    any_rows = hsdpa.Plan(16, 8, 256, 32768).workspace_bytes
    decode = hsdpa.Plan(16, 8, 256, 32768, max_rows=1).workspace_bytes
    fused = hsdpa.Plan(16, 8, 256, 32768, max_rows=1, form="fused").workspace_bytes
    # scores 2 x 8 x 32768 f32, partials of 128 workgroups x 8 columns x 256 f32 per KV head
    assert 2 * 8 * 32768 * 4 + 2 * 128 * 8 * 256 * 4 <= decode < 5 << 20
    assert any_rows > 10 * decode
    assert fused - decode >= 2 * 8 * (32768 // 16) * 4
    # no split cells where every call runs on the decode kernels
    assert hsdpa.Plan(16, 8, 256, 32768, max_rows=8).workspace_bytes < 40 << 20


def test_route_names_the_kernels():
    """hsdpa_attention_route reports what a call would run, with no device:
    the decode passes for one row, (row, head) columns for a few rows, the
    causal kernel or its split or paired form otherwise; under the Fused form the rows
    outside full chunks of 8 take the Fused numerics on the decode kernels."""
    p = hsdpa.Plan(16, 8, 256, 40000)
    assert p.route(1, 32767)["main"] == "decode"
    assert p.route(4, 100)["main"] == "few_rows"
    # up to 1024 visible keys (one row, one group of at most 8 heads) pass 2
    # writes the outputs itself: two launches; past that, or with more heads
    # per KV head, three
    assert p.route(1, 1023)["launches"] == 2 and p.route(1, 0)["launches"] == 2
    assert p.route(1, 1024)["launches"] == 3
    assert hsdpa.Plan(32, 16, 256, 4096).route(1, 100)["launches"] == 2       # 16 heads: two P blocks
    assert hsdpa.Plan(64, 32, 256, 4096).route(1, 100)["launches"] == 3       # two groups
    assert hsdpa.Plan(16, 8, 256, 4096).route(2, 100)["launches"] == 2        # 2 rows: 16 (row, head) columns
    assert hsdpa.Plan(16, 8, 256, 4096).route(3, 100)["launches"] == 3
    assert hsdpa.Plan(32, 16, 256, 4096).route(1, 1000)["launches"] == 3      # 16 columns x 1001 keys
    assert hsdpa.Plan(16, 8, 256, 4096, form="fused").route(1, 100)["launches"] == 2
    assert hsdpa.Plan(16, 8, 256, 4096, form="fused").route(1, 1024)["launches"] == 3
    assert hsdpa.Plan(16, 8, 96, 4096).route(1, 100)["launches"] == 3
    r = p.route(4096, 8192)       # one round of row groups, the longest paired with the shortest
    assert r["main"] == "causal_paired" and r["launches"] == 3 and r["tail"] == "none"
    r = p.route(8192, 0)          # two rounds: the heaviest row groups first
    assert r["main"] == "causal" and r["launches"] == 1
    # pairing needs one round of row groups whose longest sees at least 64 key
    # tiles and gains at least an eighth
    assert hsdpa.Plan(16, 8, 256, 4096).route(4096, 0)["main"] == "causal_paired"   # 1..128 tiles
    assert hsdpa.Plan(16, 8, 256, 3000).route(3000, 0)["main"] == "causal_paired"   # 94 row groups
    assert hsdpa.Plan(40, 1, 64, 1000).route(1000, 0)["main"] == "causal"           # 32 tiles at most
    assert hsdpa.Plan(64, 8, 256, 5120).route(1024, 4096)["main"] == "causal"       # 129..160: < 1/8
    assert hsdpa.Plan(32, 8, 256, 4096).route(4096, 0)["main"] == "causal"          # 512 row groups
    r = p.route(256, 32768)
    assert r["main"] == "causal_split" and r["splits"] > 1 and r["launches"] == 3
    f = hsdpa.Plan(16, 8, 256, 40000, form="fused")
    assert f.route(1, 100)["main_form"] == "fused"
    assert f.route(7, 100)["main_form"] == "fused"
    assert f.route(8, 100)["main_form"] == "chained"          # a full chunk: the block kernel's numerics
    r = f.route(13, 100)
    assert (r["main_rows"], r["main_form"], r["tail_rows"], r["tail"], r["tail_form"]) == \
        (8, "chained", 5, "few_rows", "fused")
    r = f.route(4096 + 3, 8192)
    assert (r["main"], r["tail"], r["tail_rows"], r["tail_form"]) == ("causal_paired", "few_rows", 3, "fused")
    # above head_dim 256 the Fused form falls back to Chained
    assert hsdpa.Plan(4, 2, 288, 100, form="fused").route(1, 10)["main_form"] == "chained"
    # the Fused form declines the sink (emit_sdpa.rs:468-470): Chained, on every part
    r = hsdpa.Plan(16, 8, 256, 40000, form="fused", sink=True).route(13, 100)
    assert (r["main_form"], r["tail_form"]) == ("chained", "chained")
    # a group size with no equal split into groups of at most 16 (17) takes padded
    # groups on the decode kernels at the tuned head dimensions...
    r = hsdpa.Plan(17, 17, 128, 100, form="fused").route(1, 10)
    assert r["main"] == "decode" and r["main_form"] == "fused"
    assert hsdpa.Plan(160, 80, 256, 40000).route(1, 32767)["main"] == "decode"     # 80 heads: 5 groups of 16
    # ...and at the other head dimensions a Chained plan keeps the causal kernel
    assert hsdpa.Plan(17, 17, 96, 100).route(1, 10)["main"] == "causal"
    # while a Fused plan serves every row outside full chunks of 8 with the
    # Fused numerics on padded decode groups, as the reference's Fused head
    # does: a group size with no equal split at D 96, more than 256 heads per
    # KV head, padded groups over a long cache
    for spec, rows, past in [((17, 17, 96, 100), 1, 10), ((17, 17, 96, 4000), 1, 3000),
                             ((300, 300, 64, 1000), 1, 500), ((100, 100, 128, 40000), 1, 32000),
                             ((34, 17, 160, 100), 1, 50)]:
        r = hsdpa.Plan(*spec, form="fused").route(rows, past)
        assert r["main"] == "decode" and r["main_form"] == "fused", (spec, r)
        assert hsdpa.Plan(*spec).route(rows, past)["main"] != "decode", spec
    r = hsdpa.Plan(17, 17, 96, 100, form="fused").route(11, 50)
    assert (r["main"], r["main_form"], r["tail"], r["tail_form"]) == ("causal", "chained", "decode_rows", "fused")
    # beyond 65 536 query heads per KV head the Fused form has no decode grid
    with pytest.raises(hsdpa.HsdpaError):
        hsdpa.Plan(65537, 65537, 64, 10, form="fused")
    # one row per decode where the tail does not fit the decode columns (5 rows
    # of 32 heads: 160 columns, past 128)
    r = hsdpa.Plan(64, 32, 128, 1000, form="fused").route(13, 100)
    assert r["tail"] == "decode_rows" and r["tail_form"] == "fused" and r["launches"] == 1 + 5 * 3
    # up to 16 rows within 128 columns take the few-rows kernels together
    r = hsdpa.Plan(32, 16, 128, 1000, form="fused").route(13, 100)
    assert r["main"] == "few_rows" and r["tail"] == "few_rows" and r["tail_form"] == "fused"
    assert hsdpa.Plan(16, 8, 256, 40000).route(16, 30000)["main"] == "few_rows"
    assert hsdpa.Plan(16, 8, 256, 40000).route(17, 30000)["main"] != "few_rows"
    # past 8 rows or 64 columns only while groups x keys stay within the bound:
    # 8 groups x 128K keys at D 256, 8 groups x 32K keys at D 128 go causal
    assert hsdpa.Plan(16, 8, 256, 140000).route(16, 131000)["main"] == "causal_split"
    assert hsdpa.Plan(16, 8, 256, 140000).route(9, 131000)["main"] == "few_rows"
    assert hsdpa.Plan(32, 8, 128, 40000).route(16, 32000)["main"] == "causal_split"
    assert hsdpa.Plan(32, 8, 128, 40000).route(16, 6000)["main"] == "few_rows"
    assert hsdpa.Plan(32, 8, 128, 40000).route(8, 32000)["main"] == "few_rows"


def _call(plan, rows=1, past=0, scale=0.0625, sink=0.0, ws_bytes=None, q=0x10000, k=0x20000, v=0x30000,
          out=0x40000, ws=0x50000):
    nb = plan.workspace_bytes if ws_bytes is None else ws_bytes
    c = binding.Call(q, k, v, out, rows, past, scale, sink, ws, nb)
    return hsdpa.library().hsdpa_attention(plan.handle, ctypes.byref(c), None)


def _name(rc):
    return binding.STATUS[rc]


def _frame(plan, rows=0x60000, past=0x60008, status=0, **kw):
    f = dict(q=0x10000, keys=0x20000, values=0x30000, output=0x40000, rows=rows, past=past, scale=0.0625,
             sink=0.0, workspace=0x50000, workspace_bytes=plan.workspace_bytes, status=status)
    f.update(kw)
    c = binding.FrameCall(**f)
    return _name(hsdpa.library().hsdpa_attention_frame(plan.handle, ctypes.byref(c), None))


def test_frame_call_refusals_before_any_device_work():
    """hsdpa_attention_frame takes decode-only plans at head_dim 64, 128 and
    256 with equal decode groups; everything else is refused on the host
    before any launch, as are missing pointers, misalignment and a short
    workspace (rows and past are only read on the device)."""
    assert _frame(hsdpa.Plan(16, 8, 256, 4096)) == "HSDPA_ERR_FRAME"                   # any rows
    assert _frame(hsdpa.Plan(16, 8, 96, 4096, max_rows=1)) == "HSDPA_ERR_FRAME"        # untuned head_dim
    assert _frame(hsdpa.Plan(17, 17, 128, 4096, max_rows=1)) == "HSDPA_ERR_FRAME"      # padded groups
    assert _frame(hsdpa.Plan(100, 100, 128, 4096, max_rows=1)) == "HSDPA_ERR_FRAME"    # more than 4 groups
    # the step's configuration is derived in 32 bits on the device: the
    # capacity and groups x ceil(capacity / 128) must stay below 2^31
    assert _frame(hsdpa.Plan(1024, 1, 64, 1 << 28, max_rows=1)) == "HSDPA_ERR_FRAME"
    assert _frame(hsdpa.Plan(1023, 1, 64, 1 << 28, max_rows=1)) != "HSDPA_ERR_FRAME"
    assert _frame(hsdpa.Plan(16, 8, 64, 1 << 31, max_rows=1)) == "HSDPA_ERR_FRAME"
    assert _frame(hsdpa.Plan(16, 8, 64, (1 << 31) - 1, max_rows=1)) != "HSDPA_ERR_FRAME"
    p = hsdpa.Plan(16, 8, 256, 4096, max_rows=1)
    assert _frame(p, rows=0) == "HSDPA_ERR_NULL"
    assert _frame(p, past=0) == "HSDPA_ERR_NULL"
    assert _frame(p, rows=0x60004) == "HSDPA_ERR_ALIGNMENT"
    assert _frame(p, status=0x60002) == "HSDPA_ERR_ALIGNMENT"
    assert _frame(p, q=0x10008) == "HSDPA_ERR_ALIGNMENT"
    assert _frame(p, workspace_bytes=p.workspace_bytes - 1) == "HSDPA_ERR_WORKSPACE"
    # every check passed: with no GPU the device check refuses (a sink value
    # without the plan's sink flag is ignored, as the reference's call does)
    assert _frame(p) == "HSDPA_ERR_NO_DEVICE"
    assert _frame(p, sink=1.0) == "HSDPA_ERR_NO_DEVICE"
    assert _frame(hsdpa.Plan(16, 8, 256, 4096, max_rows=1, sink=True), sink=1.0) == "HSDPA_ERR_NO_DEVICE"
    assert _frame(hsdpa.Plan(64, 32, 128, 4096, max_rows=1, form="fused")) == "HSDPA_ERR_NO_DEVICE"


def test_call_refusals_before_any_device_work():
    p = hsdpa.Plan(16, 8, 256, 100)
    assert _name(_call(p, rows=0)) == "HSDPA_OK"                     # the empty call is a no-op
    assert _name(_call(p, rows=2, past=99)) == "HSDPA_ERR_CAPACITY"
    assert _name(_call(p, rows=101)) == "HSDPA_ERR_CAPACITY"
    assert _name(_call(p, rows=1, past=2**63)) == "HSDPA_ERR_CAPACITY"
    assert _name(_call(p, sink=0.5)) == "HSDPA_ERR_NO_DEVICE"        # ignored without the flag
    assert _name(_call(hsdpa.Plan(16, 8, 256, 100, sink=True), sink=0.5)) == "HSDPA_ERR_NO_DEVICE"
    assert _name(_call(p, q=0)) == "HSDPA_ERR_NULL"
    assert _name(_call(p, ws=0)) == "HSDPA_ERR_NULL"
    assert _name(_call(p, k=0x20002)) == "HSDPA_ERR_ALIGNMENT"
    assert _name(_call(p, ws_bytes=16)) == "HSDPA_ERR_WORKSPACE"
    assert hsdpa.library().hsdpa_attention(None, None, None) == 9
    one = hsdpa.Plan(16, 8, 256, 100, max_rows=1)
    assert _name(_call(one, rows=2)) == "HSDPA_ERR_BATCH"


def test_call_without_gpu_fails_loudly():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    p = hsdpa.Plan(16, 8, 256, 100)
    assert _name(_call(p)) == "HSDPA_ERR_NO_DEVICE"


def test_workloads_are_deterministic_and_shaped():
    a = W.config("decode_1k", seed=4)
    b = W.config("decode_1k", seed=4)
    assert np.array_equal(a.q, b.q) and np.array_equal(a.k, b.k) and np.array_equal(a.v, b.v)
    assert a.q.shape == (1, 8, 256) and a.k.shape == (2, 1024, 256)
    assert a.decode_bytes() == 2105344
    c = W.config("decode_32k", seed=0)
    assert c.decode_bytes() == 67125248
    p = W.make("p", heads=16, kv_heads=2, head_dim=256, rows=4096, past=8192, capacity=12288)
    assert p.prefill_flops() == 687228321792
    x = W.normal_f32(9, 1 << 16)
    assert abs(float(x.mean())) < 0.02 and abs(float(x.std()) - 1) < 0.02


def test_outlier_workload():
    w = W.make("o", heads=4, kv_heads=2, head_dim=64, rows=1, past=999, seed=3, outlier_keys=4,
               outlier_rows_frac=0.01)
    k = W.bf16_to_f32(w.k)
    v = W.bf16_to_f32(w.v)
    for h in range(2):
        std = k[h].std(axis=0)
        assert (std > 10).sum() == 4
        rows = np.abs(v[h]).max(axis=1)
        assert (rows > 12).sum() >= 5


# ---- record layouts: the ctypes mirrors against the C header -------------------

RECORDS = {
    "hsdpa_spec": binding.Spec, "hsdpa_call": binding.Call, "hsdpa_kv_spec": binding.KvSpec,
    "hsdpa_kv_call": binding.KvCall, "hsdpa_norm_rope_spec": binding.NormRopeSpec,
    "hsdpa_norm_rope_call": binding.NormRopeCall, "hsdpa_gate_spec": binding.GateSpec,
    "hsdpa_gate_call": binding.GateCall, "hsdpa_layer_call": binding.LayerCall, "hsdpa_route": binding.Route,
    "hsdpa_frame_call": binding.FrameCall,
}


def test_record_layouts_match_the_header(tmp_path):
    """Every field of every record sits at the same offset, and every record
    has the same size, in the C compiler's layout and in the binding's."""
    if subprocess.run(["which", "gcc"], capture_output=True).returncode != 0:
        pytest.skip("no C compiler")
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "hsdpa.h"', "int main(void) {"]
    for rec, cls in RECORDS.items():
        lines.append(f'printf("{rec} size %zu\\n", sizeof({rec}));')
        for fname, _ in cls._fields_:
            lines.append(f'printf("{rec} {fname} %zu\\n", offsetof({rec}, {fname}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines():
        rec, field, value = line.split()
        got[(rec, field)] = int(value)
    for rec, cls in RECORDS.items():
        assert got[(rec, "size")] == ctypes.sizeof(cls), rec
        for fname, _ in cls._fields_:
            assert got[(rec, fname)] == getattr(cls, fname).offset, (rec, fname)


def test_decode_grids_fit_the_workspace():
    """Every decode call a plan can take fits the partials its workspace was
    sized for (the call refuses a grid beyond them with HSDPA_ERR_WORKSPACE,
    which the route query reports): group shapes, the tuned and other head
    dimensions, both forms, max_rows 1, 8 and any, rows 1 to 16 at cache
    lengths across the configurations' thresholds."""
    shapes = [(16, 8, 256), (48, 24, 256), (64, 8, 128), (32, 4, 128), (16, 16, 64), (8, 4, 256), (20, 10, 96),
              (17, 17, 128), (128, 64, 256)]
    pasts = [0, 100, 1023, 3000, 8191, 16383, 32767, 65535, 131000]
    for h, g, d in shapes:
        for form in ("chained", "fused"):
            for max_rows in (1, 8, 0):
                plan = hsdpa.Plan(h, g, d, 131072, form=form, max_rows=max_rows)
                for rows in (1, 2, 3, 4, 5, 8, 9, 16):
                    if max_rows and rows > max_rows:
                        continue
                    for past in pasts:
                        if past + rows > 131072:
                            continue
                        plan.route(rows, past)           # raises HsdpaError on a refusal
