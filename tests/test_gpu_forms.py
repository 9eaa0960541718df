"""GPU parity against the reference's other decode forms, through the C ABI.

  * Fused (a plan with form = HSDPA_FORM_FUSED): the decode kernels compute
    the Fused form's own weights (each 16-key block at its running maximum,
    times the later blocks' corrections) and are compared with the oracle's
    restatement of emit_fused (src/jit/target/x86/emit_sdpa/x86/decode.rs:
    501-669) under the node's selector: full 8-row chunks on the Chained
    numerics, the other rows Fused.
  * sdpa_qk_group = 0: the unchanged (Chained) HIP output against the bits of
    the reference's four-chain QK (src/jit/sdpa.rs:178-202);
  * AVX2: the unchanged (Chained) HIP output against the bits the reference
    emits on a host without AVX-512 BF16
    (src/jit/target/x86/emit_sdpa_avx2.rs:231-470), where every row runs the
    AVX2 head.
Each case first checks on the host which kernels and numerics the call takes
(hsdpa_attention_route).
"""
import pytest

import hsdpa
import oracle
from hsdpa import workloads as W
from parity import assert_parity

from gpu_util import run_hsdpa

pytestmark = pytest.mark.gpu

FUSED = [
    # name, heads, kv_heads, head_dim, rows, past, (main kernels, main form), (tail kernels, tail form)
    ("fused_d256_n1", 8, 2, 256, 1, 0, ("decode", "fused"), None),
    ("fused_d256_n15", 8, 2, 256, 1, 14, ("decode", "fused"), None),
    ("fused_d256_n17", 8, 2, 256, 1, 16, ("decode", "fused"), None),
    ("fused_d256_n300", 8, 2, 256, 1, 299, ("decode", "fused"), None),
    # up to 1024 keys pass 2 takes every key and writes the outputs: 64 blocks
    ("fused_d128_n1024_g8", 16, 2, 128, 1, 1023, ("decode", "fused"), None),
    ("fused_d128_n5000_g4", 16, 4, 128, 1, 4999, ("decode", "fused"), None),
    ("fused_d64_g1_n777", 4, 4, 64, 1, 776, ("decode", "fused"), None),
    ("fused_d32_n1000", 8, 2, 32, 1, 999, ("decode", "fused"), None),
    ("fused_d96_n1000", 8, 2, 96, 1, 999, ("decode", "fused"), None),
    ("fused_d160_n3000", 8, 2, 160, 1, 2999, ("decode", "fused"), None),
    ("fused_d224_n513", 4, 1, 224, 1, 512, ("decode", "fused"), None),
    # pass 1 two tiles per wave; pass 2 in chunks, each chunk rescaling the earlier ones
    ("fused_d256_n20001_two_tiles", 16, 2, 256, 1, 20000, ("decode", "fused"), None),
    ("fused_d256_n50001_chunked", 16, 2, 256, 1, 50000, ("decode", "fused"), None),
    ("fused_d128_g16_n20001_chunked", 64, 4, 128, 1, 20000, ("decode", "fused"), None),
    # two P column blocks; several groups per KV head
    ("fused_d256_g12_n40", 12, 1, 256, 1, 39, ("decode", "fused"), None),
    ("fused_d128_g48_three_groups", 48, 1, 128, 1, 3000, ("decode", "fused"), None),
    ("fused_d256_g24_two_groups", 48, 2, 256, 1, 33000, ("decode", "fused"), None),
    # more than 512 pass-2 workgroups per head: the combine scans two segments
    ("fused_d256_g12_n200001_segments", 24, 2, 256, 1, 200000, ("decode", "fused"), None),
    # a few rows: all outside a full chunk of 8, so all Fused; 8 rows are a chunk
    ("fused_few_r3_d256_g8_p37", 16, 2, 256, 3, 37, ("few_rows", "fused"), None),
    ("fused_few_r7_d128_g8_p900", 16, 2, 128, 7, 900, ("few_rows", "fused"), None),
    ("fused_few_r4_d128_p40000_chunked", 16, 2, 128, 4, 40000, ("few_rows", "fused"), None),
    ("fused_few_r8_d256_chunk", 16, 2, 256, 8, 500, ("few_rows", "chained"), None),
    # a full chunk of 8 rows over a long cache: the Chained pass 2 walking a run
    # for all four groups of a KV head
    ("fused_few_r8_d256_chunk_long", 16, 2, 256, 8, 70000, ("few_rows", "chained"), None),
    # prefill chunks: the last rows % 8 take the Fused numerics
    ("fused_prefill_r13_p100", 16, 2, 256, 13, 100, ("few_rows", "chained"), ("few_rows", "fused")),
    ("fused_prefill_r300_p9000", 16, 2, 256, 300, 9000, ("causal_split", "chained"), ("few_rows", "fused")),
    ("fused_prefill_r70_p5_d128", 8, 8, 128, 70, 5, ("causal", "chained"), ("few_rows", "fused")),
    ("fused_prefill_r9_g16", 32, 2, 128, 9, 50, ("few_rows", "chained"), ("decode", "fused")),
    ("fused_prefill_r13_g16", 32, 2, 128, 13, 100, ("few_rows", "chained"), ("few_rows", "fused")),
    ("fused_prefill_r9_g32", 64, 2, 128, 9, 50, ("causal", "chained"), ("decode", "fused")),
    ("fused_prefill_r13_g32", 64, 2, 128, 13, 100, ("causal", "chained"), ("decode_rows", "fused")),
    # padded groups (a group size with no equal split into groups of at most 16)
    ("fused_d128_g17_padded", 17, 1, 128, 1, 900, ("decode", "fused"), None),
    ("fused_d256_g17_padded_2kv_long", 34, 2, 256, 1, 40000, ("decode", "fused"), None),
    ("fused_few_r5_g7_d256_padded", 7, 1, 256, 5, 300, ("few_rows", "fused"), None),
    # shapes the Chained form serves on the causal kernels: under the Fused
    # form every row outside a full chunk of 8 takes padded decode groups
    ("fused_d96_g17_padded", 17, 1, 96, 1, 900, ("decode", "fused"), None),
    ("fused_d96_g17_prefill_tail", 17, 1, 96, 11, 50, ("causal", "chained"), ("decode_rows", "fused")),
    ("fused_d160_g34_padded_2kv", 68, 2, 160, 1, 5000, ("decode", "fused"), None),
    ("fused_d64_g300_padded", 300, 1, 64, 1, 600, ("decode", "fused"), None),
    ("fused_d128_g100_padded_long", 100, 1, 128, 1, 32000, ("decode", "fused"), None),
    # above head_dim 256 the form falls back to Chained, like the reference
    ("fused_d288_falls_back", 4, 2, 288, 1, 300, ("decode", "chained"), None),
]


@pytest.mark.parametrize("case", FUSED, ids=[c[0] for c in FUSED])
def test_fused_form(torch_cuda, case):
    name, h, kvh, d, rows, past, main, tail = case
    w = W.make(name, heads=h, kv_heads=kvh, head_dim=d, rows=rows, past=past, seed=13)
    plan = hsdpa.Plan(w.heads, w.gqa, w.head_dim, w.capacity, form="fused")
    r = plan.route(rows, past)
    assert (r["main"], r["main_form"]) == main, r
    assert (r["tail"], r["tail_form"]) == (tail or ("none", "chained")), r
    print(f"case {name}", flush=True)
    out = run_hsdpa(w, plan)
    ref = oracle.attention(w, form="fused")
    res = assert_parity(out, ref, w, name)
    print(name, res, flush=True)


@pytest.mark.parametrize("name", ["decode_1k", "decode_32k", "decode_128k_outliers"])
def test_fused_configs(torch_cuda, name):
    """The benchmark's decode configurations at full size under the Fused form."""
    w = W.config(name, seed=3)
    plan = hsdpa.Plan(w.heads, w.gqa, w.head_dim, w.capacity, form="fused")
    print(f"config {name} fused", flush=True)
    out = run_hsdpa(w, plan)
    ref = oracle.attention(w, form="fused")
    res = assert_parity(out, ref, w, name)
    print(name, res, flush=True)


def test_fused_plan_leaves_chained_rows_unchanged(torch_cuda):
    """Rows in full chunks of 8 are the Chained kernels' under either form:
    the Fused plan runs the first 16 of 21 rows as the Chained plan runs a
    16-row call (bit for bit), and the last 5 on the Fused decode kernels."""
    w = W.make("fused_mixed", heads=16, kv_heads=2, head_dim=256, rows=21, past=300, seed=4)
    fused = run_hsdpa(w, hsdpa.Plan(w.heads, w.gqa, w.head_dim, w.capacity, form="fused"))
    w16 = W.Workload("chained_16", w.heads, w.kv_heads, w.head_dim, 16, w.past, w.capacity, w.q[:16], w.k, w.v,
                     w.scale)
    chained16 = run_hsdpa(w16, hsdpa.Plan(w.heads, w.gqa, w.head_dim, w.capacity))
    assert (fused[:16] == chained16).all()
    chained = run_hsdpa(w, hsdpa.Plan(w.heads, w.gqa, w.head_dim, w.capacity))
    assert not (fused[16:] == chained[16:]).all()
    assert_parity(fused, oracle.attention(w, form="fused"), w, "fused_mixed")


@pytest.mark.parametrize("name", ["decode_1k", "decode_32k", "prefill_512", "decode_128k_outliers"])
def test_chained_output_against_avx2_bits(torch_cuda, name):
    """The default HIP path is within the parity bar of the reference's AVX2
    arm too (other summation orders, the same exponentials at the row maximum)."""
    w = W.config(name, seed=3)
    print(f"config {name} against the AVX2 arm", flush=True)
    out = run_hsdpa(w)
    ref = oracle.attention(w, form="avx2")
    res = assert_parity(out, ref, w, name)
    print(name, res, flush=True)


@pytest.mark.parametrize("name", ["decode_1k", "decode_32k", "prefill_512"])
def test_chained_output_against_qk_group0_bits(torch_cuda, name):
    """The default HIP path is within the parity bar of the bits the reference
    emits under the knob sdpa_qk_group = 0 too (src/jit/sdpa.rs:178-202: the
    QK in four chains instead of one, decode and prefill block alike; the same
    exponentials at the row maximum)."""
    w = W.config(name, seed=3)
    print(f"config {name} against sdpa_qk_group = 0", flush=True)
    out = run_hsdpa(w)
    ref = oracle.attention(w, form="chained_qk0")
    res = assert_parity(out, ref, w, name)
    print(name, res, flush=True)


AVX2_SMALL = [
    ("avx2_decode_d64_n777", 4, 4, 64, 1, 776),
    ("avx2_decode_d128_n9000", 16, 4, 128, 1, 8999),
    ("avx2_prefill_d256_r19_p37", 8, 2, 256, 19, 37),
    ("avx2_few_r5_d128", 16, 2, 128, 5, 900),
    ("avx2_decode_d96_n1000", 8, 2, 96, 1, 999),
]


@pytest.mark.parametrize("case", AVX2_SMALL, ids=[c[0] for c in AVX2_SMALL])
def test_avx2_small(torch_cuda, case):
    name, h, kvh, d, rows, past = case
    w = W.make(name, heads=h, kv_heads=kvh, head_dim=d, rows=rows, past=past, seed=19)
    print(f"case {name}", flush=True)
    out = run_hsdpa(w)
    ref = oracle.attention(w, form="avx2")
    res = assert_parity(out, ref, w, name)
    print(name, res, flush=True)
