"""GPU parity: libhsdpa.so (called through its C ABI) against the oracle, the
CPU restatement of the reference's emitted SDPA, on identical seeded inputs."""
import numpy as np
import pytest

import hsdpa
import oracle
from hsdpa import workloads as W
from parity import assert_parity

from gpu_util import run_hsdpa

pytestmark = pytest.mark.gpu

SMALL = [
    # name, heads, kv_heads, head_dim, rows, past, the kernels the call must take
    ("decode_d256_n1", 8, 2, 256, 1, 0, "decode"),
    ("decode_d256_n37", 8, 2, 256, 1, 36, "decode"),
    ("decode_d128_n300", 16, 4, 128, 1, 299, "decode"),
    ("decode_d64_g1", 4, 4, 64, 1, 77, "decode"),
    # up to 1024 keys pass 2 writes the outputs itself (no combine): both
    # sides of 1024, one partial tile, one head per KV head, odd groups
    ("decode_direct_d256_n1024_g8", 16, 2, 256, 1, 1023, "decode"),
    ("decode_combine_d128_n1025_g8", 16, 2, 128, 1, 1024, "decode"),
    ("decode_direct_d64_n33_g8", 8, 1, 64, 1, 32, "decode"),
    ("decode_direct_d128_n32_g1", 4, 4, 128, 1, 31, "decode"),
    ("decode_direct_d256_n700_g3_kv5", 15, 5, 256, 1, 699, "decode"),
    ("decode_direct_d256_g16_n200", 32, 2, 256, 1, 199, "decode"),               # two P column blocks
    ("decode_direct_d128_g12_n300", 12, 1, 128, 1, 299, "decode"),
    # more of them: partial tiles, odd groups
    ("decode_direct_d256_n17_g7", 7, 1, 256, 1, 16, "decode"),
    ("decode_direct_d128_n257_g5_kv3", 15, 3, 128, 1, 256, "decode"),
    ("decode_direct_d64_n512_g2", 4, 2, 64, 1, 511, "decode"),
    ("decode_direct_d256_n1000_g6", 12, 2, 256, 1, 999, "decode"),
    ("prefill_d256_r2_g80", 160, 2, 256, 2, 0, "causal"),             # 160 columns: past the decode kernels
    ("prefill_d256_r19_p37", 8, 2, 256, 19, 37, "causal"),
    ("prefill_d128_r70_p5", 8, 8, 128, 70, 5, "causal"),
    ("prefill_d64_r33_p100_g2", 8, 4, 64, 33, 100, "causal"),
    ("prefill_d256_r129_p0_g3", 6, 2, 256, 129, 0, "causal"),
    # pass 1 in several rounds per workgroup, the last workgroup partial
    ("decode_d256_n50001_two_rounds", 16, 2, 256, 1, 50000, "decode"),
    ("decode_d128_n70001_five_rounds", 16, 4, 128, 1, 70000, "decode"),
    # two tiles per wave once one tile per wave needs more than a workgroup per CU
    ("decode_d256_n20001_two_tiles", 16, 2, 256, 1, 20000, "decode"),
    ("decode_d128_n9000_kv4_two_tiles", 16, 4, 128, 1, 8999, "decode"),
    # pass 2 in chunks, one round of workgroups, the last chunk of each run partial
    ("decode_d256_n40001_chunked", 16, 2, 256, 1, 40000, "decode"),
    ("decode_d128_kv8_n9000_chunked", 64, 8, 128, 1, 8999, "decode"),
    ("decode_d128_g16_n20001_chunked", 64, 4, 128, 1, 20000, "decode"),   # two P column blocks
    # one round of causal workgroups whose longest row groups are paired with
    # the shortest (the heavy row group's last tiles walked by the light one's
    # workgroup): odd row-group counts (a middle row group alone), partial last
    # row groups, the other head dimensions
    ("prefill_paired_d64_r2200_g1", 24, 24, 64, 2200, 0, "causal_paired"),
    ("prefill_paired_d128_r3000", 16, 2, 128, 3000, 0, "causal_paired"),
    ("prefill_paired_d256_r2200_p1000_odd", 16, 2, 256, 2200, 1000, "causal_paired"),
    ("prefill_paired_d256_r4000_p300", 16, 2, 256, 4000, 300, "causal_paired"),
    ("prefill_paired_d96_r2200_g1", 24, 24, 96, 2200, 0, "causal_paired"),
    ("prefill_paired_d384_r2200_g1", 12, 12, 384, 2200, 0, "causal_paired"),
    ("prefill_d64_r1000_g1_short_rows", 40, 40, 64, 1000, 0, "causal"),    # 32 tiles: too few to pair
    # short chunks after long caches: the causal kernel split over the keys
    ("prefill_split_d256_r64_p3000", 16, 2, 256, 64, 3000, "causal_split"),
    ("prefill_split_d256_r300_p9000", 16, 2, 256, 300, 9000, "causal_split"),
    ("prefill_split_d128_r100_p5000_g4", 16, 4, 128, 100, 5000, "causal_split"),
    ("prefill_split_d64_r40_p2000_g2", 8, 4, 64, 40, 2000, "causal_split"),
    ("prefill_split_d96_r50_p4000", 8, 2, 96, 50, 4000, "causal_split"),
    ("prefill_split_d384_r33_p2500", 4, 2, 384, 33, 2500, "causal_split"),
    ("prefill_split_d256_r7_p1200_uneven_g40", 80, 2, 256, 7, 1200, "causal_split"),  # 38 tiles over 9 splits
    # short chunks that few key tiles: each row block's keys split among its waves
    ("prefill_short_d256_r512_p0_g4", 16, 4, 256, 512, 0, "causal_short"),
    ("prefill_short_d256_r1024_p0_g8", 16, 2, 256, 1024, 0, "causal_short"),
    ("prefill_short_d128_r300_p100", 16, 2, 128, 300, 100, "causal_short"),
    ("prefill_short_d256_r200_p300_g8", 32, 4, 256, 200, 300, "causal_short"),
    ("prefill_short_d256_r7_p257_g40", 80, 2, 256, 7, 257, "causal_short"),       # one partial row block
    ("prefill_short_d64_r500_p0", 8, 2, 64, 500, 0, "causal_short"),
    ("prefill_short_d256_r33_p0", 16, 2, 256, 33, 0, "causal"),                   # fills no split: one-workgroup kernel
    # at D 128 and 256 the waves split the dimensions for P.V, every workgroup
    # running the launch's tile count in rounds of 4 (D 128) or 8 (D 256)
    ("prefill_short_d128_r200_p50_g4_8_tiles", 16, 4, 128, 200, 50, "causal_short"),
    ("prefill_short_d256_r150_p90_8_tiles", 16, 2, 256, 150, 90, "causal_short"),
    ("prefill_short_d128_r300_p60_12_tiles", 16, 2, 128, 300, 60, "causal_short"),
    ("prefill_short_d256_r481_p30_16_tiles_partial_block", 16, 2, 256, 481, 30, "causal_short"),
    # beyond 16 tiles the P operands of two rounds at a time: 24 and 32 tiles
    ("prefill_short_d256_r256_p500_24_tiles", 16, 2, 256, 256, 500, "causal_short"),
    ("prefill_short_d128_r300_p400_g4_24_tiles", 16, 4, 128, 300, 400, "causal_short"),
    ("prefill_short_d128_r512_p400_32_tiles", 16, 2, 128, 512, 400, "causal_short"),
]


@pytest.mark.parametrize("case", SMALL, ids=[c[0] for c in SMALL])
def test_small_shapes(torch_cuda, case):
    name, h, kvh, d, rows, past, kernels = case
    w = W.make(name, heads=h, kv_heads=kvh, head_dim=d, rows=rows, past=past, seed=11)
    plan = hsdpa.Plan(w.heads, w.gqa, w.head_dim, w.capacity)
    assert plan.route(rows, past)["main"] == kernels, plan.route(rows, past)
    print(f"case {name}", flush=True)
    out = run_hsdpa(w, plan)
    ref = oracle.attention(w)
    r = assert_parity(out, ref, w, name)
    print(name, r, flush=True)


# A few rows after a cache run on the decode kernels: one column per (row,
# head) pair, each row with its own causal limit, up to 4 groups of 16 columns
# per KV head; more columns take the causal kernel.
FEW = [
    # name, heads, kv_heads, head_dim, rows, past
    ("few_r2_d256_g8_p5000", 16, 2, 256, 2, 5000),
    ("few_r3_d256_g8_p37", 16, 2, 256, 3, 37),             # 24 columns: two groups of 12
    ("few_r4_d256_g8_p40000", 16, 2, 256, 4, 40000),       # two groups of 16, long cache
    ("few_r8_d128_g8_p3000", 16, 2, 128, 8, 3000),         # four groups of 16
    ("few_r5_d128_g8_p900", 16, 2, 128, 5, 900),           # four groups of 10
    ("few_r8_d64_g1_p100", 8, 8, 64, 8, 100),
    ("few_r2_d256_g16_p2000", 32, 2, 256, 2, 2000),
    ("few_r4_d128_g4_p0", 8, 2, 128, 4, 0),                # row r sees keys 0..r only
    ("few_r7_d256_g8_p0", 16, 2, 256, 7, 0),
    ("few_r8_d128_g16_p500", 32, 2, 128, 8, 500),           # 128 columns: 8 groups
    ("few_r2_d128_g32_p700", 32, 1, 128, 2, 700),          # 64 columns: four groups of 16
    ("few_r5_d256_g3_p333", 6, 2, 256, 5, 333),            # 15 columns: one group, two P blocks
    # pass 1 scoring every group of a KV head in one workgroup (more than one
    # round of such workgroups): four groups, two tiles per wave; two groups,
    # three tiles per wave at D 128
    ("few_r8_d256_g8_p20000", 16, 2, 256, 8, 20000),
    ("few_r4_d128_g8_p33000", 16, 2, 128, 4, 33000),
    # 9 to 16 rows: up to 8 groups of 16 columns (the last one padded), all
    # groups per workgroup over long caches, one workgroup per group otherwise
    # (within the groups x keys bound past 8 rows or 64 columns)
    ("few_r12_d256_g8_p20000", 16, 2, 256, 12, 20000),
    ("few_r14_d256_g8_p20000", 16, 2, 256, 14, 20000),     # 7 groups
    ("few_r16_d256_g8_p24000", 16, 2, 256, 16, 24000),     # 8 groups
    ("few_r16_d256_g8_p1500", 16, 2, 256, 16, 1500),
    ("few_r9_d64_g8_p700", 16, 2, 64, 9, 700),
    ("few_r16_d128_g8_p6000", 16, 2, 128, 16, 6000),
    ("few_r11_d128_g4_p0", 16, 4, 128, 11, 0),             # 44 columns, row r sees keys 0..r
    # up to 16 columns after a short cache: one launch for pass 2 and the outputs
    ("few_r2_d256_g8_p200_direct", 16, 2, 256, 2, 200),
    ("few_r3_d128_g4_p0_direct", 16, 4, 128, 3, 0),
    ("few_r2_d64_g8_p150_direct", 16, 2, 64, 2, 150),
    ("few_r2_d128_g4_p900_direct", 8, 2, 128, 2, 900),      # 8 columns: one P block, 902 keys
    # long caches at D 256 in 2 to 4 groups: pass 2 walks a run for all of a
    # KV head's groups in each workgroup (the last run partial; 3 groups; 4
    # groups of 10 columns; 3 padded groups of 12 for 34 columns)
    ("few_r8_d256_g8_p70000_all_chunked", 16, 2, 256, 8, 70000),
    ("few_r6_d256_g8_p50000_all_chunked", 16, 2, 256, 6, 50000),
    ("few_r5_d256_g8_p40000_all_chunked", 16, 2, 256, 5, 40000),
    ("few_r2_d256_g17_p70000_all_chunked_padded", 17, 1, 256, 2, 70000),
    ("few_r6_d256_kv4_p20000_all_chunked", 32, 4, 256, 6, 20000),             # 4 KV heads: 64 CUs each
    # long caches at D 64 and 128: pass 2 in chunks
    ("few_r4_d128_g8_p40000_chunked", 16, 2, 128, 4, 40000),
    ("few_r2_d128_g8_p70000_chunked", 16, 2, 128, 2, 70000),
    ("few_r3_d64_g4_p50000_chunked", 8, 2, 64, 3, 50000),
]


@pytest.mark.parametrize("case", FEW, ids=[c[0] for c in FEW])
def test_few_rows(torch_cuda, case):
    name, h, kvh, d, rows, past = case
    w = W.make(name, heads=h, kv_heads=kvh, head_dim=d, rows=rows, past=past, seed=17)
    print(f"case {name}", flush=True)
    out = run_hsdpa(w)
    ref = oracle.attention(w)
    r = assert_parity(out, ref, w, name)
    print(name, r, flush=True)


@pytest.mark.parametrize("name", ["decode_1k", "prefill_512"])
def test_configs_small(torch_cuda, name):
    w = W.config(name, seed=1)
    print(f"config {name}", flush=True)
    out = run_hsdpa(w)
    ref = oracle.attention(w)
    r = assert_parity(out, ref, w, name)
    print(name, r, flush=True)


@pytest.mark.parametrize("name", ["decode_32k", "prefill_4096_after_8192", "decode_128k_outliers"])
def test_configs_full(torch_cuda, name):
    """The benchmark configurations at full size (the oracle runs on the host's
    AVX-512 BF16 restatement, bit-identical to the scalar emulation)."""
    if not oracle.avx512_available():
        pytest.skip("host lacks AVX-512 BF16: the scalar oracle is too slow at this size")
    w = W.config(name, seed=3)
    print(f"config {name}", flush=True)
    out = run_hsdpa(w)
    ref = oracle.attention(w, "avx512")
    r = assert_parity(out, ref, w, name)
    print(name, r, flush=True)


# Both forms of the score scaling on every kernel family at D 256 (whose
# default 1/16 is a power of two, folded into the exponential's constants): a
# general scale, and a power of two other than the default.
SCALED = [
    # name, heads, kv_heads, head_dim, rows, past, the kernels the call must take
    ("decode_32k", 16, 2, 256, 1, 32767, "decode"),
    ("few_r4", 16, 2, 256, 4, 3000, "few_rows"),
    ("short_16_tiles", 16, 4, 256, 512, 0, "causal_short"),
    ("short_24_tiles", 16, 2, 256, 256, 500, "causal_short"),
    ("short_32_tiles", 16, 2, 256, 1024, 0, "causal_short"),
    ("split", 16, 2, 256, 256, 4000, "causal_split"),
    ("paired", 16, 2, 256, 2200, 1000, "causal_paired"),
    ("causal", 16, 2, 256, 19, 37, "causal"),
]


@pytest.mark.parametrize("scale", [0.0731, 0.125])
@pytest.mark.parametrize("case", SCALED, ids=[c[0] for c in SCALED])
def test_scales(torch_cuda, case, scale):
    name, h, kvh, d, rows, past, kernels = case
    w = W.make(name, heads=h, kv_heads=kvh, head_dim=d, rows=rows, past=past, seed=23, scale=scale)
    plan = hsdpa.Plan(w.heads, w.gqa, w.head_dim, w.capacity)
    assert plan.route(rows, past)["main"] == kernels, plan.route(rows, past)
    print(f"case {name} scale {scale}", flush=True)
    out = run_hsdpa(w, plan)
    ref = oracle.attention(w)
    r = assert_parity(out, ref, w, f"{name} scale {scale}")
    print(name, scale, r, flush=True)


GROUPS = [
    # more than 16 query heads per KV head: the decode kernels take them in 2, 3
    # or 4 equal groups; a group size with no such split (17), or more than 64
    # columns, in padded groups of at most 16 at head dimensions 64, 128 and
    # 256 (the last group's extra columns computed and never stored); the causal
    # kernel serves the row at the other head dimensions
    # name, heads, kv_heads, head_dim, rows, past, the kernels the call must take
    ("decode_g32_d128", 32, 1, 128, 1, 500, "decode"),
    ("decode_g16_d256", 32, 2, 256, 1, 999, "decode"),
    ("decode_g12_d256", 12, 1, 256, 1, 40, "decode"),
    ("decode_g48_d128_three_groups", 48, 1, 128, 1, 3000, "decode"),
    ("decode_g64_d64_four_groups", 128, 2, 64, 1, 20000, "decode"),
    ("decode_g24_d256_two_groups_8_wave", 48, 2, 256, 1, 33000, "decode"),
    ("decode_g20_d256_loop", 40, 2, 256, 1, 70000, "decode"),
    ("decode_g17_d128_padded", 17, 1, 128, 1, 900, "decode"),                 # 2 groups of 9, one padded
    # 3 groups of 12, one padded, all scored in each pass-1 workgroup
    ("decode_g34_d128_padded_all_groups", 34, 1, 128, 1, 40000, "decode"),
    ("decode_g17_d256_padded_2kv_long", 34, 2, 256, 1, 40000, "decode"),
    ("decode_g80_d64_five_groups", 80, 1, 64, 1, 300, "decode"),              # 5 groups of 16
    ("decode_g80_d64_five_groups_long", 80, 1, 64, 1, 6000, "decode"),
    ("decode_g100_d128_padded", 100, 1, 128, 1, 2000, "decode"),              # 7 groups of 15, 5 padded
    ("few_r2_g17_d128_padded", 17, 1, 128, 2, 500, "few_rows"),              # 34 columns: 3 groups of 12
    ("few_r5_g7_d256_padded", 7, 1, 256, 5, 300, "few_rows"),                # 35 columns: 3 groups of 12
    ("decode_g17_d96_through_split_prefill", 17, 1, 96, 1, 900, "causal_split"),
    ("decode_g300_d64_through_split_prefill", 300, 1, 64, 1, 6000, "causal_split"),   # 19 groups: above 16
]


@pytest.mark.parametrize("case", GROUPS, ids=[c[0] for c in GROUPS])
def test_gqa_groups(torch_cuda, case):
    name, h, kvh, d, rows, past, kernels = case
    w = W.make(name, heads=h, kv_heads=kvh, head_dim=d, rows=rows, past=past, seed=5)
    plan = hsdpa.Plan(w.heads, w.gqa, w.head_dim, w.capacity)
    assert plan.route(rows, past)["main"] == kernels, plan.route(rows, past)
    print(f"case {name}", flush=True)
    out = run_hsdpa(w, plan)
    ref = oracle.attention(w)
    r = assert_parity(out, ref, w, name)
    print(name, r, flush=True)


def test_prefill_4096_as_engine_passes(torch_cuda):
    """The 4096-row chunk after 8192 keys as the reference engine sends it to
    the attention node: 16 calls of 256 rows after 8192, 8448, ... keys
    (prefill_pass, src/jit/schedule.rs:290-298), on a plan with max_rows 256.
    The oracle's rows do not depend on how the chunk is cut (it runs passes of
    256 rows itself), so the whole output meets the bar against it."""
    import torch

    if not oracle.avx512_available():
        pytest.skip("host lacks AVX-512 BF16: the scalar oracle is too slow at this size")
    w = W.config("prefill_4096_after_8192", seed=5)
    plan = hsdpa.Plan(w.heads, w.gqa, w.head_dim, w.capacity, max_rows=256)
    dev = torch.device("cuda")
    q = torch.from_numpy(np.ascontiguousarray(w.q).view(np.int16)).to(dev)
    k = torch.from_numpy(np.ascontiguousarray(w.k).view(np.int16)).to(dev)
    v = torch.from_numpy(np.ascontiguousarray(w.v).view(np.int16)).to(dev)
    out = torch.full((w.rows, w.heads, w.head_dim), -1, dtype=torch.int16, device=dev)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    for r0 in range(0, w.rows, 256):
        print(f"pass rows {r0}..{r0 + 255} after {w.past + r0}: {plan.route(256, w.past + r0)['main']}", flush=True)
        plan.attention_raw(q.data_ptr() + 2 * r0 * w.q_row, k.data_ptr(), v.data_ptr(),
                           out.data_ptr() + 2 * r0 * w.out_row, 256, w.past + r0, w.scale, ws.data_ptr(),
                           plan.workspace_bytes, stream)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    r = assert_parity(got, oracle.attention(w, "avx512"), w, "prefill_4096_passes")
    print("prefill_4096_passes", r, flush=True)
