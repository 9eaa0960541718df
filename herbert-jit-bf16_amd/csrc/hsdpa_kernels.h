// hsdpa_kernels.h — launch interface between the C ABI layer and the gfx950
// kernels. Internal to libhsdpa.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <tuple>
#include <type_traits>
#include <utility>

namespace hsdpa {

// Launch `kernel` on stream `s` and return that launch's own status; a HIP
// error left over from an earlier, unrelated call is not reported as this
// one's (hipLaunchKernel returns the launch's result, where
// hipGetLastError would also return a stale one).
template <typename K, typename T, size_t... I>
inline hipError_t launch_held(K kernel, dim3 grid, dim3 block, hipStream_t s, T &held, std::index_sequence<I...>)
{
    void *ptrs[] = {static_cast<void *>(&std::get<I>(held))...};
    return hipLaunchKernel(reinterpret_cast<const void *>(kernel), grid, block, ptrs, 0, s);
}

template <typename... P, typename... A>
inline hipError_t launch(void (*kernel)(P...), dim3 grid, dim3 block, hipStream_t s, A &&...args)
{
    static_assert(sizeof...(P) == sizeof...(A), "one argument per kernel parameter");
    std::tuple<std::decay_t<P>...> held(std::forward<A>(args)...);
    return launch_held(kernel, grid, block, s, held, std::index_sequence_for<P...>{});
}

// Decode: one query row, g query heads per KV head, n visible keys.
struct DecodeArgs {
    const uint16_t *q;      // row 0; head h at q + h*q_head
    const uint16_t *k;      // cache, head kvh at k + kvh*kv_stride
    const uint16_t *v;
    uint16_t *out;          // head h at out + h*head_dim
    float *scores;          // [groups][g][npad] scaled scores (groups = kv_heads * sub)
    float *wgmax;           // [groups][g][nwg_qk] per-workgroup maxima
    float *part_o;          // [groups][nwg_pv][g][head_dim] unnormalised partial outputs
    float *part_l;          // [groups][nwg_pv][g] partial sums of exponentials
    uint64_t n;             // visible keys (past + 1)
    uint64_t npad;          // scores row length, a multiple of the key tile
    uint64_t kv_stride;
    uint64_t q_head;
    int g;                  // columns per group (<= kDecodeMaxGroup)
    int sub;                // groups per KV head: g * sub columns share one (the grid's z)
    int nwg_qk, nwg_pv;     // workgroups per KV head of the two passes
    int keys_qk, keys_pv;   // keys per workgroup of the two passes
    float scale;
    const uint16_t *gate;   // null, or the output gate: head h at gate + h*head_dim
    // A few query rows after a cache (the MR kernels): the columns of KV head
    // y are (row, head) pairs, column c serving row c / G and query head
    // y G + c % G, whose visible keys are [0, past + row].
    int xcd;                // 1: the groups of a key range numbered onto one XCD (several groups)
    int qk_all;             // 1: pass 1 scores all sub groups of a KV head in each workgroup
    int pv_all;             // 1: pass 2 (256-key workgroups) takes all sub groups in each workgroup
    int direct;             // 1: pass 2 writes the outputs itself (decode_direct_ok), no combine
    int rows;               // 1 for a decode step
    int G;                  // query heads per KV head
    int cols;               // columns per KV head that hold a (row, head) pair: rows * G; sub * g may
                            // exceed it by padding (the MR kernels compute a padded column and store nothing)
    uint64_t past;
    uint64_t q_row, out_row, gate_row;
    // The Fused form (the online softmax over blocks of 16 keys): pass 1 also
    // stores each block's maximum, pass 2 the product of its blocks'
    // corrections; unused by the Chained form.
    float *bmax;            // [groups][g][nblk] maxima of the 16-key blocks
    float *part_x;          // [groups][nwg_pv][g] products of a workgroup's corrections
    uint64_t nblk;          // bmax row length: npad / 16
    // A frame call (hsdpa_attention_frame, the FRAME kernels): rows and past
    // are read from device memory at run time, and n, past, keys_qk, keys_pv,
    // nwg_qk and nwg_pv are derived from them on the device (frame_args);
    // unused otherwise.
    const uint64_t *f_rows, *f_past;
    uint32_t *f_status;     // null, or receives the call's hsdpa_status (the combine writes it)
    uint32_t *f_cfg;        // workspace: the step's configuration, stored by pass 1 for pass 2 and the combine
    uint64_t f_cap;         // the plan's KV capacity
    int f_groups;           // kv_heads * sub
    int f_cus;              // compute units the grids were sized for
    int f_loop;             // 1: pass 2 walks a run of keys per workgroup (decode_pv_loop_ok)
    // The softmax sink (SdpaShape::sink), the Chained kernels only: with
    // sink_on, each column's maximum is the larger of its scores' and `sink`,
    // the sum of its exponentials gains P(sink - M) (pass-2 workgroup 0 adds
    // it to its partial sum), and the output is the sum times its reciprocal.
    float sink;
    int sink_on;
};

// Causal prefill: `rows` query rows after `past` cached positions.
struct PrefillArgs {
    const uint16_t *q;
    const uint16_t *k;
    const uint16_t *v;
    uint16_t *out;
    uint64_t rows, past, n; // n = past + rows
    uint64_t q_row, q_head, out_row, kv_stride;
    int gqa;
    float scale;
    const uint16_t *gate;   // null, or the output gate: row r, head h at gate + r*gate_row + h*head_dim
    uint64_t gate_row;
    // The softmax sink, as DecodeArgs': the row maximum is the larger of the
    // scores' and `sink`, the row sum gains P(sink - M), and the output is the
    // sum times its reciprocal.
    float sink;
    int sink_on;
};

// The split form of the causal kernel (see prefill_split_max): workspace for
// its partial maxima, outputs and sums, and what the launcher needs to choose
// the number of splits. units: the most (split, 32-row group, head) cells the
// workspace holds (so and sl: 32 rows of each); smax holds kSplitMaxCells
// floats per unit. No split when units is 0.
struct PrefillSplit {
    float *smax, *so, *sl;
    uint64_t units;
    int cus;
};
constexpr uint64_t kSplitMaxCells = 128;

// Constants of the kernels the host needs to size grids and workspaces.
constexpr int kKeyTile = 32;          // keys per MFMA key block
constexpr int kDecodeKeysQK = 128;    // keys per decode pass-1 workgroup (4 waves x 1 tile)
constexpr int kDecodeKeysPV = 256;    // keys per decode pass-2 workgroup (8 waves x 1 tile; 4 x 1 on short caches)
constexpr int kDecodeMaxGroup = 16;   // query heads per KV head the decode kernels take
constexpr int kSplitUnits = 2048;     // (split, 32-row group, head) cells of the split prefill's workspace

// KV append: token-major block rows into the head-major cache.
struct KvAppendArgs {
    uint16_t *keys, *values;
    const uint16_t *in_keys, *in_values;
    uint64_t rows, past, heads, head_dim, stride;
};

// Head RMS norm + RoPE, one wave per (row, head).
struct NormRopeArgs {
    uint16_t *data;
    const uint16_t *w, *cos, *sin;
    uint64_t rows, past, row_stride, head_stride, table_row;
    int heads, dim, rotary, plus_one;
    float eps;
};

// Output gate: attn <- attn / (1 + exp(min(-gate, 88))).
struct GateArgs {
    uint16_t *attn;
    const uint16_t *gate;
    uint64_t rows, width, attn_row, gate_row;
};

// The element work of a layer before its attention, one wave per (row, head):
// query heads are normalised and rotated in place; KV heads have k normalised
// and rotated in place and copied, with the v row, into the cache at position
// past + row.
struct LayerPrepArgs {
    uint16_t *q, *k;
    const uint16_t *v;
    uint16_t *keys, *values;
    const uint16_t *q_norm, *k_norm, *cos, *sin;
    uint64_t rows, past, q_row, q_head, kv_row, kv_stride, table_row;
    int heads, kv_heads, dim, rotary, plus_one;
    float eps;
};

// Head dimensions the kernels take: multiples of 32 from 32 to 512 (the
// reference's SdpaShape::check, ir.rs:130-162).
bool head_dim_supported(int d);

// Decode configurations a head dimension allows. Pass 1 loops over several key
// tiles per wave up to D = 256 (above, one tile's registers are the budget);
// pass 2 takes 8 waves (256 keys) only where their V tiles fit the LDS (D <=
// 256) and the waves split the D/16 dimension blocks evenly or take whole ones.
inline bool decode_loop_ok(int d) { return d <= 256; }

// The decode kernels take the g query heads of a KV head in `sub` equal groups
// of at most kDecodeMaxGroup; each group streams the KV head's cache, so up to
// 4 of them (a larger g, or one without such a divisor, runs on the causal
// kernel). Returns sub, or 0.
inline int decode_groups(int g)
{
    for (int sub = 1; sub <= 4; sub++)
        if (g % sub == 0 && g / sub <= kDecodeMaxGroup) return sub;
    return 0;
}
// Columns that no such split fits (a group size without a divisor up to 4
// into groups of at most 16, more than 64 columns) run on the kernels that map
// each column to a (row, head) pair, the few-rows instantiations: ceil(cols /
// 16) groups of ceil(cols / sub) columns, the last one padded, up to
// kDecodePadGroups groups (each streams the KV head's cache; where the causal
// kernel would compute 32-row tiles for one row). Returns sub, or 0.
constexpr int kDecodePadGroups = 16;
inline int decode_groups_pad(int cols)
{
    const int sub = (cols + kDecodeMaxGroup - 1) / kDecodeMaxGroup;
    return cols > 0 && sub <= kDecodePadGroups ? sub : 0;
}
// columns per group for `cols` columns in `sub` groups
inline int decode_group_cols(int cols, int sub) { return (cols + sub - 1) / sub; }
inline bool decode_wide_ok(int d) { return d <= 256 && (d / 16 >= 8 || 8 % (d / 16) == 0); }
// A few rows after a cache run on the decode kernels (one column per (row,
// head) pair, up to 8 groups of 16 columns per KV head) for the tuned head
// dimensions; the causal kernel computes 32-row tiles, most of them wasted on
// so few rows.
constexpr int kDecodeMaxRows = 16;
constexpr int kDecodeMaxCols = 8 * kDecodeMaxGroup;     // columns per KV head
// pass 1 scores up to this many groups of a KV head in one workgroup
constexpr int kDecodeMaxSub = 8;
// pass 2 walks a run of keys for up to this many groups of a KV head in one
// workgroup (their accumulators stay in registers over the run)
constexpr int kDecodeLoopMaxSub = 4;
// Past 8 rows or 64 columns (up to 16 rows, 128 columns) the few-rows decode
// beats the split causal kernel only while its groups times the visible keys
// stay small: 16/2 heads at D = 256, 9 and 16 rows after 32K 110 -> 49 and 114
// -> 66 us, 9 rows after 128K (5 groups) 204 -> 162 us, but 16 rows after 128K
// (8 groups) 218 -> 235 us; 32/4 heads at D = 128, 9 and 16 rows after 8K 57
// -> 43 and 60 -> 40 us, but 9 rows after 32K 84 -> 102 us.
inline bool decode_wide_ok_n(int d, int rows, int cols, int sub, uint64_t n)
{
    if (rows <= 8 && cols <= 4 * kDecodeMaxGroup) return true;
    const uint64_t budget = d == 256 ? uint64_t{768} << 10 : uint64_t{64} << 10;
    return static_cast<uint64_t>(sub) * n <= budget;
}
// Whether pass 1 of a Chained decode call on the tuned head dimensions takes
// all of a KV head's groups in each workgroup (its grid then has no group
// axis): 2 to kDecodeMaxSub groups, where a tile per wave of these workgroups
// (kv_wgs = kv_heads x the 128-key blocks) would still take more than one
// round of the compute units, so that every wave scores at least two tiles.
// On 2 KV heads at head_dim 256 from 24K keys on (24K: 8 rows 48.0 -> 42.7 us,
// 32 query heads per KV head 31.6 -> 31.1 us; 32K: 8 rows 59.6 -> 53.7 us);
// below it, one workgroup per group fills the compute units better (8K: 8 rows
// 21.9 us per group, 24.1 all groups; 16K: 2 groups of 16 heads 20.3 and 21.9).
inline bool decode_qk_groups(int sub, uint64_t kv_wgs, uint64_t cus)
{
    return sub >= 2 && sub <= kDecodeMaxSub && kv_wgs > cus;
}
inline bool decode_rows_ok(int d) { return d == 64 || d == 128 || d == 256; }
// Short caches: pass 2 over every key in each workgroup, which writes the
// outputs itself (no combine launch): one group of at most 16 columns per KV
// head (the query heads of one row, or the (row, head) columns of a few rows;
// under the Fused form one row of at most 8 heads), at most kDirectKeys
// visible keys, the tuned head dimensions. Past 8 columns (two P column
// blocks) only while columns x keys <= kDirectWideWork: each workgroup
// computes every column's exponentials (16 heads at 256 keys 11.97 -> 11.36
// us, 3 rows of 4 heads after 100 keys 12.39 -> 11.17; 16 heads at 1024 keys
// 12.86 -> 13.82, 4 rows of 4 heads after 500 keys at D = 128 11.65 -> 12.34).
constexpr int kDirectKeys = 1024;
constexpr uint64_t kDirectWideWork = 4096;
// dimensions per workgroup of that pass: 16, one MFMA block (twice the
// workgroups of 32-dimension slices, 1024 keys on 8/2 heads at D = 256 10.96
// -> 9.95 us)
constexpr int kDirectSlice = 16;
inline bool decode_direct_ok(int d, int rows, int sub, int g, uint64_t n, bool fused)
{
    return decode_rows_ok(d) && sub == 1 && n <= static_cast<uint64_t>(kDirectKeys) &&
           (fused ? rows == 1 && g <= 8 : g <= 8 || static_cast<uint64_t>(g) * n <= kDirectWideWork);
}

// Pass 2 in chunks (one round of workgroups over a long cache) is built for
// the tuned head dimensions; under the Fused form at D = 256 for one row in
// groups of up to 8 columns (with 16 its running maxima and corrections and
// the P columns' operands no longer fit beside the next chunk's V tile).
inline bool decode_pv_loop_ok(int d, int g, int rows, bool fused)
{
    return d == 64 || d == 128 || (d == 256 && (!fused || (g <= 8 && rows == 1)));
}
// Several rows at D = 256 in 2 or more groups: pass 2 over all the groups of
// a KV head per workgroup loads each V tile once for all of them; chunked
// runs per group stream V once per group, but in one round of workgroups.
// The runs go with at most 4 groups where the all-group form would take more
// than one round of 256-key workgroups (kv_chunks = kv_heads x ceil(n/256)):
// 16/2 heads at D = 256, 4 rows after 64K and 128K 58.7 -> 55.3 and 105.6 ->
// 90.9 us, 8 rows after 128K 147.9 -> 139.8; but 8 rows after 32K (one round)
// 46.2 -> 49.0 and 16 rows (8 groups) after 64K 126.6 -> 131.4.
inline bool decode_pv_loop_rows_ok(int d, int rows, int sub, uint64_t kv_chunks, uint64_t cus)
{
    return d != 256 || rows == 1 || sub == 1 || (sub <= 4 && kv_chunks > cus);
}
// Several rows at D = 256 in 3 to kDecodeLoopMaxSub groups where pass 1 takes
// every group of a KV head in one workgroup and 256-key pass-2 workgroups
// would take more than one round: one round of workgroups that each walk a
// run of keys for all the groups (decode_pv_all_loop; each V tile loaded once
// for all the groups, where a run per group streams V once per group). 8 rows
// of 8 heads (4 groups) after 64K / 128K: 73.8 / 130.9 -> 70.6 / 120.5 us;
// with 2 groups the runs per group were as fast (4 rows: 50.6 / 87.5 against
// 51.6 / 88.7 us).
inline bool decode_pv_all_loop_ok(int d, int rows, int sub, bool qk_all, uint64_t kv_chunks, uint64_t cus)
{
    return d == 256 && rows > 1 && sub >= 3 && sub <= kDecodeLoopMaxSub && qk_all && kv_chunks > cus;
}
hipError_t launch_layer_prep(const LayerPrepArgs &a, hipStream_t s);
hipError_t launch_norm_rope(const NormRopeArgs &a, hipStream_t s);
hipError_t launch_gate(const GateArgs &a, hipStream_t s);
hipError_t launch_kv_append(const KvAppendArgs &a, bool vec, hipStream_t s);
hipError_t launch_decode(const DecodeArgs &a, int head_dim, int kv_heads, hipStream_t s);
// A frame call's decode passes (hsdpa_frame.hip): one row, equal groups, the
// tuned head dimensions; the grids sized for any past below the capacity.
hipError_t launch_decode_frame(const DecodeArgs &a, int head_dim, int kv_heads, bool fused, hipStream_t s);
hipError_t launch_prefill(const PrefillArgs &a, int head_dim, int heads, const PrefillSplit &ps, hipStream_t s);
// the key splits launch_prefill would choose (1: the one-workgroup kernel)
int prefill_split_count(const PrefillArgs &a, int head_dim, int heads, const PrefillSplit &ps);
struct PairRows;
// the rows with partials of the paired form launch_prefill would choose
// (srows 0: not paired)
PairRows prefill_pair_rows(const PrefillArgs &a, int head_dim, int heads, const PrefillSplit &ps);
// the head dimensions other than 64, 128 and 256 (hsdpa_attn_more.hip)
hipError_t launch_decode_more(const DecodeArgs &a, int head_dim, int kv_heads, hipStream_t s);
// the Fused form of the decode passes, head dimensions 32 to 256 (hsdpa_fused.hip)
hipError_t launch_decode_fused(const DecodeArgs &a, int head_dim, int kv_heads, hipStream_t s);
// The causal prefill of a short chunk with the keys split among the waves of
// each 32-row block's workgroup (hsdpa_prefill_short.hip), head dimensions 64,
// 128 and 256: for chunks that would leave compute units idle, while each row
// block sees at most kShortMaxTiles key tiles (beyond, the split kernels
// spread the keys over more workgroups).
constexpr int kShortWaves = 4;
constexpr int kShortMaxTiles = 32;
// at head dimensions 128 and 256 O is accumulated by dimensions (prefill_kd), at
// 64 by keys (prefill_ks)
inline bool prefill_short_ok(int d) { return d == 64 || d == 128 || d == 256; }
hipError_t launch_prefill_short(const PrefillArgs &a, int head_dim, int heads, hipStream_t s);
// the current device's copy of the static scratch of hsdpa_attention_static
// (hsdpa_static.hip)
hipError_t static_scratch(void **ptr);
// the pass-2 workgroups a Fused combine can scan per head (its LDS)
constexpr int kFusedMaxSeg = 512;
hipError_t launch_prefill_more(const PrefillArgs &a, int head_dim, int heads, const PrefillSplit &ps, hipStream_t s);
// the causal prefill with the softmax sink, every head dimension (hsdpa_sink.hip):
// one query head per workgroup, as the grid of prefill_hpw for a sink call
hipError_t launch_prefill_sink(const PrefillArgs &a, int head_dim, int heads, const PrefillSplit &ps, hipStream_t s);

// Splits for a causal call whose one-workgroup grid has `wgs` workgroups: enough
// to fill the compute units once, at least 4 tiles of the longest row group
// each, within the workspace; 1 when the grid fills half the units already or
// the rows see fewer than 8 tiles.
inline int prefill_splits(const PrefillArgs &a, uint64_t wgs, int heads, const PrefillSplit &ps)
{
    if (ps.units == 0 || ps.cus <= 0 || wgs * 2 > static_cast<uint64_t>(ps.cus)) return 1;
    const uint64_t ntiles = (a.past + a.rows + kKeyTile - 1) / kKeyTile;
    if (ntiles < 8) return 1;
    uint64_t s = static_cast<uint64_t>(ps.cus) / wgs;
    if (s > ntiles / 4) s = ntiles / 4;
    const uint64_t cells = (a.rows + 31) / 32 * static_cast<uint64_t>(heads);
    if (s > ps.units / cells) s = ps.units / cells;
    return s >= 2 ? static_cast<int>(s) : 1;
}

// The paired form of the causal kernel, for a grid of R row groups (rpw rows
// each) x head groups that the compute units hold in one round: row group r
// sees causal_tiles(r) key tiles, more the later it lies, and the round lasts
// as long as its longest workgroup. Row groups i and j = R - 1 - i (i < j) are
// paired: j's last h = (T_j - T_i) / 2 tiles go to i's workgroup, which walks
// them after its own row group, so that the two workgroups walk T_i + h and
// T_j - h tiles. The split row groups (the last ones) pass partial outputs to
// a combine: slot 0 the head, slot 1 the tail.
constexpr uint64_t kPairMinTiles = 4;

__host__ __device__ inline uint64_t causal_tiles(uint64_t past, uint64_t rows, uint64_t r, uint64_t rpw)
{
    const uint64_t e = (r + 1) * rpw < rows ? (r + 1) * rpw : rows;
    return (past + e + kKeyTile - 1) / kKeyTile;
}

__host__ __device__ inline uint64_t pair_share(uint64_t ti, uint64_t tj)
{
    const uint64_t h = (tj - ti) / 2;
    return h >= kPairMinTiles ? h : 0;
}

// The rows with partials of a paired call: [r0, r0 + srows); srows 0 when the
// call is not paired. Paired when one round of the grid holds it, its longest
// row group sees at least kPairMinLongest tiles (below, the two extra launches
// and the second range's first loads cost more than the balance saves: 1000
// rows at D 64, 32 tiles, 56.7 -> 60.9 us), pairing shortens its longest
// workgroup by at least an eighth, and the partials fit the workspace.
constexpr uint64_t kPairMinLongest = 64;
struct PairRows {
    uint64_t r0, srows;
};

inline PairRows prefill_pairs(const PrefillArgs &a, uint64_t R, uint64_t wgs, uint64_t rpw, int heads,
                              const PrefillSplit &ps)
{
    const PairRows none{0, 0};
    if (ps.units == 0 || ps.cus <= 0 || R < 2 || wgs > static_cast<uint64_t>(ps.cus)) return none;
    uint64_t longest = R % 2 ? causal_tiles(a.past, a.rows, R / 2, rpw) : 0, split = 0;
    for (uint64_t i = 0; i < R - 1 - i; i++) {
        const uint64_t ti = causal_tiles(a.past, a.rows, i, rpw), tj = causal_tiles(a.past, a.rows, R - 1 - i, rpw);
        const uint64_t h = pair_share(ti, tj);
        const uint64_t w = ti + h > tj - h ? ti + h : tj - h;
        if (w > longest) longest = w;
        if (h) split = i + 1;
    }
    const uint64_t tmax = causal_tiles(a.past, a.rows, R - 1, rpw);
    if (split == 0 || tmax < kPairMinLongest || 8 * longest > 7 * tmax) return none;
    const uint64_t r0 = (R - split) * rpw, srows = a.rows - r0;
    const uint64_t h = static_cast<uint64_t>(heads);
    if (2 * srows * h > ps.units * 32 || 2 * a.rows * h > ps.units * kSplitMaxCells) return none;
    return PairRows{r0, srows};
}

}  // namespace hsdpa
