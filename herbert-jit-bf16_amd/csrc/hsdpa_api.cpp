// hsdpa_api.cpp — the C ABI of include/hsdpa.h: geometry validation at plan
// time, call validation on the host before any launch, workspace layout and
// the choice between the decode and the prefill kernels.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <new>

#include "hsdpa.h"
#include "hsdpa_kernels.h"

struct hsdpa_plan {
    hsdpa_spec spec;
    uint64_t kv_heads;
    uint32_t form;            // the effective form: Fused only up to head_dim 256
    int cus;                  // compute units the grids are chosen (and the workspace sized) for
    uint64_t max_rows;        // spec.max_rows, or kv_capacity when 0
    // decode workspace (floats): scores, per-workgroup maxima, partials; with
    // the Fused form also the 16-key block maxima and the partials' products
    uint64_t dec_npad;        // scores row length for a full cache
    uint64_t dec_nwg_qk;      // pass-1 workgroups per group, at most
    uint64_t dec_cols;        // columns per KV head: query heads, or (row, head) pairs (0: no decode)
    uint64_t dec_part;        // (pass-2 workgroup, column) partials per KV head, at most
    uint64_t off_scores, off_wgmax, off_part_o, off_part_l, off_bmax, off_part_x, off_fcfg, dec_bytes;
    // split causal workspace (floats), after the decode's: partial row maxima,
    // outputs and sums of split_units (split, 32-row group, head) cells
    uint64_t split_units;
    uint64_t off_smax, off_so, off_sl;
    uint64_t ws_bytes;
};

namespace {

constexpr uint64_t kAlign = 256;
uint64_t align_up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }
bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// SdpaShape::check (src/jit/ir.rs:130-148) and tile_selector's geometry
// checks (src/jit/target/x86/execution/attention.rs:61-98), plus the cache
// geometry of KvSpec::validate (src/jit/execution/abi.rs:75-103).
hsdpa_status check_spec(const hsdpa_spec &s)
{
    if (s.heads == 0 || s.gqa == 0 || s.head_dim == 0) return HSDPA_ERR_EMPTY;
    if (s.head_dim % 32 != 0 || s.head_dim > 512) return HSDPA_ERR_HEAD_DIM;
    if (!hsdpa::head_dim_supported(static_cast<int>(s.head_dim))) return HSDPA_ERR_HEAD_DIM;
    if (s.heads % s.gqa != 0) return HSDPA_ERR_GQA;
    if (s.sink > 1) return HSDPA_ERR_SINK_UNSUPPORTED;         // SdpaShape::sink is a flag
    const uint64_t lim = static_cast<uint64_t>(INT32_MAX) / 2;
    if (s.heads > lim || s.gqa > lim || s.q_row > lim || s.q_head > lim || s.out_row > lim)
        return HSDPA_ERR_STRIDE;
    if (s.q_head < s.head_dim || s.heads * s.q_head > s.q_row) return HSDPA_ERR_STRIDE;
    if (s.heads * s.head_dim > s.out_row) return HSDPA_ERR_STRIDE;
    if (s.kv_capacity == 0) return HSDPA_ERR_CAPACITY;
    if (s.kv_capacity > (static_cast<uint64_t>(1) << 40) / s.head_dim) return HSDPA_ERR_CAPACITY;
    if (s.kv_stride < s.kv_capacity * s.head_dim) return HSDPA_ERR_STRIDE;
    if (s.form > HSDPA_FORM_FUSED || s.reserved != 0) return HSDPA_ERR_FORM;
    if (s.max_rows > s.kv_capacity) return HSDPA_ERR_CAPACITY;
    // the kernels move 16-byte vectors
    if (s.q_row % 8 || s.q_head % 8 || s.out_row % 8 || s.kv_stride % 8) return HSDPA_ERR_ALIGNMENT;
    return HSDPA_OK;
}

// One architecture check per device, cached with its compute-unit count.
std::mutex g_dev_mu;
int g_dev_state[64];  // 0 unknown, 1 gfx950, 2 other
int g_dev_cus[64];

hsdpa_status check_device(int *cus = nullptr)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return HSDPA_ERR_NO_DEVICE;
    if (dev < 0 || dev >= 64) return HSDPA_ERR_NO_DEVICE;
    std::lock_guard<std::mutex> lk(g_dev_mu);
    if (g_dev_state[dev] == 0) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, dev) != hipSuccess) return HSDPA_ERR_NO_DEVICE;
        g_dev_state[dev] = std::strncmp(p.gcnArchName, "gfx950", 6) == 0 ? 1 : 2;
        g_dev_cus[dev] = p.multiProcessorCount;
    }
    if (cus) *cus = g_dev_cus[dev];
    return g_dev_state[dev] == 1 ? HSDPA_OK : HSDPA_ERR_NO_DEVICE;
}

// KvSpec::validate (src/jit/execution/abi.rs:74-103) and the x86 refusal of
// the R16 copies (src/jit/target/x86/execution/kv.rs:17-21).
hsdpa_status check_kv_spec(const hsdpa_kv_spec &s)
{
    if (s.heads == 0 || s.head_dim == 0 || s.max_batch == 0) return HSDPA_ERR_EMPTY;
    if (s.capacity < s.max_batch) return HSDPA_ERR_CAPACITY;
    const uint64_t i32 = static_cast<uint64_t>(INT32_MAX);
    if (s.stride > i32 / 2) return HSDPA_ERR_STRIDE;
    if (s.capacity > s.stride / s.head_dim || s.capacity * s.head_dim > s.stride) return HSDPA_ERR_STRIDE;
    if (s.heads > i32 || s.heads * s.head_dim > i32 / 2) return HSDPA_ERR_STRIDE;
    if (s.r16 != 0) return HSDPA_ERR_LAYOUT;
    return HSDPA_OK;
}

}  // namespace

extern "C" {

// norm_rope's checks (transforms.rs:38-40), the element kernels' shapes (a
// multiple of 32 elements, emit_elem.rs spec.check) and the binding's strides.
static hsdpa_status check_norm_rope(const hsdpa_norm_rope_spec &s)
{
    if (s.heads == 0 || s.head_dim == 0) return HSDPA_ERR_EMPTY;
    if (s.head_dim % 32 != 0 || s.head_dim > 512) return HSDPA_ERR_HEAD_DIM;
    if (s.rotary_dims % 32 != 0 || s.rotary_dims > s.head_dim) return HSDPA_ERR_HEAD_DIM;
    const uint64_t i32 = static_cast<uint64_t>(INT32_MAX);
    if (s.heads > i32 || s.head_stride > i32 / 2 || s.row_stride > i32 / 2) return HSDPA_ERR_STRIDE;
    if (s.head_stride < s.head_dim || s.heads * s.head_stride > s.row_stride) return HSDPA_ERR_STRIDE;
    if (s.rotary_dims && s.table_row < s.rotary_dims / 2) return HSDPA_ERR_STRIDE;
    return HSDPA_OK;
}

hsdpa_status hsdpa_head_norm_rope(const hsdpa_norm_rope_spec *spec, const hsdpa_norm_rope_call *call, void *stream)
{
    if (!spec || !call) return HSDPA_ERR_NULL;
    const hsdpa_status st = check_norm_rope(*spec);
    if (st != HSDPA_OK) return st;
    if (call->rows == 0) return HSDPA_OK;
    if (call->rows > (1u << 31) - 1) return HSDPA_ERR_CAPACITY;
    if (spec->rotary_dims && (call->past > spec->positions || call->rows > spec->positions - call->past))
        return HSDPA_ERR_CAPACITY;
    if (!call->data || !call->weight || (spec->rotary_dims && (!call->cos || !call->sin))) return HSDPA_ERR_NULL;
    const hsdpa_status dv = check_device();
    if (dv != HSDPA_OK) return dv;
    hsdpa::NormRopeArgs a;
    a.data = call->data;
    a.w = call->weight;
    a.cos = call->cos;
    a.sin = call->sin;
    a.rows = call->rows;
    a.past = call->past;
    a.row_stride = spec->row_stride;
    a.head_stride = spec->head_stride;
    a.table_row = spec->table_row;
    a.heads = static_cast<int>(spec->heads);
    a.dim = static_cast<int>(spec->head_dim);
    a.rotary = static_cast<int>(spec->rotary_dims);
    a.plus_one = spec->plus_one ? 1 : 0;
    a.eps = call->eps;
    if (hsdpa::launch_norm_rope(a, static_cast<hipStream_t>(stream)) != hipSuccess) return HSDPA_ERR_HIP;
    return HSDPA_OK;
}

hsdpa_status hsdpa_output_gate(const hsdpa_gate_spec *spec, const hsdpa_gate_call *call, void *stream)
{
    if (!spec || !call) return HSDPA_ERR_NULL;
    if (spec->width == 0) return HSDPA_ERR_EMPTY;
    if (spec->attn_row < spec->width || spec->gate_row < spec->width) return HSDPA_ERR_STRIDE;
    if (call->rows == 0) return HSDPA_OK;
    if (!call->attn || !call->gate) return HSDPA_ERR_NULL;
    const hsdpa_status dv = check_device();
    if (dv != HSDPA_OK) return dv;
    hsdpa::GateArgs a;
    a.attn = call->attn;
    a.gate = call->gate;
    a.rows = call->rows;
    a.width = spec->width;
    a.attn_row = spec->attn_row;
    a.gate_row = spec->gate_row;
    if (hsdpa::launch_gate(a, static_cast<hipStream_t>(stream)) != hipSuccess) return HSDPA_ERR_HIP;
    return HSDPA_OK;
}

// One layer's KV between a snapshot block (host: K[heads][snap_positions][head_dim]
// then V, model.rs:675-697) and the live cache (device: head h at h * stride):
// the copy loops of Runner::snapshot_take (model.rs:749-766) and
// Runner::restore_from (model.rs:820-851), keys then values, the leading
// `positions` of every head, as one 2-D copy per half. restore_from skips rows
// the live cache already holds (first_different_row, model.rs:861-865); copying
// them again leaves the same bytes, so the cache ends identical.
static hsdpa_status kv_snapshot_check(const hsdpa_kv_spec *spec, const void *snapshot_layer, const void *keys,
                                      const void *values, uint64_t snap_positions, uint64_t positions,
                                      bool *nothing)
{
    *nothing = false;
    if (!spec) return HSDPA_ERR_NULL;
    const hsdpa_status st = check_kv_spec(*spec);
    if (st != HSDPA_OK) return st;
    if (positions > snap_positions || positions > spec->capacity) return HSDPA_ERR_CAPACITY;
    // A layer's block is one u16 run of the format: 64 GiB at most (MAX_BLOCK_SNAPSHOT, model.rs:105-108)
    if (snap_positions > (uint64_t{64} << 30) / (4 * spec->heads * spec->head_dim)) return HSDPA_ERR_CAPACITY;
    if (positions == 0) {
        *nothing = true;
        return HSDPA_OK;
    }
    if (!snapshot_layer || !keys || !values) return HSDPA_ERR_NULL;
    return check_device();
}

static hsdpa_status kv_snapshot_copy(const hsdpa_kv_spec *spec, bool to_device, uint16_t *snapshot_layer,
                                     uint16_t *keys, uint16_t *values, uint64_t snap_positions, uint64_t positions,
                                     void *stream)
{
    const uint64_t snap_pitch = snap_positions * spec->head_dim * 2, live_pitch = spec->stride * 2;
    const uint64_t width = positions * spec->head_dim * 2;
    uint16_t *const snap[2] = {snapshot_layer, snapshot_layer + spec->heads * snap_positions * spec->head_dim};
    uint16_t *const live[2] = {keys, values};
    const hipStream_t s = static_cast<hipStream_t>(stream);
    for (int half = 0; half < 2; half++) {
        const hipError_t e =
            to_device
                ? hipMemcpy2DAsync(live[half], live_pitch, snap[half], snap_pitch, width, spec->heads,
                                   hipMemcpyHostToDevice, s)
                : hipMemcpy2DAsync(snap[half], snap_pitch, live[half], live_pitch, width, spec->heads,
                                   hipMemcpyDeviceToHost, s);
        if (e != hipSuccess) return HSDPA_ERR_HIP;
    }
    return HSDPA_OK;
}

hsdpa_status hsdpa_kv_restore(const hsdpa_kv_spec *spec, const uint16_t *snapshot_layer, uint64_t snap_positions,
                              uint16_t *keys, uint16_t *values, uint64_t positions, void *stream)
{
    bool nothing;
    const hsdpa_status st = kv_snapshot_check(spec, snapshot_layer, keys, values, snap_positions, positions, &nothing);
    if (st != HSDPA_OK || nothing) return st;
    return kv_snapshot_copy(spec, true, const_cast<uint16_t *>(snapshot_layer), keys, values, snap_positions,
                            positions, stream);
}

hsdpa_status hsdpa_kv_take(const hsdpa_kv_spec *spec, const uint16_t *keys, const uint16_t *values,
                           uint16_t *snapshot_layer, uint64_t snap_positions, uint64_t positions, void *stream)
{
    bool nothing;
    const hsdpa_status st = kv_snapshot_check(spec, snapshot_layer, keys, values, snap_positions, positions, &nothing);
    if (st != HSDPA_OK || nothing) return st;
    return kv_snapshot_copy(spec, false, snapshot_layer, const_cast<uint16_t *>(keys), const_cast<uint16_t *>(values),
                            snap_positions, positions, stream);
}

hsdpa_status hsdpa_kv_check(const hsdpa_kv_spec *spec)
{
    if (!spec) return HSDPA_ERR_NULL;
    return check_kv_spec(*spec);
}

hsdpa_status hsdpa_kv_append(const hsdpa_kv_spec *spec, const hsdpa_kv_call *call, void *stream)
{
    if (!spec || !call) return HSDPA_ERR_NULL;
    const hsdpa_status st = check_kv_spec(*spec);
    if (st != HSDPA_OK) return st;
    if (call->rows == 0) return HSDPA_OK;                        // kv.rs:33-34
    if (call->rows > spec->max_batch) return HSDPA_ERR_BATCH;
    if (call->past > spec->capacity || call->rows > spec->capacity - call->past) return HSDPA_ERR_CAPACITY;
    if (!call->keys || !call->values || !call->input_keys || !call->input_values) return HSDPA_ERR_NULL;
    const hsdpa_status dv = check_device();
    if (dv != HSDPA_OK) return dv;
    hsdpa::KvAppendArgs a;
    a.keys = call->keys;
    a.values = call->values;
    a.in_keys = call->input_keys;
    a.in_values = call->input_values;
    a.rows = call->rows;
    a.past = call->past;
    a.heads = spec->heads;
    a.head_dim = spec->head_dim;
    a.stride = spec->stride;
    const bool vec = spec->head_dim % 8 == 0 && spec->stride % 8 == 0 && aligned16(call->keys) &&
                     aligned16(call->values) && aligned16(call->input_keys) && aligned16(call->input_values);
    if (hsdpa::launch_kv_append(a, vec, static_cast<hipStream_t>(stream)) != hipSuccess) return HSDPA_ERR_HIP;
    return HSDPA_OK;
}


// ---- decode configuration --------------------------------------------------

namespace {

// How the decode passes cover a call: `sub` groups of `g` columns per KV
// head, keys per workgroup and workgroups per group of each pass.
struct DecodeCfg {
    int sub, g, keys_qk, keys_pv, nwg_qk, nwg_pv, xcd, qk_all, pv_all, direct;
};

// Whether `rows` rows over n visible keys run on the decode kernels: one row
// whose g query heads split into at most 4 groups of at most 16, or up to 16
// rows as (row, head) columns at head dimensions 64, 128 and 256 within the
// plan's columns (past 8 rows or 64 columns, within decode_wide_ok_n); at
// those head dimensions, columns no equal split fits take padded groups
// (decode_groups_pad). n = 0: any n (the most a call of `rows` rows may take).
int decode_sub(const hsdpa_plan *p, uint64_t rows, uint64_t n)
{
    const uint64_t cols = rows * p->spec.gqa;
    const int d = static_cast<int>(p->spec.head_dim);
    const int even = cols <= static_cast<uint64_t>(4 * hsdpa::kDecodeMaxGroup) ? hsdpa::decode_groups(static_cast<int>(cols)) : 0;
    if (rows == 1 && even) return even;
    if (rows > hsdpa::kDecodeMaxRows || !hsdpa::decode_rows_ok(d) || cols > p->dec_cols) return 0;
    const int sub = even ? even : hsdpa::decode_groups_pad(static_cast<int>(cols));
    if (sub && n && !hsdpa::decode_wide_ok_n(d, static_cast<int>(rows), static_cast<int>(cols), sub, n)) return 0;
    return sub;
}

// Query heads per KV head beyond which a Fused plan is refused: its rows
// would need more padded groups than one grid's z dimension holds.
constexpr uint64_t kFusedMaxGqa = uint64_t{4096} * hsdpa::kDecodeMaxGroup;

// The groups of one row under the Fused form (head_dim <= 256). The reference
// serves such a row with its Fused head whatever its shape
// (src/jit/sdpa.rs:491-510), so it always takes the decode kernels, which
// compute the Fused weights: where decode_sub would send it to the causal
// kernels (Chained numerics) -- a group size with no equal split at the head
// dimensions other than 64, 128 and 256, more than 16 padded groups, or padded
// groups over a cache longer than decode_wide_ok_n allows -- it takes
// ceil(g / 16) padded groups on the kernels that map each column to its
// (row, head) pair. n = 0: any n.
int fused_row_sub(const hsdpa_plan *p, uint64_t n)
{
    const int sub = decode_sub(p, 1, n);
    if (sub) return sub;
    return static_cast<int>((p->spec.gqa + hsdpa::kDecodeMaxGroup - 1) / hsdpa::kDecodeMaxGroup);
}

// The decode passes' grids for `rows` rows over n visible keys (decode_sub
// already > 0).
DecodeCfg decode_cfg(const hsdpa_plan *p, uint64_t rows, uint64_t n, int sub, bool fused)
{
    DecodeCfg c{};
    const int d = static_cast<int>(p->spec.head_dim);
    const uint64_t cols = rows * p->spec.gqa;
    c.sub = sub;
    c.g = hsdpa::decode_group_cols(static_cast<int>(cols), sub);
    const uint64_t groups = p->kv_heads * static_cast<uint64_t>(sub);
    const uint64_t nqk1 = (n + hsdpa::kDecodeKeysQK - 1) / hsdpa::kDecodeKeysQK;
    const uint64_t cu1 = static_cast<uint64_t>(p->cus);
    // pass 1 of the Chained form on the tuned head dimensions may score all of
    // a KV head's groups in each workgroup: its grid then has kv_heads rows of
    // workgroups, not one per group, and two tiles per wave at least (below)
    c.qk_all = !fused && hsdpa::decode_rows_ok(d) && hsdpa::decode_loop_ok(d) &&
                       hsdpa::decode_qk_groups(sub, p->kv_heads * nqk1, cu1)
                   ? 1
                   : 0;
    const uint64_t groups_qk = c.qk_all ? p->kv_heads : groups;
    // pass 1: a tile per wave, or several in turn (the next one in flight)
    // once one tile per wave would need more than one workgroup per compute
    // unit: at least two, and as many as one round of two workgroups per
    // compute unit needs; this bounds the maxima pass 2 reads. Two tiles per
    // wave from one workgroup per compute unit on measured 0.3-0.5 us faster
    // than one tile per wave between 20K and 32K keys at 2 KV heads, and the
    // same elsewhere. From there up to twice as many tiles per wave, the
    // count that leaves the fewest tiles on the busiest compute unit (the
    // looped kernel runs one workgroup per CU at a time; the smaller count on
    // a tie): a partial last round costs a whole one (40K keys: 3 tiles in
    // one round, 27.8 us, against 2 tiles in two rounds, 29.2 us).
    // (all groups per workgroup: their Q columns fill the LDS beside the K tiles,
    // one workgroup per compute unit)
    const uint64_t per_cu = c.qk_all ? 1 : 2;
    const uint64_t rounds = (groups_qk * nqk1 + per_cu * cu1 - 1) / (per_cu * cu1);
    uint64_t rq = !hsdpa::decode_loop_ok(d) ? 1 : groups_qk * nqk1 > cu1 && rounds < 2 ? 2 : rounds;
    if (rq > 1) {
        uint64_t best = rq, cost = ~0ull;
        for (uint64_t r = rq; r <= 2 * rq; r++) {
            const uint64_t wgs = groups_qk * ((nqk1 + r - 1) / r);
            const uint64_t cc = (wgs + cu1 - 1) / cu1 * r;
            if (cc < cost) {
                cost = cc;
                best = r;
            }
        }
        rq = best;
    }
    c.keys_qk = hsdpa::kDecodeKeysQK * static_cast<int>(rq > 1 ? rq : 1);
    // pass 2 takes 8 tiles per workgroup, or 4 while the smaller workgroups
    // still fit the compute units in one round (short caches: twice the
    // workgroups, measured faster up to 16K keys at 2 KV heads); past one
    // round of 8-wave workgroups, one round of chunked ones: the CUs shared
    // among the groups, each workgroup a run of whole tiles (equal runs stream
    // equal bytes, where rounds of fixed workgroups leave a partial last round)
    const uint64_t nwg4 = (n + 4 * hsdpa::kKeyTile - 1) / (4 * hsdpa::kKeyTile);
    const uint64_t nch = (n + hsdpa::kDecodeKeysPV - 1) / hsdpa::kDecodeKeysPV;
    if (groups * nwg4 <= cu1 || !hsdpa::decode_wide_ok(d)) {
        c.keys_pv = 4 * hsdpa::kKeyTile;
    } else {
        const uint64_t per = cu1 / groups > 0 ? cu1 / groups : 1;
        const uint64_t tiles = (n + hsdpa::kKeyTile - 1) / hsdpa::kKeyTile;
        const uint64_t run = hsdpa::kKeyTile * ((tiles + per - 1) / per);
        c.keys_pv = groups * nch <= cu1 || !hsdpa::decode_pv_loop_ok(d, c.g, static_cast<int>(rows), fused) ||
                            !hsdpa::decode_pv_loop_rows_ok(d, static_cast<int>(rows), sub, p->kv_heads * nch, cu1) ||
                            run > (1u << 30)
                        ? hsdpa::kDecodeKeysPV
                        : static_cast<int>(run);
    }
    // a few rows at D = 256 in 2 to 4 groups where pass 1 takes all of a KV
    // head's groups and 256-key workgroups would take more than one round:
    // one round of workgroups that each walk a run for all the groups
    // (decode_pv_all_loop_ok), the CUs shared among the KV heads only
    bool all_loop = false;
    if (!fused && hsdpa::decode_pv_all_loop_ok(d, static_cast<int>(rows), sub, c.qk_all != 0, p->kv_heads * nch, cu1)) {
        const uint64_t per = cu1 / p->kv_heads > 0 ? cu1 / p->kv_heads : 1;
        const uint64_t tiles = (n + hsdpa::kKeyTile - 1) / hsdpa::kKeyTile;
        const uint64_t run = hsdpa::kKeyTile * ((tiles + per - 1) / per);
        if (run > static_cast<uint64_t>(hsdpa::kDecodeKeysPV) && run <= (uint64_t{1} << 30)) {
            c.keys_pv = static_cast<int>(run);
            all_loop = true;
        }
    }
    c.nwg_qk = static_cast<int>((n + c.keys_qk - 1) / c.keys_qk);
    c.nwg_pv = static_cast<int>((n + c.keys_pv - 1) / c.keys_pv);
    // where pass 1 takes all of a KV head's groups and pass 2 runs 256-key
    // workgroups (D = 256; at D = 64 and 128 it takes chunks there), pass 2
    // takes them all too: each V tile loaded once instead of once per group
    c.pv_all = (c.qk_all && c.keys_pv == hsdpa::kDecodeKeysPV && d == 256) || all_loop ? 1 : 0;
    // a short cache: pass 2 writes the outputs itself, no combine launch
    c.direct = hsdpa::decode_direct_ok(d, static_cast<int>(rows), sub, c.g, n, fused) ? 1 : 0;
    // several groups: a key range's groups on one XCD, whose L2 then serves
    // the later ones (a few rows: 3-8 rows after 32K 11-14 % faster; one row
    // where pass 2 takes several rounds of workgroups, not chunks: 48 heads on
    // 2 KV heads at 128K, 126 -> 109 us; with chunks, or in one round, the
    // plain grid is faster)
    c.xcd = sub > 1 && (rows > 1 || (c.keys_pv <= hsdpa::kDecodeKeysPV && groups * nch > cu1)) ? 1 : 0;
    // the other head dimensions' launchers number the groups on the plain grid
    if (!hsdpa::decode_rows_ok(d)) c.xcd = 0;
    return c;
}

// The most pass-2 workgroups per group over any n <= cap: one round of CUs
// shared among the groups wherever the chunked pass 2 applies, otherwise a
// workgroup per 256 (or 128) keys.
uint64_t decode_nwg_pv_max(const hsdpa_plan *p, uint64_t rows, int sub)
{
    const int d = static_cast<int>(p->spec.head_dim);
    const uint64_t cap = p->spec.kv_capacity, groups = p->kv_heads * static_cast<uint64_t>(sub);
    const uint64_t per = static_cast<uint64_t>(p->cus) / groups > 0 ? static_cast<uint64_t>(p->cus) / groups : 1;
    const uint64_t by128 = (cap + 127) / 128, by256 = (cap + 255) / 256;
    const int g = hsdpa::decode_group_cols(static_cast<int>(rows * p->spec.gqa), sub);
    if (!hsdpa::decode_wide_ok(d)) return by128;
    const uint64_t one_round = std::min(by128, per);
    // the chunked pass 2 gives way to 256-key workgroups where it cannot run
    // (decode_pv_loop_ok) or a run would exceed 2^30 keys
    const uint64_t run_max = 32 * (((cap + 31) / 32 + per - 1) / per);
    // (a Fused plan's tail rows take the Fused rule, its full chunks the Chained one)
    const bool loop = hsdpa::decode_pv_loop_ok(d, g, static_cast<int>(rows), false) &&
                      (p->form != HSDPA_FORM_FUSED || hsdpa::decode_pv_loop_ok(d, g, static_cast<int>(rows), true));
    if (!loop || run_max > (uint64_t{1} << 30))
        return std::max(one_round, by256);
    // several rows at D = 256: 256-key workgroups where decode_pv_loop_rows_ok
    // declines the runs (for any past with more than 4 groups; up to
    // CUs / kv_heads of them where they fit one round)
    if (d == 256 && rows > 1 && sub > 1) {
        if (sub > 4) return std::max(one_round, by256);
        return std::max(one_round, std::min(by256, static_cast<uint64_t>(p->cus) / p->kv_heads));
    }
    return one_round;
}

// The Fused form's rows outside full chunks of 8: the last rows % 8 (the
// reference's passes of 256 rows are multiples of 8, so only the last pass
// ends on a partial chunk), all rows of a call shorter than 8.
uint64_t fused_tail(uint64_t rows) { return rows < 8 ? rows : rows % 8; }

// Whether a call of `rows` rows can reach the causal kernels: under the Fused
// form only its rows in full chunks of 8 can (the others take the decode
// kernels, fused_row_sub).
bool reaches_causal(const hsdpa_plan *p, uint64_t rows)
{
    if (p->form == HSDPA_FORM_FUSED) rows -= fused_tail(rows);
    return rows > 0 && decode_sub(p, rows, std::max<uint64_t>(p->spec.kv_capacity, rows)) == 0;
}

// One sub-call of the node: rows [row0, row0 + rows) of the call, their
// numerics (Fused or Chained) and their kernels.
struct Part {
    uint64_t row0, rows;
    bool fused;
};

}  // namespace

hsdpa_status hsdpa_plan_create(const hsdpa_spec *spec, hsdpa_plan **out)
{
    if (!spec || !out) return HSDPA_ERR_NULL;
    *out = nullptr;
    const hsdpa_status st = check_spec(*spec);
    if (st != HSDPA_OK) return st;
    hsdpa_plan *p = new (std::nothrow) hsdpa_plan();
    if (!p) return HSDPA_ERR_HIP;
    p->spec = *spec;
    const uint64_t d = spec->head_dim, g = spec->gqa, kvh = spec->heads / spec->gqa;
    const uint64_t cap = spec->kv_capacity;
    p->kv_heads = kvh;
    // the Fused form declines the sink (src/jit/emit_sdpa.rs:468-470) and the
    // engine then emits the Chained one
    p->form = spec->form == HSDPA_FORM_FUSED && d <= 256 && !spec->sink ? HSDPA_FORM_FUSED : HSDPA_FORM_CHAINED;
    if (p->form == HSDPA_FORM_FUSED && g > kFusedMaxGqa) {
        delete p;
        return HSDPA_ERR_FORM;
    }
    p->max_rows = spec->max_rows ? spec->max_rows : cap;
    // the grids (and so the workspace) follow the device's compute units; with
    // no device current, the MI355X's 256
    int cus = 0;
    const bool on_gfx950 = check_device(&cus) == HSDPA_OK;
    p->cus = on_gfx950 && cus > 0 ? cus : 256;
    // the static scratch's address on this device, so that no call of
    // hsdpa_attention_static (possibly under graph capture) looks it up
    if (on_gfx950) {
        void *scratch = nullptr;
        if (hsdpa::static_scratch(&scratch) != hipSuccess) {
            delete p;
            return HSDPA_ERR_HIP;
        }
    }
    // decode columns: the query heads of one row, or up to 16 rows of them
    const int gi = static_cast<int>(std::min<uint64_t>(g, 1u << 20));
    const bool pad_ok = hsdpa::decode_rows_ok(static_cast<int>(d)) && hsdpa::decode_groups_pad(gi) > 0;
    uint64_t cols = hsdpa::decode_groups(gi) || pad_ok ? g : 0;
    if (hsdpa::decode_rows_ok(static_cast<int>(d)) && p->max_rows > 1) {
        const uint64_t mr = std::min<uint64_t>(hsdpa::kDecodeMaxRows, p->max_rows);
        cols = std::max(cols, std::min<uint64_t>(hsdpa::kDecodeMaxCols, mr * g));
    }
    p->dec_cols = cols;
    p->dec_npad = align_up(cap, hsdpa::kDecodeKeysPV);
    p->dec_nwg_qk = (cap + hsdpa::kDecodeKeysQK - 1) / hsdpa::kDecodeKeysQK;
    // the largest (pass-2 workgroup, column) count of any call the plan
    // serves, its columns counting the padding of the last group
    uint64_t part = 0, cols_used = 0, cols_pad = 0;
    for (uint64_t r = 1; r <= std::min<uint64_t>(hsdpa::kDecodeMaxRows, p->max_rows); r++) {
        const int sub = r == 1 && p->form == HSDPA_FORM_FUSED ? fused_row_sub(p, 0) : decode_sub(p, r, 0);
        if (sub == 0) continue;
        const uint64_t padded = static_cast<uint64_t>(sub) * hsdpa::decode_group_cols(static_cast<int>(r * g), sub);
        cols_used = std::max(cols_used, r * g);
        cols_pad = std::max(cols_pad, padded);
        part = std::max(part, decode_nwg_pv_max(p, r, sub) * padded);
    }
    p->dec_cols = cols_used;
    p->dec_part = part;
    uint64_t off = 0;
    p->off_scores = off;
    off = align_up(off + kvh * cols_pad * p->dec_npad * 4, kAlign);
    p->off_wgmax = off;
    off = align_up(off + kvh * p->dec_nwg_qk * cols_pad * 4, kAlign);
    p->off_part_o = off;
    off = align_up(off + kvh * part * d * 4, kAlign);
    p->off_part_l = off;
    off = align_up(off + kvh * part * 4, kAlign);
    p->off_bmax = p->off_part_x = off;
    if (p->form == HSDPA_FORM_FUSED) {
        off = align_up(off + kvh * cols_pad * (p->dec_npad / 16) * 4, kAlign);
        p->off_part_x = off;
        off = align_up(off + kvh * part * 4, kAlign);
    }
    // a frame call's step configuration (decode-only plans)
    p->off_fcfg = off;
    if (p->max_rows == 1) off += kAlign;
    p->dec_bytes = off;
    // the split causal kernel: (split, 32-row group, head) cells, enough for
    // one round of the compute units (8 row blocks of 32 per workgroup), when
    // some call of the plan reaches the causal kernels
    bool causal = false;
    for (uint64_t r = 1; r <= std::min<uint64_t>(hsdpa::kDecodeMaxRows + 8, p->max_rows) && !causal; r++)
        causal = reaches_causal(p, r);
    p->split_units = causal ? std::min<uint64_t>(hsdpa::kSplitUnits, 8 * static_cast<uint64_t>(p->cus)) : 0;
    const uint64_t cells = p->split_units * 32;
    p->off_smax = off;
    off = align_up(off + p->split_units * hsdpa::kSplitMaxCells * 4, kAlign);
    p->off_so = off;
    off = align_up(off + cells * d * 4, kAlign);
    p->off_sl = off;
    off = align_up(off + cells * 4, kAlign);
    p->ws_bytes = off;
    *out = p;
    return HSDPA_OK;
}

void hsdpa_plan_destroy(hsdpa_plan *plan) { delete plan; }

uint64_t hsdpa_workspace_bytes(const hsdpa_plan *plan) { return plan ? plan->ws_bytes : 0; }

// Rows [part.row0, part.row0 + part.rows) of a validated call: the decode
// kernels or the causal ones. `route` (optional) receives the kernels, and
// nothing is launched when `launch` is false. `gate`, when not null, is
// applied to the output as it is written (row r, head h at gate +
// r*gate_row + h*head_dim).
static hsdpa_status run_part(const hsdpa_plan *plan, const hsdpa_call *call, const Part &part, const uint16_t *gate,
                             uint64_t gate_row, hipStream_t st, bool launch, uint32_t *kernels, uint32_t *splits,
                             uint32_t *launches)
{
    const hsdpa_spec &s = plan->spec;
    char *ws = static_cast<char *>(call->workspace);
    const uint64_t rows = part.rows, past = call->past + part.row0;
    const uint64_t n = past + rows;
    const int d = static_cast<int>(s.head_dim);
    const uint16_t *q = call->q ? call->q + part.row0 * s.q_row : nullptr;
    uint16_t *outp = call->output ? call->output + part.row0 * s.out_row : nullptr;
    const uint16_t *gp = gate ? gate + part.row0 * gate_row : nullptr;
    const int sub = part.fused && rows == 1 ? fused_row_sub(plan, n) : decode_sub(plan, rows, n);
    if (sub > 0) {
        const DecodeCfg c = decode_cfg(plan, rows, n, sub, part.fused);
        // the workspace holds dec_part (pass-2 workgroup, column) partials per
        // KV head: a grid beyond it is refused, never written past
        if (static_cast<uint64_t>(c.nwg_pv) * static_cast<uint64_t>(c.sub) * static_cast<uint64_t>(c.g) >
            plan->dec_part)
            return HSDPA_ERR_WORKSPACE;
        if (kernels) *kernels = rows == 1 ? HSDPA_KERNELS_DECODE : HSDPA_KERNELS_FEW_ROWS;
        if (splits) *splits = 1;
        if (launches) *launches += c.direct ? 2 : 3;
        if (!launch) return HSDPA_OK;
        hsdpa::DecodeArgs a{};
        a.q = q;
        a.k = call->keys;
        a.v = call->values;
        a.out = outp;
        a.scores = reinterpret_cast<float *>(ws + plan->off_scores);
        a.wgmax = reinterpret_cast<float *>(ws + plan->off_wgmax);
        a.part_o = reinterpret_cast<float *>(ws + plan->off_part_o);
        a.part_l = reinterpret_cast<float *>(ws + plan->off_part_l);
        a.bmax = reinterpret_cast<float *>(ws + plan->off_bmax);
        a.part_x = reinterpret_cast<float *>(ws + plan->off_part_x);
        a.nblk = plan->dec_npad / 16;
        a.n = n;
        a.npad = plan->dec_npad;
        a.kv_stride = s.kv_stride;
        a.q_head = s.q_head;
        a.g = c.g;
        a.sub = c.sub;
        a.rows = static_cast<int>(rows);
        a.G = static_cast<int>(s.gqa);
        a.cols = static_cast<int>(rows * s.gqa);
        a.past = past;
        a.q_row = s.q_row;
        a.out_row = s.out_row;
        a.gate_row = gate_row;
        a.keys_qk = c.keys_qk;
        a.keys_pv = c.keys_pv;
        a.nwg_qk = c.nwg_qk;
        a.nwg_pv = c.nwg_pv;
        a.xcd = c.xcd;
        a.qk_all = c.qk_all;
        a.pv_all = c.pv_all;
        a.direct = c.direct;
        a.scale = call->scale;
        a.sink = call->sink;
        a.sink_on = s.sink != 0;
        a.gate = gp;
        const hipError_t e = part.fused ? hsdpa::launch_decode_fused(a, d, static_cast<int>(plan->kv_heads), st)
                                        : hsdpa::launch_decode(a, d, static_cast<int>(plan->kv_heads), st);
        return e == hipSuccess ? HSDPA_OK : HSDPA_ERR_HIP;
    }
    hsdpa::PrefillArgs a{};
    a.q = q;
    a.k = call->keys;
    a.v = call->values;
    a.out = outp;
    a.rows = rows;
    a.past = past;
    a.n = n;
    a.q_row = s.q_row;
    a.q_head = s.q_head;
    a.out_row = s.out_row;
    a.kv_stride = s.kv_stride;
    a.gqa = static_cast<int>(s.gqa);
    a.scale = call->scale;
    a.sink = call->sink;
    a.sink_on = s.sink != 0;
    a.gate = gp;
    a.gate_row = gate_row;
    hsdpa::PrefillSplit ps{};
    if (plan->split_units) {
        ps.smax = reinterpret_cast<float *>(ws + plan->off_smax);
        ps.so = reinterpret_cast<float *>(ws + plan->off_so);
        ps.sl = reinterpret_cast<float *>(ws + plan->off_sl);
    }
    ps.units = plan->split_units;
    ps.cus = plan->cus;
    // a chunk the one-workgroup causal kernel would spread too thin (it would be
    // split over its keys) and whose row blocks see few key tiles: the waves
    // of each row block's workgroup split its keys instead, in one launch
    hsdpa::PrefillSplit probe = ps;
    probe.units = hsdpa::kSplitUnits;
    const int sp_any = hsdpa::prefill_split_count(a, d, static_cast<int>(s.heads), probe);
    const uint64_t ntiles = (n + hsdpa::kKeyTile - 1) / hsdpa::kKeyTile;
    // (not with the sink: those kernels are not instantiated with it)
    if (sp_any > 1 && !a.sink_on && hsdpa::prefill_short_ok(d) &&
        ntiles <= static_cast<uint64_t>(hsdpa::kShortMaxTiles)) {
        if (kernels) *kernels = HSDPA_KERNELS_CAUSAL_SHORT;
        if (splits) *splits = 1;
        if (launches) *launches += 1;
        if (!launch) return HSDPA_OK;
        const hipError_t e = hsdpa::launch_prefill_short(a, d, static_cast<int>(s.heads), st);
        return e == hipSuccess ? HSDPA_OK : HSDPA_ERR_HIP;
    }
    const int sp = hsdpa::prefill_split_count(a, d, static_cast<int>(s.heads), ps);
    const bool paired = sp == 1 && hsdpa::prefill_pair_rows(a, d, static_cast<int>(s.heads), ps).srows > 0;
    if (kernels)
        *kernels = sp > 1 ? HSDPA_KERNELS_CAUSAL_SPLIT : paired ? HSDPA_KERNELS_CAUSAL_PAIRED : HSDPA_KERNELS_CAUSAL;
    if (splits) *splits = static_cast<uint32_t>(sp);
    if (launches) *launches += sp > 1 || paired ? 3 : 1;
    if (!launch) return HSDPA_OK;
    const hipError_t e = hsdpa::launch_prefill(a, d, static_cast<int>(s.heads), ps, st);
    return e == hipSuccess ? HSDPA_OK : HSDPA_ERR_HIP;
}

// The attention node on validated arguments: under the Fused form the rows
// outside full chunks of 8 take the Fused numerics on the decode kernels (as
// one few-rows call where the decode kernels take them together, else one
// decode per row, fused_row_sub), the others the Chained ones.
static hsdpa_status run_attention(const hsdpa_plan *plan, const hsdpa_call *call, const uint16_t *gate,
                                  uint64_t gate_row, hipStream_t st, bool launch, hsdpa_route *route)
{
    hsdpa_route r{};
    const uint64_t rows = call->rows;
    const uint64_t tail = plan->form == HSDPA_FORM_FUSED ? fused_tail(rows) : 0;
    const uint64_t main = rows - tail;
    uint32_t splits = 1;
    hsdpa_status stt = HSDPA_OK;
    if (main) {
        stt = run_part(plan, call, Part{0, main, false}, gate, gate_row, st, launch, &r.main, &splits, &r.launches);
        r.main_rows = main;
        r.main_form = HSDPA_FORM_CHAINED;
    }
    if (stt == HSDPA_OK && tail) {
        // the tail's kernels decide its numerics: the decode kernels compute the
        // Fused weights, the causal ones the Chained
        const bool together = decode_sub(plan, tail, call->past + rows) > 0;
        uint32_t kern = HSDPA_KERNELS_NONE, sp = 1;
        if (together) {
            stt = run_part(plan, call, Part{main, tail, true}, gate, gate_row, st, launch, &kern, &sp, &r.launches);
        } else {
            for (uint64_t i = 0; i < tail && stt == HSDPA_OK; i++)
                stt = run_part(plan, call, Part{main + i, 1, true}, gate, gate_row, st, launch, &kern, &sp,
                               &r.launches);
            if (tail > 1 && kern == HSDPA_KERNELS_DECODE) kern = HSDPA_KERNELS_DECODE_ROWS;
        }
        const bool on_decode = kern == HSDPA_KERNELS_DECODE || kern == HSDPA_KERNELS_FEW_ROWS ||
                               kern == HSDPA_KERNELS_DECODE_ROWS;
        if (main) {
            r.tail = kern;
            r.tail_rows = tail;
            r.tail_form = on_decode ? HSDPA_FORM_FUSED : HSDPA_FORM_CHAINED;
        } else {
            r.main = kern;
            r.main_rows = tail;
            r.main_form = on_decode ? HSDPA_FORM_FUSED : HSDPA_FORM_CHAINED;
            splits = sp;
        }
    }
    r.splits = splits;
    if (route) *route = r;
    return stt;
}

// The host checks of the attention node (rows > 0 already established).
static hsdpa_status check_attention_call(const hsdpa_plan *plan, const hsdpa_call *call)
{
    const hsdpa_spec &s = plan->spec;
    if (call->rows > s.kv_capacity || call->past > s.kv_capacity - call->rows) return HSDPA_ERR_CAPACITY;
    if (call->rows > plan->max_rows) return HSDPA_ERR_BATCH;
    if (!call->q || !call->keys || !call->values || !call->output || !call->workspace) return HSDPA_ERR_NULL;
    if (!aligned16(call->q) || !aligned16(call->keys) || !aligned16(call->values) || !aligned16(call->output) ||
        !aligned16(call->workspace))
        return HSDPA_ERR_ALIGNMENT;
    if (call->workspace_bytes < plan->ws_bytes) return HSDPA_ERR_WORKSPACE;
    return HSDPA_OK;
}

hsdpa_status hsdpa_attention(const hsdpa_plan *plan, const hsdpa_call *call, void *stream)
{
    if (!plan || !call) return HSDPA_ERR_NULL;
    if (call->rows == 0) return HSDPA_OK;  // the selector's empty call (attention.rs:129-130)
    const hsdpa_status st = check_attention_call(plan, call);
    if (st != HSDPA_OK) return st;
    int cus = 0;
    const hsdpa_status dev = check_device(&cus);
    if (dev != HSDPA_OK) return dev;
    (void)cus;
    return run_attention(plan, call, nullptr, 0, static_cast<hipStream_t>(stream), true, nullptr);
}

hsdpa_status hsdpa_attention_static(const hsdpa_plan *plan, const hsdpa_call *call, void *stream)
{
    if (!plan || !call) return HSDPA_ERR_NULL;
    if (call->rows == 0) return HSDPA_OK;
    if (plan->ws_bytes > HSDPA_STATIC_SCRATCH_BYTES) return HSDPA_ERR_STATIC_SCRATCH;
    int cus = 0;
    const hsdpa_status dev = check_device(&cus);
    if (dev != HSDPA_OK) return dev;
    void *scratch = nullptr;
    if (hsdpa::static_scratch(&scratch) != hipSuccess) return HSDPA_ERR_HIP;
    hsdpa_call c = *call;
    c.workspace = scratch;
    c.workspace_bytes = HSDPA_STATIC_SCRATCH_BYTES;
    const hsdpa_status st = check_attention_call(plan, &c);
    if (st != HSDPA_OK) return st;
    return run_attention(plan, &c, nullptr, 0, static_cast<hipStream_t>(stream), true, nullptr);
}

// A decode step whose rows and past the kernels read from device memory
// (AttentionCall's pointers, src/jit/execution/abi.rs:166-168): the decode
// passes with their configuration derived on the device (frame_args).
hsdpa_status hsdpa_attention_frame(const hsdpa_plan *plan, const hsdpa_frame_call *call, void *stream)
{
    if (!plan || !call) return HSDPA_ERR_NULL;
    const hsdpa_spec &s = plan->spec;
    const int d = static_cast<int>(s.head_dim);
    const int sub = s.gqa <= static_cast<uint64_t>(4 * hsdpa::kDecodeMaxGroup)
                        ? hsdpa::decode_groups(static_cast<int>(s.gqa))
                        : 0;
    if (plan->max_rows != 1 || !hsdpa::decode_rows_ok(d) || sub == 0) return HSDPA_ERR_FRAME;
    // the kernels derive the step's configuration in 32-bit arithmetic
    // (frame_args): the capacity and groups * ceil(capacity / 128) below 2^31
    constexpr uint64_t k31 = static_cast<uint64_t>(1) << 31;
    if (s.kv_capacity >= k31 ||
        plan->kv_heads * static_cast<uint64_t>(sub) *
                ((s.kv_capacity + hsdpa::kDecodeKeysQK - 1) / hsdpa::kDecodeKeysQK) >= k31)
        return HSDPA_ERR_FRAME;
    if (!call->q || !call->keys || !call->values || !call->output || !call->rows || !call->past ||
        !call->workspace)
        return HSDPA_ERR_NULL;
    if (!aligned16(call->q) || !aligned16(call->keys) || !aligned16(call->values) || !aligned16(call->output) ||
        !aligned16(call->workspace) || (reinterpret_cast<uintptr_t>(call->rows) & 7u) ||
        (reinterpret_cast<uintptr_t>(call->past) & 7u) || (reinterpret_cast<uintptr_t>(call->status) & 3u))
        return HSDPA_ERR_ALIGNMENT;
    if (call->workspace_bytes < plan->ws_bytes) return HSDPA_ERR_WORKSPACE;
    int cus = 0;
    const hsdpa_status dev = check_device(&cus);
    if (dev != HSDPA_OK) return dev;
    char *ws = static_cast<char *>(call->workspace);
    hsdpa::DecodeArgs a{};
    a.q = call->q;
    a.k = call->keys;
    a.v = call->values;
    a.out = call->output;
    a.scores = reinterpret_cast<float *>(ws + plan->off_scores);
    a.wgmax = reinterpret_cast<float *>(ws + plan->off_wgmax);
    a.part_o = reinterpret_cast<float *>(ws + plan->off_part_o);
    a.part_l = reinterpret_cast<float *>(ws + plan->off_part_l);
    a.bmax = reinterpret_cast<float *>(ws + plan->off_bmax);
    a.part_x = reinterpret_cast<float *>(ws + plan->off_part_x);
    a.nblk = plan->dec_npad / 16;
    a.npad = plan->dec_npad;
    a.kv_stride = s.kv_stride;
    a.q_head = s.q_head;
    a.sub = sub;
    a.g = hsdpa::decode_group_cols(static_cast<int>(s.gqa), sub);
    a.rows = 1;
    a.G = static_cast<int>(s.gqa);
    a.cols = static_cast<int>(s.gqa);
    a.q_row = s.q_row;
    a.out_row = s.out_row;
    a.scale = call->scale;
    a.sink = call->sink;
    a.sink_on = s.sink != 0;
    a.f_rows = call->rows;
    a.f_past = call->past;
    a.f_status = call->status;
    a.f_cfg = reinterpret_cast<uint32_t *>(ws + plan->off_fcfg);
    a.f_cap = s.kv_capacity;
    a.f_groups = static_cast<int>(plan->kv_heads) * sub;
    a.f_cus = plan->cus;
    // pass 2 walks runs of keys where it can and where 256-key workgroups
    // would not fit the compute units in one round at the capacity
    const uint64_t nch_cap = (s.kv_capacity + hsdpa::kDecodeKeysPV - 1) / hsdpa::kDecodeKeysPV;
    a.f_loop = hsdpa::decode_pv_loop_ok(d, a.g, 1, plan->form == HSDPA_FORM_FUSED) &&
                       static_cast<uint64_t>(a.f_groups) * nch_cap > static_cast<uint64_t>(plan->cus)
                   ? 1
                   : 0;
    const hipError_t e = hsdpa::launch_decode_frame(a, d, static_cast<int>(plan->kv_heads),
                                                    plan->form == HSDPA_FORM_FUSED, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? HSDPA_OK : HSDPA_ERR_HIP;
}

hsdpa_status hsdpa_attention_route(const hsdpa_plan *plan, uint64_t rows, uint64_t past, hsdpa_route *out)
{
    if (!plan || !out) return HSDPA_ERR_NULL;
    *out = hsdpa_route{};
    if (rows == 0) return HSDPA_OK;
    const hsdpa_spec &s = plan->spec;
    if (rows > s.kv_capacity || past > s.kv_capacity - rows) return HSDPA_ERR_CAPACITY;
    if (rows > plan->max_rows) return HSDPA_ERR_BATCH;
    hsdpa_call c{};
    c.rows = rows;
    c.past = past;
    return run_attention(plan, &c, nullptr, 0, nullptr, false, out);
}

hsdpa_status hsdpa_attention_layer(const hsdpa_plan *plan, const hsdpa_layer_call *call, void *stream)
{
    if (!plan || !call) return HSDPA_ERR_NULL;
    const hsdpa_spec &s = plan->spec;
    // the layer's attention node has no sink (its shape: src/jit/schedule/scheduler.rs:111,
    // its call: src/jit/schedule/lowering.rs:609), and the layer call carries none
    if (s.sink) return HSDPA_ERR_SINK_UNSUPPORTED;
    if (call->rows == 0) return HSDPA_OK;
    // the two head-norm-rope nodes (q, then k), checked as hsdpa_head_norm_rope does
    const hsdpa_norm_rope_spec qs = {s.heads, s.head_dim, s.q_head, s.q_row, call->rotary_dims,
                                     call->table_row, call->positions, call->plus_one, 0};
    const hsdpa_norm_rope_spec ks = {plan->kv_heads, s.head_dim, s.head_dim, call->kv_row, call->rotary_dims,
                                     call->table_row, call->positions, call->plus_one, 0};
    hsdpa_status st = check_norm_rope(qs);
    if (st == HSDPA_OK) st = check_norm_rope(ks);
    if (st != HSDPA_OK) return st;
    if (call->rotary_dims && (call->past > call->positions || call->rows > call->positions - call->past))
        return HSDPA_ERR_CAPACITY;
    if (call->rows > (1u << 31) - 1) return HSDPA_ERR_CAPACITY;
    // the attention node
    const hsdpa_call ac = {call->q,     call->keys, call->values, call->output,    call->rows,
                           call->past,  call->scale, 0.0f,        call->workspace, call->workspace_bytes};
    st = check_attention_call(plan, &ac);
    if (st != HSDPA_OK) return st;
    if (!call->k || !call->v || !call->q_norm || !call->k_norm || (call->rotary_dims && (!call->cos || !call->sin)))
        return HSDPA_ERR_NULL;
    // the gate node: compact heads on each row, read 8 bytes at a time
    if (call->gate) {
        if (call->gate_row < s.heads * s.head_dim || call->gate_row > static_cast<uint64_t>(INT32_MAX) / 2)
            return HSDPA_ERR_STRIDE;
        if (!aligned16(call->gate) || call->gate_row % 8 != 0) return HSDPA_ERR_ALIGNMENT;
    }
    int cus = 0;
    const hsdpa_status dev = check_device(&cus);
    if (dev != HSDPA_OK) return dev;
    hipStream_t stream_h = static_cast<hipStream_t>(stream);
    hsdpa::LayerPrepArgs p{};
    p.q = call->q;
    p.k = call->k;
    p.v = call->v;
    p.keys = call->keys;
    p.values = call->values;
    p.q_norm = call->q_norm;
    p.k_norm = call->k_norm;
    p.cos = call->cos;
    p.sin = call->sin;
    p.rows = call->rows;
    p.past = call->past;
    p.q_row = s.q_row;
    p.q_head = s.q_head;
    p.kv_row = call->kv_row;
    p.kv_stride = s.kv_stride;
    p.table_row = call->table_row;
    p.heads = static_cast<int>(s.heads);
    p.kv_heads = static_cast<int>(plan->kv_heads);
    p.dim = static_cast<int>(s.head_dim);
    p.rotary = static_cast<int>(call->rotary_dims);
    p.plus_one = call->plus_one ? 1 : 0;
    p.eps = call->eps;
    if (hsdpa::launch_layer_prep(p, stream_h) != hipSuccess) return HSDPA_ERR_HIP;
    (void)cus;
    return run_attention(plan, &ac, call->gate, call->gate_row, stream_h, true, nullptr);
}

const char *hsdpa_status_string(hsdpa_status status)
{
    switch (status) {
    case HSDPA_OK: return "ok";
    case HSDPA_ERR_EMPTY: return "empty shape (heads, gqa or head_dim is 0)";
    case HSDPA_ERR_HEAD_DIM: return "head_dim out of domain (a multiple of 32 from 32 to 512)";
    case HSDPA_ERR_GQA: return "heads is not a multiple of gqa";
    case HSDPA_ERR_STRIDE: return "invalid q/out/kv strides for this geometry";
    case HSDPA_ERR_SINK_UNSUPPORTED: return "sink flag above 1, or a layer call on a plan with the sink";
    case HSDPA_ERR_CAPACITY: return "past + rows exceeds the KV capacity";
    case HSDPA_ERR_WORKSPACE: return "workspace missing or too small";
    case HSDPA_ERR_ALIGNMENT: return "pointer or stride not 16-byte aligned";
    case HSDPA_ERR_NULL: return "null pointer";
    case HSDPA_ERR_HIP: return "HIP launch or runtime error";
    case HSDPA_ERR_NO_DEVICE: return "no gfx950 device is current";
    case HSDPA_ERR_BATCH: return "more rows than the reserve's max_batch or the plan's max_rows";
    case HSDPA_ERR_LAYOUT: return "the R16 copies of the KV cache are an AArch64 layout";
    case HSDPA_ERR_FORM: return "unknown decode form, or a Fused plan with more than 65536 query heads per KV head";
    case HSDPA_ERR_STATIC_SCRATCH: return "the plan's workspace exceeds the static scratch (HSDPA_STATIC_SCRATCH_BYTES)";
    case HSDPA_ERR_FRAME:
        return "the plan has no frame route (max_rows 1, head_dim 64/128/256, at most 4 equal groups of at most 16 "
               "query heads per KV head)";
    }
    return "unknown status";
}

uint32_t hsdpa_version(void) { return 200; }

}  // extern "C"
