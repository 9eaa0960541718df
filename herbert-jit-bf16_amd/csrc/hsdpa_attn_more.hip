// hsdpa_attn_more.hip — the attention kernels for the head dimensions other
// than 64, 128 and 256: every multiple of 32 from 32 to 512, the range the
// reference's SdpaShape::check accepts (src/jit/ir.rs:130-162). Same templates
// and numerics as hsdpa_kernels.hip, in a translation unit of their own so that
// the tuned instantiations there are compiled exactly as before.
//
// Configurations: the causal kernel serves one query head per workgroup
// (HPW = 1, valid for every group size) and always scales the scores first
// (the general path; with a power-of-two scale it rounds identically to the
// folded one). Up to D = 256 it runs 8 waves, two per SIMD; above, the O and
// Q registers of a 32-row wave (D/2 + D/4) exceed the 256 of two waves per
// SIMD, so it runs 4 waves, one per SIMD. The decode passes take the
// configurations decode_loop_ok / decode_wide_ok allow.

#include "hsdpa_attn_kernels.h"

namespace hsdpa {

template <int D>
static hipError_t decode_more_d(const DecodeArgs &a, int kv_heads, hipStream_t s)
{
    if (a.rows != 1) return hipErrorInvalidValue;           // decode_rows_ok
    const dim3 gqk(a.nwg_qk, kv_heads, a.sub), gpv(a.nwg_pv, kv_heads, a.sub);
    hipError_t e;
    if constexpr (D <= 256) {
        e = a.keys_qk > 4 * kKeyTile ? launch(decode_qk<D, true>, gqk, dim3(256), s, a)
                                     : launch(decode_qk<D, false>, gqk, dim3(256), s, a);
    } else {
        if (a.keys_qk != 4 * kKeyTile) return hipErrorInvalidValue;
        e = launch(decode_qk<D, false>, gqk, dim3(256), s, a);
    }
    if (e != hipSuccess) return e;
    constexpr bool WIDE = D <= 256 && (D / 16 >= 8 || 8 % (D / 16) == 0);   // decode_wide_ok
    if (a.keys_pv == 4 * kKeyTile) {
        e = a.g <= 8 ? launch(decode_pv<D, 4, 1>, gpv, dim3(256), s, a) : launch(decode_pv<D, 4, 2>, gpv, dim3(256), s, a);
    } else {
        if constexpr (WIDE) {
            e = a.g <= 8 ? launch(decode_pv<D, 8, 1>, gpv, dim3(512), s, a)
                         : launch(decode_pv<D, 8, 2>, gpv, dim3(512), s, a);
        } else {
            return hipErrorInvalidValue;
        }
    }
    if (e != hipSuccess) return e;
    return launch(decode_combine<D>, dim3(kv_heads * a.sub * a.g, (D + 63) / 64), dim3(64 * kCombineSubs), s, a);
}

template <int D>
static hipError_t prefill_more_d(const PrefillArgs &a, int heads, const PrefillSplit &ps, hipStream_t s)
{
    constexpr int NW = D > 256 ? 4 : 8;
    constexpr int ROWS = 32 * NW;                                // HPW = 1: NW row blocks of one head
    const dim3 grid(static_cast<unsigned>((a.rows + ROWS - 1) / ROWS), heads);
    const int splits = prefill_splits(a, static_cast<uint64_t>(grid.x) * grid.y, heads, ps);
    if (splits > 1) return launch_prefill_split<D, 1, NW, false>(a, heads, ps, grid, splits, s);
    const PairRows pr = prefill_pairs(a, grid.x, static_cast<uint64_t>(grid.x) * grid.y, ROWS, heads, ps);
    if (pr.srows) return launch_prefill_paired<D, 1, NW, false>(a, heads, ps, grid, pr, s);
    return launch(prefill_attn<D, 1, false, NW>, grid, dim3(64 * NW), s, a);
}

#define HSDPA_MORE_DIMS(X) \
    X(32) X(96) X(160) X(192) X(224) X(288) X(320) X(352) X(384) X(416) X(448) X(480) X(512)

hipError_t launch_decode_more(const DecodeArgs &a, int head_dim, int kv_heads, hipStream_t s)
{
    switch (head_dim) {
#define HSDPA_CASE(D) \
    case D: return decode_more_d<D>(a, kv_heads, s);
        HSDPA_MORE_DIMS(HSDPA_CASE)
#undef HSDPA_CASE
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_prefill_more(const PrefillArgs &a, int head_dim, int heads, const PrefillSplit &ps, hipStream_t s)
{
    switch (head_dim) {
#define HSDPA_CASE(D) \
    case D: return prefill_more_d<D>(a, heads, ps, s);
        HSDPA_MORE_DIMS(HSDPA_CASE)
#undef HSDPA_CASE
    default: return hipErrorInvalidValue;
    }
}

}  // namespace hsdpa
