// hsdpa_fused.hip — the decode passes under the reference's Fused form (the
// sdpa_form = fused knob, src/jit/knobs.rs:66-68; emit_fused,
// src/jit/target/x86/emit_sdpa/x86/decode.rs:501-669): the online softmax over
// blocks of 16 keys, whose exponentials are taken at the running maximum of
// the blocks so far and rescaled by the later blocks' corrections.
//
// The GPU keeps the two passes of the Chained kernels (scores first, then the
// exponentials and P.V), because the exponentials must be evaluated where the
// reference evaluates them: at each block's running maximum, which depends on
// every key before the block. Pass 1 also stores the block maxima where pass
// 2 reads them; pass 2 computes each block's running maximum and correction;
// the combine applies the corrections of the later workgroups (decode_qk,
// decode_pv and decode_combine with FUSED in hsdpa_attn_kernels.h). Head dimensions 32 to
// 256: the form declines above (src/jit/ir.rs:146-148).
//
// In a translation unit of its own, like hsdpa_attn_more.hip, so that the
// tuned Chained module compiles exactly as before.

#include "hsdpa_attn_kernels.h"

namespace hsdpa {

// Pass 1 differs from the Chained one only in storing the maximum of every
// 16-key block (bmax). Pass 2 reads those only for the blocks between the last
// pass-1 workgroup wholly before its keys and its first key, and decode_direct
// reads them all; where every pass-2 workgroup starts at a pass-1 workgroup's
// first key (keys_pv a multiple of keys_qk) the Chained pass 1 writes all that
// pass 2 reads.
static bool fused_needs_bmax(const DecodeArgs &a) { return a.direct || a.keys_pv % a.keys_qk != 0; }

template <int D, int MR, bool BMAX>
static hipError_t fused_pass1(const DecodeArgs &a, dim3 gqk, hipStream_t s)
{
    return a.keys_qk == 8 * kKeyTile ? launch(decode_qk<D, true, MR, BMAX, true>, gqk, dim3(256), s, a)
           : a.keys_qk > 4 * kKeyTile  ? launch(decode_qk<D, true, MR, BMAX>, gqk, dim3(256), s, a)
                                       : launch(decode_qk<D, false, MR, BMAX>, gqk, dim3(256), s, a);
}

// The tuned head dimensions (64, 128, 256): the configurations of the Chained
// launcher, one row (MR = 0), a few rows (MR = 1) or several groups on one
// XCD per key range (MR = 2).
template <int D, int MR>
static hipError_t fused_dm(const DecodeArgs &a, int kv_heads, hipStream_t s)
{
    constexpr bool xcd = MR == 2;
    const auto pad8 = [](int n) { return static_cast<unsigned>((n + 7) / 8 * 8); };
    const dim3 gqk = xcd ? dim3(pad8(a.nwg_qk) * a.sub, kv_heads, 1) : dim3(a.nwg_qk, kv_heads, a.sub);
    const dim3 gpv = xcd ? dim3(pad8(a.nwg_pv) * a.sub, kv_heads, 1) : dim3(a.nwg_pv, kv_heads, a.sub);
    hipError_t e = fused_needs_bmax(a) ? fused_pass1<D, MR, true>(a, gqk, s) : fused_pass1<D, MR, false>(a, gqk, s);
    if (e != hipSuccess) return e;
    if (a.direct) {
        // a short cache: pass 2 over every key writes the outputs (decode_direct_ok)
        if constexpr (MR == 0)
            return launch(decode_direct<D, true, 1, false>, dim3(D / kDirectSlice, kv_heads), dim3(512), s, a);
        else return hipErrorInvalidValue;
    }
    if (a.g <= 8) {
        if (a.keys_pv == 4 * kKeyTile) e = launch(decode_pv<D, 4, 1, false, MR, true>, gpv, dim3(256), s, a);
        else if (a.keys_pv <= kDecodeKeysPV) e = launch(decode_pv<D, 8, 1, false, MR, true>, gpv, dim3(512), s, a);
        else if constexpr (!MR || D < 256) e = launch(decode_pv<D, 8, 1, true, MR, true>, gpv, dim3(512), s, a);
        else return hipErrorInvalidValue;                   // decode_pv_loop_ok
    } else {
        if (a.keys_pv == 4 * kKeyTile) {
            e = launch(decode_pv<D, 4, 2, false, MR, true>, gpv, dim3(256), s, a);
        } else if (a.keys_pv > kDecodeKeysPV) {
            if constexpr (D < 256) e = launch(decode_pv<D, 8, 2, true, MR, true>, gpv, dim3(512), s, a);
            else return hipErrorInvalidValue;               // decode_pv_loop_ok
        } else {
            e = launch(decode_pv<D, 8, 2, false, MR, true>, gpv, dim3(512), s, a);
        }
    }
    if (e != hipSuccess) return e;
    return launch(decode_combine<D, MR != 0, true>, dim3(kv_heads * a.sub * a.g, (D + 63) / 64),
                  dim3(64 * kCombineSubs), s, a);
}

template <int D>
static hipError_t fused_tuned(const DecodeArgs &a, int kv_heads, hipStream_t s)
{
    if (a.xcd) return fused_dm<D, 2>(a, kv_heads, s);
    // one row in equal groups: the one-row kernels; a few rows, or padded
    // groups: the kernels that map each column to its (row, head)
    return a.rows == 1 && a.g * a.sub == a.cols ? fused_dm<D, 0>(a, kv_heads, s) : fused_dm<D, 1>(a, kv_heads, s);
}

// The other head dimensions up to 256: one row, the configurations of
// hsdpa_attn_more.hip; MR = 1 for a group size with no equal split into
// groups of at most 16 (padded groups: the Fused form serves every row on the
// decode kernels, where the Chained form would take the causal kernel).
template <int D, int MR>
static hipError_t fused_more_m(const DecodeArgs &a, int kv_heads, hipStream_t s)
{
    const dim3 gqk(a.nwg_qk, kv_heads, a.sub), gpv(a.nwg_pv, kv_heads, a.sub);
    hipError_t e = fused_needs_bmax(a) ? fused_pass1<D, MR, true>(a, gqk, s) : fused_pass1<D, MR, false>(a, gqk, s);
    if (e != hipSuccess) return e;
    constexpr bool WIDE = D / 16 >= 8 || 8 % (D / 16) == 0;        // decode_wide_ok
    if (a.keys_pv == 4 * kKeyTile) {
        e = a.g <= 8 ? launch(decode_pv<D, 4, 1, false, MR, true>, gpv, dim3(256), s, a)
                     : launch(decode_pv<D, 4, 2, false, MR, true>, gpv, dim3(256), s, a);
    } else {
        if constexpr (WIDE) {
            e = a.g <= 8 ? launch(decode_pv<D, 8, 1, false, MR, true>, gpv, dim3(512), s, a)
                         : launch(decode_pv<D, 8, 2, false, MR, true>, gpv, dim3(512), s, a);
        } else {
            return hipErrorInvalidValue;
        }
    }
    if (e != hipSuccess) return e;
    return launch(decode_combine<D, MR != 0, true>, dim3(kv_heads * a.sub * a.g, (D + 63) / 64),
                  dim3(64 * kCombineSubs), s, a);
}

template <int D>
static hipError_t fused_more(const DecodeArgs &a, int kv_heads, hipStream_t s)
{
    if (a.rows != 1 || a.xcd) return hipErrorInvalidValue;  // decode_rows_ok; decode_cfg
    return a.g * a.sub == a.cols ? fused_more_m<D, 0>(a, kv_heads, s) : fused_more_m<D, 1>(a, kv_heads, s);
}

hipError_t launch_decode_fused(const DecodeArgs &a, int head_dim, int kv_heads, hipStream_t s)
{
    switch (head_dim) {
    case 32: return fused_more<32>(a, kv_heads, s);
    case 64: return fused_tuned<64>(a, kv_heads, s);
    case 96: return fused_more<96>(a, kv_heads, s);
    case 128: return fused_tuned<128>(a, kv_heads, s);
    case 160: return fused_more<160>(a, kv_heads, s);
    case 192: return fused_more<192>(a, kv_heads, s);
    case 224: return fused_more<224>(a, kv_heads, s);
    case 256: return fused_tuned<256>(a, kv_heads, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace hsdpa
