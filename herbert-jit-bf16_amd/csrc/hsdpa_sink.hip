// hsdpa_sink.hip — the causal prefill with the softmax sink (SdpaShape::sink,
// src/jit/ir.rs:55-60), every head dimension from 32 to 512. The sink joins
// each row's maximum, M = vmaxss(max of the scores, sink), its exponential
// P(sink - M) joins the row's sum, and the output is the sum times its
// reciprocal (emit_softmax with the sink,
// src/jit/target/x86/emit_sdpa/x86/decode.rs:239-290). The decode passes take
// the sink at run time (DecodeArgs::sink_on): the Chained ones here and in
// hsdpa_kernels.hip, hsdpa_attn_more.hip and hsdpa_frame.hip.
//
// The kernels are prefill_attn and the split pair of hsdpa_attn_kernels.h with
// SINK set: one query head per workgroup (HPW = 1, valid for every group
// size), the scores scaled first (the general path), 8 waves up to D = 256 and
// 4 above, as hsdpa_attn_more.hip configures the other head dimensions. The
// short-chunk kernels are not instantiated with the sink: such chunks take
// these. In a translation unit of its own, so that the kernels without the
// sink compile exactly as before.

#include "hsdpa_attn_kernels.h"

namespace hsdpa {

template <int D>
static hipError_t prefill_sink_d(const PrefillArgs &a, int heads, const PrefillSplit &ps, hipStream_t s)
{
    constexpr int NW = D > 256 ? 4 : 8;
    constexpr int ROWS = 32 * NW;                                // NW row blocks of one head
    const dim3 grid(static_cast<unsigned>((a.rows + ROWS - 1) / ROWS), heads);
    const int splits = prefill_splits(a, static_cast<uint64_t>(grid.x) * grid.y, heads, ps);
    if (splits > 1) return launch_prefill_split<D, 1, NW, false, true>(a, heads, ps, grid, splits, s);
    const PairRows pr = prefill_pairs(a, grid.x, static_cast<uint64_t>(grid.x) * grid.y, ROWS, heads, ps);
    if (pr.srows) return launch_prefill_paired<D, 1, NW, false, true>(a, heads, ps, grid, pr, s);
    return launch(prefill_attn<D, 1, false, NW, true>, grid, dim3(64 * NW), s, a);
}

#define HSDPA_SINK_DIMS(X)                                                                                  \
    X(32) X(64) X(96) X(128) X(160) X(192) X(224) X(256) X(288) X(320) X(352) X(384) X(416) X(448) X(480) \
    X(512)

hipError_t launch_prefill_sink(const PrefillArgs &a, int head_dim, int heads, const PrefillSplit &ps, hipStream_t s)
{
    switch (head_dim) {
#define HSDPA_CASE(D) \
    case D: return prefill_sink_d<D>(a, heads, ps, s);
        HSDPA_SINK_DIMS(HSDPA_CASE)
#undef HSDPA_CASE
    default: return hipErrorInvalidValue;
    }
}

}  // namespace hsdpa
