// hsdpa_frame.hip — the decode passes of a frame call (hsdpa_attention_frame):
// the row count and past come from device memory at run time, as the
// reference's attention tasks read them through AttentionCall's pointers
// (src/jit/execution/abi.rs:166-168, attention.rs:228-265), so that one
// enqueued sequence, or one captured HIP graph, serves every decode step of a
// conversation. The kernels are decode_qk, decode_pv and decode_combine with
// FRAME (hsdpa_attn_kernels.h): each derives the step's configuration from n =
// past + 1 (frame_args) and its workgroups past the visible keys exit at once.
// The grids are sized here for any past below the capacity.
//
// In a translation unit of its own, like hsdpa_fused.hip, so that the tuned
// module compiles exactly as before.

#include "hsdpa_attn_kernels.h"

namespace hsdpa {

template <int D, bool FUSED>
static hipError_t frame_d(const DecodeArgs &a, int kv_heads, hipStream_t s)
{
    const uint64_t cap = a.f_cap, groups = static_cast<uint64_t>(a.f_groups), cus = static_cast<uint64_t>(a.f_cus);
    // pass 1: at most ceil(2 CUs / groups) workgroups per group (frame_args
    // takes enough tiles per wave for one round of two per compute unit), and
    // no more than the capacity's 128-key blocks
    const uint64_t by128 = (cap + kDecodeKeysQK - 1) / kDecodeKeysQK;
    const uint64_t qk_round = (2 * cus + groups - 1) / groups;
    const dim3 gqk(static_cast<unsigned>(by128 < qk_round ? by128 : qk_round), kv_heads, a.sub);
    hipError_t e = launch(decode_qk<D, true, 0, FUSED, false, false, true>, gqk, dim3(256), s, a);
    if (e != hipSuccess) return e;
    if (a.f_loop) {
        // a run of at least 128 keys per workgroup, the compute units shared
        // among the groups: at most CUs / groups workgroups, and at most the
        // capacity's 128-key blocks
        const uint64_t per = cus / groups > 0 ? cus / groups : 1;
        const dim3 gpv(static_cast<unsigned>(by128 < per ? by128 : per), kv_heads, a.sub);
        e = a.g <= 8 ? launch(decode_pv<D, 8, 1, true, 0, FUSED, true>, gpv, dim3(512), s, a)
                     : launch(decode_pv<D, 8, 2, true, 0, FUSED, true>, gpv, dim3(512), s, a);
    } else {
        // 256 keys per workgroup: where every past below the capacity fits one
        // round of them (the host's choice up to that length, faster there
        // than a one-chunk run), or where the run cannot loop (D = 256 with
        // more than 8 heads per group)
        const dim3 gpv(static_cast<unsigned>((cap + kDecodeKeysPV - 1) / kDecodeKeysPV), kv_heads, a.sub);
        e = a.g <= 8 ? launch(decode_pv<D, 8, 1, false, 0, FUSED, true>, gpv, dim3(512), s, a)
                     : launch(decode_pv<D, 8, 2, false, 0, FUSED, true>, gpv, dim3(512), s, a);
    }
    if (e != hipSuccess) return e;
    return launch(decode_combine<D, false, FUSED, true>, dim3(kv_heads * a.sub * a.g, (D + 63) / 64),
                  dim3(64 * kCombineSubs), s, a);
}

hipError_t launch_decode_frame(const DecodeArgs &a, int head_dim, int kv_heads, bool fused, hipStream_t s)
{
    switch (head_dim) {
    case 64: return fused ? frame_d<64, true>(a, kv_heads, s) : frame_d<64, false>(a, kv_heads, s);
    case 128: return fused ? frame_d<128, true>(a, kv_heads, s) : frame_d<128, false>(a, kv_heads, s);
    case 256: return fused ? frame_d<256, true>(a, kv_heads, s) : frame_d<256, false>(a, kv_heads, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace hsdpa
