// hsdpa_prefill_short.hip — the causal prefill of short chunks with the keys of
// each 32-row block split among the waves of its workgroup (prefill_ks in
// hsdpa_attn_kernels.h), at the tuned head dimensions 64, 128 and 256. In a
// translation unit of its own so that the tuned module compiles as before.

#include "hsdpa_attn_kernels.h"

namespace hsdpa {

template <int D>
static hipError_t prefill_short_d(const PrefillArgs &a, int heads, hipStream_t s)
{
    const dim3 grid(static_cast<unsigned>((a.rows + 31) / 32), static_cast<unsigned>(heads));
    if (scale_is_pow2(a.scale)) return launch(prefill_ks<D, kShortWaves, kShortMaxTiles / kShortWaves, true>, grid, dim3(64 * kShortWaves), s, a);
    return launch(prefill_ks<D, kShortWaves, kShortMaxTiles / kShortWaves, false>, grid, dim3(64 * kShortWaves), s, a);
}

hipError_t launch_prefill_short(const PrefillArgs &a, int head_dim, int heads, hipStream_t s)
{
    switch (head_dim) {
    case 64: return prefill_short_d<64>(a, heads, s);
    case 128: return prefill_short_d<128>(a, heads, s);
    case 256: return prefill_short_d<256>(a, heads, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace hsdpa
