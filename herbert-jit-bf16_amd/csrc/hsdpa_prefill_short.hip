// hsdpa_prefill_short.hip — the causal prefill of short chunks, the keys of
// each 32-row block split among the waves of its workgroup (prefill_kd and
// prefill_ks in hsdpa_attn_kernels.h), at the tuned head dimensions 64, 128
// and 256. In a translation unit of its own so that the tuned module compiles
// as before.

#include "hsdpa_attn_kernels.h"

namespace hsdpa {

template <int D, int MT, bool POW2, int KS = kShortWaves>
static hipError_t prefill_kd_mt(const PrefillArgs &a, int heads, hipStream_t s)
{
    const dim3 grid(static_cast<unsigned>((a.rows + 31) / 32), static_cast<unsigned>(heads));
    return launch(prefill_kd<D, KS, MT, 4, POW2>, grid, dim3(64 * KS), s, a);
}

template <int D, bool POW2>
static hipError_t prefill_short_dp(const PrefillArgs &a, int heads, hipStream_t s)
{
    const uint64_t ntiles = (a.past + a.rows + kKeyTile - 1) / kKeyTile;
    // up to kShortKdTiles tiles at D = 128 and 256: O by dimensions, no partial
    // outputs between the waves, every workgroup running the launch's tile
    // count rounded up to 8, 12 or 16 (a chunk reaches this kernel only with
    // more than 4 tiles: the split it replaces takes at least 4 per split);
    // beyond (their exponentials no longer fit the LDS), and at D = 64: O by
    // keys. At D = 256 the row block's keys go to 8 waves, two per SIMD (one
    // or two tiles each, 32 dimensions of O), in rounds of 8 tiles: 512 rows
    // with no cache 20.5 -> 16.7 us, 481 after 30 23.0 -> 16.7, 100 after 220
    // 18.5 -> 14.8 against 4 waves.
    if constexpr (D == 256) {
        if (ntiles <= 8) return prefill_kd_mt<D, 8, POW2, 8>(a, heads, s);
        if (ntiles <= 16) return prefill_kd_mt<D, 16, POW2, 8>(a, heads, s);
    }
    if constexpr (D == 128) {
        if (ntiles <= 8) return prefill_kd_mt<D, 8, POW2>(a, heads, s);
        if (ntiles <= 12) return prefill_kd_mt<D, 12, POW2>(a, heads, s);
        if (ntiles <= static_cast<uint64_t>(kShortKdTiles)) return prefill_kd_mt<D, kShortKdTiles, POW2>(a, heads, s);
    }
    const dim3 grid(static_cast<unsigned>((a.rows + 31) / 32), static_cast<unsigned>(heads));
    return launch(prefill_ks<D, kShortWaves, kShortMaxTiles / kShortWaves, POW2>, grid, dim3(64 * kShortWaves), s, a);
}

template <int D>
static hipError_t prefill_short_d(const PrefillArgs &a, int heads, hipStream_t s)
{
    return scale_is_pow2(a.scale) ? prefill_short_dp<D, true>(a, heads, s) : prefill_short_dp<D, false>(a, heads, s);
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
