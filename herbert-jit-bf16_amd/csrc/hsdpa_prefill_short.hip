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
    // D = 128 and 256: O by dimensions, no partial outputs between the waves,
    // every workgroup running the launch's tile count rounded up to 8, 12, 16,
    // 24 or 32 (a chunk reaches this kernel only with more than 4 tiles: the
    // split it replaces takes at least 4 per split; the host sends none with
    // more than kShortMaxTiles). The P operands of two rounds at a time in the
    // LDS, so the tile count is bounded by the scores kept in registers: 512
    // rows after 512 39.5 -> 29.3 us, 256 after 768 38.0 -> 26.7, 1024 rows
    // with no cache 72.8 -> 55.0 against O by keys (prefill_ks) at D = 256.
    // At D = 256 the row block's keys go to 8 waves, two per SIMD (one to four
    // tiles each, 32 dimensions of O), in rounds of 8 tiles: 512 rows with no
    // cache 20.5 -> 16.7 us, 481 after 30 23.0 -> 16.7, 100 after 220 18.5 ->
    // 14.8 against 4 waves. D = 64: O by keys.
    if constexpr (D == 64) {
        const dim3 grid(static_cast<unsigned>((a.rows + 31) / 32), static_cast<unsigned>(heads));
        return launch(prefill_ks<D, kShortWaves, kShortMaxTiles / kShortWaves, POW2>, grid, dim3(64 * kShortWaves),
                      s, a);
    } else {
        constexpr int KS = D == 256 ? 8 : kShortWaves;
        if (ntiles <= 8) return prefill_kd_mt<D, 8, POW2, KS>(a, heads, s);
        if constexpr (D == 128)
            if (ntiles <= 12) return prefill_kd_mt<D, 12, POW2, KS>(a, heads, s);
        if (ntiles <= 16) return prefill_kd_mt<D, 16, POW2, KS>(a, heads, s);
        if (ntiles <= 24) return prefill_kd_mt<D, 24, POW2, KS>(a, heads, s);
        if (ntiles <= static_cast<uint64_t>(kShortMaxTiles)) return prefill_kd_mt<D, 32, POW2, KS>(a, heads, s);
        return hipErrorInvalidValue;
    }
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
