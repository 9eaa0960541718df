// hsdpa_attn_kernels.h — gfx950 attention kernels (decode passes, combine, causal
// prefill) as templates over the head dimension, and their launch helpers.
// Included by hsdpa_kernels.hip (head dimensions 64, 128 and 256) and by
// hsdpa_attn_more.hip (the other multiples of 32 up to 512), so that each
// translation unit instantiates only its own head dimensions.
#pragma once

// Numerical contract (the reference's emitted SDPA, x86 AVX-512 BF16):
//   s_j   = fl(dot(q, K_j) * scale)           bf16 products, f32 sums
//   M     = max_j s_j over the visible keys   (the EXACT row maximum)
//   e_j   = P(fl(s_j - M))                    the reference's degree-4 exp
//   out   = bf16(sum_j e_j V_j / sum_j e_j), nearest even
// (src/jit/target/x86/emit_sdpa/x86/decode.rs:212-293 for the softmax,
//  base.rs:189-212 for P, decode.rs:348-428 for the SV pass.)
//
// Two choices follow from matching that contract to within one bf16 ulp:
//  * P is evaluated at the exact row maximum, so the softmax is two-pass
//    (maximum, then exponentials): an online softmax rescaled by P(m_old -
//    m_new) mixes the polynomial's error across blocks and drifts by more
//    than the tolerance allows.
//  * P.V runs on bf16 MFMA with P carried as hi + lo bf16 halves
//    (e = hi + lo exactly to 16 significant bits), two MFMAs per block.
//
// MFMA layout (v_mfma_f32_32x32x16_bf16): lane l, c = l % 32, g = l / 32.
// A[i][k]: lane (i, g) holds k = 8g..8g+7; B[k][j]: lane (j, g) holds the same
// k slots; D[i][j]: lane (j, g) register r holds row i = 8(r/4) + 4g + r%4.
// Scores are computed transposed (S^T = K . Q^T): the key is the MFMA row and
// the query the column, so each lane owns one query and its P^T values feed
// the P.V MFMA (O^T = V^T . P^T) with no data movement. The A-operand rows
// are loaded as K row swap23(i) (bits 2 and 3 of the row swapped), which
// makes score register r of lane group g hold key 16(r/8) + 8g + r%8: eight
// consecutive keys per P.V k-block.
//
// V stays row-major in LDS; its V^T operands come from the gfx950 transpose
// read ds_read_b64_tr_b16. In each 16-lane group, lane j supplies the address
// of four consecutive b16 and lane i receives element i%4 of the chunks of
// lanes i/4 + 4k, k = 0..3. Pointing lane j at V[base + j/4][d0 + 4(j%4)]
// hands lane i the four keys base..base+3 of dimension d0 + i.

#include "hsdpa.h"
#include "hsdpa_kernels.h"

#include <type_traits>

namespace hsdpa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

static constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c)
{
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// v_mfma_f32_16x16x32_bf16, lane l, i = l % 16, G = l / 16: A[i][k] and
// B[k][i] for k = 8G..8G+7; D[4G + r][i] in register r.
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ u32x4 load16(const uint16_t *p) { return *reinterpret_cast<const u32x4 *>(p); }
__device__ __forceinline__ void store16(uint16_t *p, u32x4 v) { *reinterpret_cast<u32x4 *>(p) = v; }

// The emitted exponential (base.rs:189-212, constants exp_constants.rs:14-23):
// clamp at -87.33654, t = x*log2(e), k = rne(t), f = t - k, Horner with FMA,
// times 2^k built from the exponent bits. This file is compiled with
// -ffp-contract=off so that only the written fmaf calls fuse.
__device__ __forceinline__ float exp_poly(float x)
{
    float io = x > -87.33654f ? x : -87.33654f;
    float t1 = io * 1.442695f;
    float t2 = __builtin_rintf(t1);
    t1 = t1 - t2;
    float t3 = __builtin_fmaf(t1, 0.00967248f, 0.05550411f);
    t3 = __builtin_fmaf(t1, t3, 0.2402265f);
    t3 = __builtin_fmaf(t1, t3, 0.6931472f);
    t3 = __builtin_fmaf(t1, t3, 1.0f);
    const uint32_t sc = (static_cast<uint32_t>(static_cast<int32_t>(t2)) << 23) + 0x3F800000u;
    return t3 * __uint_as_float(sc);
}

// The output conversion of the reference epilogue, vcvtneps2bf16: zeros and
// denormals to signed zero, NaN quieted, otherwise nearest even.
__device__ __forceinline__ uint32_t cvt_out(float x)
{
    const uint32_t b = __float_as_uint(x);
    const uint32_t e = b & 0x7F800000u;
    const uint32_t rne = (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
    const uint32_t special = (b & 0x7FFFFFu) ? ((b >> 16) | 0x40u) : (b >> 16);
    const uint32_t r = e == 0x7F800000u ? special : rne;
    return e == 0 ? ((b >> 16) & 0x8000u) : r;
}

// The output gate of one element (ElemOp::SigmoidMul, emit_elem.rs:350-440):
// e = 0 - g; e = e < 88 ? e : 88 (vminps: the bound when e is NaN); the
// softmax's exponential; bf16(a / (e + 1)), a the bf16 attention output.
__device__ __forceinline__ uint16_t gate_bf16(uint16_t a, uint16_t g)
{
    float e = 0.0f - __uint_as_float(static_cast<uint32_t>(g) << 16);
    e = e < 88.0f ? e : 88.0f;
    e = exp_poly(e);
    e = e + 1.0f;
    return static_cast<uint16_t>(cvt_out(__uint_as_float(static_cast<uint32_t>(a) << 16) / e));
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Round two finite f32 to bf16, nearest even, packed low/high
// (v_cvt_pk_bf16_f32: one instruction for the integer rounding
// (b + 0x7FFF + ((b >> 16) & 1)) >> 16 of each value's bits b, with the same
// result).
__device__ __forceinline__ uint32_t pk_bf16(float a, float b)
{
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{a, b}), bf16x2));
}

// Two exponentials as hi and lo bf16 halves, hi = bf16(e), lo = bf16(e - hi),
// each pair packed (e0 low, e1 high).
__device__ __forceinline__ void split2(float e0, float e1, uint32_t &hi, uint32_t &lo)
{
    hi = pk_bf16(e0, e1);
    lo = pk_bf16(e0 - __uint_as_float(hi << 16), e1 - __uint_as_float(hi & 0xFFFF0000u));
}

// Eight exponentials as hi and lo bf16 halves, packed in k order.
__device__ __forceinline__ void split_pack_hw(const float *e, u32x4 &hi, u32x4 &lo)
{
#pragma unroll
    for (int s = 0; s < 4; s++) {
        uint32_t h, q;
        split2(e[2 * s], e[2 * s + 1], h, q);
        hi[s] = h;
        lo[s] = q;
    }
}

__device__ __forceinline__ int swap23(int i) { return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1); }

// Wave reductions on the DPP paths (no LDS round trips). Within each row of
// 16 lanes: swap neighbours, swap pairs, half-row mirror, row mirror; every
// lane of a row then holds the row's result. Across rows, row_bcast:15 folds
// row 0 into row 1 and row 2 into row 3, row_bcast:31 folds lane 31 into rows
// 2 and 3: lane 31 holds the result of lanes 0..31, lane 63 of all 64.
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp(float x, float old)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(x), CTRL, ROWS, 0xF, false));
}

// Lane k of each 16-lane row, in every lane of the row (row_newbcast; k a
// constant once unrolled).
__device__ __forceinline__ float row_lane(float x, int k)
{
    switch (k) {
    case 0: return dpp<0x150, 0xF>(x, x);
    case 1: return dpp<0x151, 0xF>(x, x);
    case 2: return dpp<0x152, 0xF>(x, x);
    case 3: return dpp<0x153, 0xF>(x, x);
    case 4: return dpp<0x154, 0xF>(x, x);
    case 5: return dpp<0x155, 0xF>(x, x);
    case 6: return dpp<0x156, 0xF>(x, x);
    case 7: return dpp<0x157, 0xF>(x, x);
    case 8: return dpp<0x158, 0xF>(x, x);
    case 9: return dpp<0x159, 0xF>(x, x);
    case 10: return dpp<0x15A, 0xF>(x, x);
    case 11: return dpp<0x15B, 0xF>(x, x);
    case 12: return dpp<0x15C, 0xF>(x, x);
    case 13: return dpp<0x15D, 0xF>(x, x);
    case 14: return dpp<0x15E, 0xF>(x, x);
    default: return dpp<0x15F, 0xF>(x, x);
    }
}

// Lane l ^ 8 in lane l (row_ror:8 within the 16-lane row): a DPP move where
// __shfl_xor takes an LDS permute.
__device__ __forceinline__ float row_xor8(float x) { return dpp<0x128, 0xF>(x, x); }

// Lane b - n of the same 16-lane row in lane b (row_shr:n, n = 1, 2, 4 or 8);
// lanes b < n keep `old`.
__device__ __forceinline__ float row_shr_n(float x, int n, float old)
{
    switch (n) {
    case 1: return dpp<0x111, 0xF>(x, old);
    case 2: return dpp<0x112, 0xF>(x, old);
    case 4: return dpp<0x114, 0xF>(x, old);
    default: return dpp<0x118, 0xF>(x, old);
    }
}

__device__ __forceinline__ float row_sum16(float x)
{
    x += dpp<0xB1, 0xF>(x, 0.0f);    // quad_perm [1,0,3,2]
    x += dpp<0x4E, 0xF>(x, 0.0f);    // quad_perm [2,3,0,1]
    x += dpp<0x141, 0xF>(x, 0.0f);   // row_half_mirror
    x += dpp<0x140, 0xF>(x, 0.0f);   // row_mirror
    return x;
}

// Sum over the 64 lanes, valid in lane 63.
__device__ __forceinline__ float wave_sum_hi(float x)
{
    x = row_sum16(x);
    x += dpp<0x142, 0xA>(x, 0.0f);   // row_bcast:15 into rows 1 and 3
    x += dpp<0x143, 0xC>(x, 0.0f);   // row_bcast:31 into rows 2 and 3
    return x;
}

__device__ __forceinline__ float fmaxnn(float a, float b) { return b > a ? b : a; }

// A workgroup barrier that orders LDS only. __syncthreads' fence also waits
// for every global load the wave has in flight, so a barrier placed while the
// next tiles stream in would wait for them.
__device__ __forceinline__ void lds_barrier()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Maximum over each half wave (lanes 0..31 in lane 31, 32..63 in lane 63) and
// over the whole wave (in lane 63) when `whole`. -inf is the identity; NaN
// inputs are ignored like in the scalar reductions.
// The maximum over groups of `lanes` (16, 32 or 64) consecutive lanes: after
// the row steps every lane of a row holds the row's maximum; row_bcast:15
// leaves a 32-lane group's in its lane 31, row_bcast:31 the wave's in lane 63.
__device__ __forceinline__ float group_max_hi(float x, int lanes)
{
    x = fmaxnn(x, dpp<0xB1, 0xF>(x, kNegInf));
    x = fmaxnn(x, dpp<0x4E, 0xF>(x, kNegInf));
    x = fmaxnn(x, dpp<0x141, 0xF>(x, kNegInf));
    x = fmaxnn(x, dpp<0x140, 0xF>(x, kNegInf));
    if (lanes >= 32) x = fmaxnn(x, dpp<0x142, 0xA>(x, kNegInf));
    if (lanes >= 64) x = fmaxnn(x, dpp<0x143, 0xC>(x, kNegInf));
    return x;
}

__device__ __forceinline__ float lane_value(float x, int lane)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

// Key offset inside a 32-key tile of score register r for lane group g.
__device__ __forceinline__ int key_of(int r, int g) { return 16 * (r >> 3) + 8 * g + (r & 7); }

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ u32x2 tr_read(const uint16_t *p)
{
    const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16 *)(p));
    return __builtin_bit_cast(u32x2, r);
}



// A 32-key tile of K or V is 32 * D/8 chunks of 16 bytes. Lanes (or threads)
// take consecutive chunks so every load instruction reads whole rows.
template <int D, int THREADS> struct Tile {
    static constexpr int kChunks = kKeyTile * (D / 8);
    static constexpr int kPer = (kChunks + THREADS - 1) / THREADS;
};

// Loads are unconditional from a clamped in-bounds address (row 0 of the head
// when the chunk is out of range): a conditional load becomes control flow
// that waits on each load before issuing the next. tile_mask zeroes the
// out-of-range chunks afterwards; it waits on the loads, so it goes where the
// data is consumed, not next to the loads.
// NT: non-temporal loads, for the decode streams that no other workgroup
// reads again. The causal kernels load ordinary ones: the workgroups of a KV
// head on one XCD walk the same tiles at about the same time, and the L2 then
// serves all but the first (4096 rows after 8192: 1.50 -> 1.40 ms); so do the
// decode passes whose column groups share an XCD (MR = 2).
template <int D, int THREADS, bool NT = true>
__device__ __forceinline__ void tile_gload(const uint16_t *base, uint64_t t0, uint64_t lim, int tid,
                                           u32x4 (&r)[Tile<D, THREADS>::kPer])
{
    // t0 and lim are uniform: the tile base stays in scalar registers and each
    // lane adds a 32-bit offset. A tile starting at or past lim reads row 0.
    const bool any = t0 < lim;
    const uint16_t *tb = base + (any ? t0 : 0) * D;
    const uint32_t nvalid = any ? static_cast<uint32_t>(lim - t0 < kKeyTile ? lim - t0 : kKeyTile) : 0u;
#pragma unroll
    for (int i = 0; i < Tile<D, THREADS>::kPer; i++) {
        const int c = tid + THREADS * i, key = c / (D / 8), dc = c % (D / 8);
        const bool ok = c < Tile<D, THREADS>::kChunks && static_cast<uint32_t>(key) < nvalid;
        const uint32_t off = ok ? static_cast<uint32_t>(key * D + 8 * dc) : 0u;
        if constexpr (NT) r[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(tb + off));
        else r[i] = *reinterpret_cast<const u32x4 *>(tb + off);
    }
}

template <int D, int THREADS>
__device__ __forceinline__ void tile_mask(uint64_t t0, uint64_t lim, int tid, u32x4 (&r)[Tile<D, THREADS>::kPer])
{
    const uint32_t nvalid = t0 < lim ? static_cast<uint32_t>(lim - t0 < kKeyTile ? lim - t0 : kKeyTile) : 0u;
    if (nvalid == kKeyTile) return;                             // a whole tile (uniform): no selects
#pragma unroll
    for (int i = 0; i < Tile<D, THREADS>::kPer; i++) {
        const int c = tid + THREADS * i;
        const bool ok = c < Tile<D, THREADS>::kChunks && static_cast<uint32_t>(c / (D / 8)) < nvalid;
        r[i] = ok ? r[i] : u32x4{0, 0, 0, 0};
    }
}

// Decode V tiles are [32 keys][D] bf16 without padding. The V^T operand of
// v_mfma_f32_16x16x32_bf16 is two transpose reads; half a wave of one read
// covers rows {k, k+1, k+2, k+3, k+8, .., k+11} (k a multiple of 16) at the
// same 32 bytes of dimensions. XOR-ing the 32-byte slot index of each row
// with f(key) = key % 4 + 4 ((key / 8) % 2) puts those eight rows on eight
// distinct 32-byte bank slots.
// The XOR stays inside an aligned group of swz_group<D>() chunks, the largest
// power of two (at most 16) that divides D/8, so it never leaves the row.
template <int D> constexpr int swz_group()
{
    constexpr int C = D / 8, low = C & -C;       // 16-byte chunks per row, its lowest set bit
    return low < 16 ? low : 16;
}

template <int D> __device__ __forceinline__ int swz16(int key, int chunk)
{
    const int f = (key & 3) | (((key >> 3) & 1) << 2);
    return chunk ^ ((2 * f) & (swz_group<D>() - 1));
}

template <int D, int THREADS>
__device__ __forceinline__ void tile_lstore_v16(uint16_t *tile, int tid, const u32x4 (&r)[Tile<D, THREADS>::kPer])
{
#pragma unroll
    for (int i = 0; i < Tile<D, THREADS>::kPer; i++) {
        const int c = tid + THREADS * i, key = c / (D / 8), dc = c % (D / 8);
        if (c < Tile<D, THREADS>::kChunks) store16(tile + key * D + 8 * swz16<D>(key, dc), r[i]);
    }
}

// tile_mask and tile_lstore_v16 chunk by chunk: each chunk is stored as soon
// as its own load has returned, so the stores overlap the later chunks' arrival.
template <int D, int THREADS>
__device__ __forceinline__ void tile_mask_lstore_v16(uint16_t *tile, uint64_t t0, uint64_t lim, int tid,
                                                     const u32x4 (&r)[Tile<D, THREADS>::kPer])
{
    const uint32_t nvalid = t0 < lim ? static_cast<uint32_t>(lim - t0 < kKeyTile ? lim - t0 : kKeyTile) : 0u;
    if (nvalid == kKeyTile) {                                   // a whole tile (uniform): no selects
        tile_lstore_v16<D, THREADS>(tile, tid, r);
        return;
    }
#pragma unroll
    for (int i = 0; i < Tile<D, THREADS>::kPer; i++) {
        const int c = tid + THREADS * i, key = c / (D / 8), dc = c % (D / 8);
        if (c < Tile<D, THREADS>::kChunks)
            store16(tile + key * D + 8 * swz16<D>(key, dc),
                    static_cast<uint32_t>(key) < nvalid ? r[i] : u32x4{0, 0, 0, 0});
    }
}

// The V^T A operand of v_mfma_f32_16x16x32_bf16 for dimensions [d0, d0+16)
// and the 32 keys of a swizzled tile: lane (i, G) receives keys 8G..8G+7 of
// dimension d0 + i from two transpose reads of four keys each.
template <int D>
__device__ __forceinline__ u32x4 vt16_operand(const uint16_t *vtile, int d0, int l)
{
    const int j = l & 15, G = l >> 4;
    const int key = 8 * G + (j >> 2);
    const int dim = d0 + 4 * (j & 3);
    const u32x2 a = tr_read(vtile + key * D + 8 * swz16<D>(key, dim >> 3) + (dim & 7));
    const u32x2 b = tr_read(vtile + (key + 4) * D + 8 * swz16<D>(key + 4, dim >> 3) + (dim & 7));
    return u32x4{a.x, a.y, b.x, b.y};
}

// Padded tiles: row stride D + 8 for K (a read of 32 rows at one 16-byte
// chunk walks all 16 chunk slots of the banks) and D + 32 for V (the 4 rows
// of a transpose read land in the 4 quarters of the banks). Addresses stay
// affine, so per-access offsets fold into immediates.
template <int D> struct Pad {
    static constexpr int K = D + 8;
    static constexpr int V = D + 32;
};

template <int D, int THREADS>
__device__ __forceinline__ void tile_lstore_padded(uint16_t *tile, int stride, int tid,
                                                   const u32x4 (&r)[Tile<D, THREADS>::kPer])
{
#pragma unroll
    for (int i = 0; i < Tile<D, THREADS>::kPer; i++) {
        const int c = tid + THREADS * i, key = c / (D / 8), dc = c % (D / 8);
        if (c < Tile<D, THREADS>::kChunks) store16(tile + key * stride + 8 * dc, r[i]);
    }
}

// V^T operand from a padded V tile (row stride Pad<D>::V).
template <int D>
__device__ __forceinline__ u32x4 vt_operand_padded(const uint16_t *vtile, int kb, int d0, int l)
{
    constexpr int S = Pad<D>::V;
    const int j = l & 15, G = l >> 4;
    const int key = kb + 8 * (G >> 1) + (j >> 2);
    const int dim = d0 + 16 * (G & 1) + 4 * (j & 3);
    const u32x2 a = tr_read(vtile + key * S + dim);
    const u32x2 b = tr_read(vtile + (key + 4) * S + dim);
    return u32x4{a.x, a.y, b.x, b.y};
}

// ---------------------------------------------------------------------------
// Decode pass 1: scores and per-workgroup maxima.
// grid (nwg_qk, kv_heads), 256 threads, keys_qk = 128: wave w computes the
// 32 keys j0 + 32w .. +32 as two 16-key blocks of v_mfma_f32_16x16x32_bf16
// (S^T = K . Q^T, the g <= 16 query heads of the KV head as the columns).
// The wave loads its 32 K rows whole (each load instruction reads 1 KB of
// contiguous cache), stages them through its own LDS rows with the 16-byte
// chunks XOR-swizzled by key % 16, and reads the A operands from there:
// lane (i, G) takes row i, dimensions 32s + 8G .. +8. Loading the operands
// straight from HBM would request 64 bytes of 16 rows per instruction, which
// streams measurably slower than whole rows.
// ---------------------------------------------------------------------------
// The decode passes' workgroup: key range wg of group z (of a.sub) of KV head
// blockIdx.y. MR = 0 (one row) or 1 (a few rows in one group): wg = blockIdx.x,
// z = blockIdx.z. MR = 2 (a few rows in several groups): x = (wg / 8 * sub +
// z) * 8 + wg % 8, the groups of a key range
// eight workgroups apart, so on one XCD (workgroup i runs on XCD i % 8) and
// close in time: the later ones find the range's tiles in its L2 (3 to 8 rows
// after 32K 11-14 % faster, 4 rows after 128K 16 %). x runs over the key
// ranges padded to a multiple of 8; the padding exits at once.
// The row of column c = r G + rem (c = 0, 1, ..) of a KV head's (row, head)
// columns, for c, c + 2, c + 4, ..: one division, then a step of two columns
// by at most two subtractions (G >= 1), with no branch.
struct ColumnRows {
    int row, rem, G;
    __device__ __forceinline__ ColumnRows(int c, int g) : row(c / g), rem(c - (c / g) * g), G(g) {}
    __device__ __forceinline__ void next2()
    {
        rem += 2;
        const bool w1 = rem >= G;
        rem = w1 ? rem - G : rem;
        row += w1 ? 1 : 0;
        const bool w2 = rem >= G;
        rem = w2 ? rem - G : rem;
        row += w2 ? 1 : 0;
    }
};

template <int MR> struct DecodeIds {
    int wg, z;
    __device__ __forceinline__ explicit DecodeIds(const DecodeArgs &a)
    {
        if constexpr (MR == 2) {
            const int x = static_cast<int>(blockIdx.x), lo = x & 7, t = x >> 3;
            const int hi = t / a.sub;
            z = t - hi * a.sub;
            wg = hi * 8 + lo;
        } else {
            wg = static_cast<int>(blockIdx.x);
            z = static_cast<int>(blockIdx.z);
        }
    }
};

// A frame call (FRAME kernels, hsdpa_attention_frame): the row count and
// past are read from device memory, as the reference's tasks read them
// through AttentionCall's pointers (src/jit/execution/abi.rs:166-168), and
// the decode configuration of n = past + 1 keys is derived here, by the rule
// decode_cfg applies on the host for this grid family (one group per
// workgroup, no short-cache or all-group forms): pass 1 takes decode_cfg's
// tiles per wave (at least as many as one round of two workgroups per
// compute unit needs); pass 2 a
// run of whole tiles per workgroup (at least 128 keys) that shares the
// compute units among the groups, or (f_loop 0: every past below the
// capacity fits one round of them, or the run cannot loop) 256 keys per
// workgroup. Pass 1 derives them (each workgroup alike) and its first
// workgroup leaves them in the workspace (f_cfg) for pass 2 and the combine
// (frame_cfg_load): deriving them again took the step 0.9 us at 32K, the
// divisions of the tile rule on each kernel's critical path. Returns the
// call's status: HSDPA_OK with the arguments set (rows 1), or a status with
// nothing to compute (rows 0: HSDPA_OK with n = 0; more rows than one, or
// past at the capacity: a refusal).
__device__ __forceinline__ uint32_t frame_args(DecodeArgs &a, bool &run)
{
    const uint64_t rows = *a.f_rows, past = *a.f_past;
    run = false;
    if (rows == 0) return HSDPA_OK;
    if (rows > 1) return HSDPA_ERR_BATCH;
    if (past >= a.f_cap) return HSDPA_ERR_CAPACITY;
    run = true;
    // in 32 bits: every kernel of the call runs this before its first load, and
    // 64-bit divisions made it hundreds of instructions. The frame entry
    // refuses capacities of 2^31 keys or more, and group counts with
    // groups * ceil(capacity / 128) of 2^31 or more.
    const uint32_t n = static_cast<uint32_t>(past) + 1u, groups = static_cast<uint32_t>(a.f_groups);
    const uint32_t cus = static_cast<uint32_t>(a.f_cus);
    const uint32_t nqk1 = (n + kDecodeKeysQK - 1) / kDecodeKeysQK;
    // decode_cfg's rule: two tiles per wave at least once one per wave
    // needs more than one workgroup per compute unit, as many as one round
    // of two per unit needs, then the count up to twice that which leaves
    // the fewest tiles on the busiest unit
    const uint32_t rounds = (groups * nqk1 + 2 * cus - 1) / (2 * cus);
    uint32_t rq = groups * nqk1 > cus && rounds < 2 ? 2 : rounds > 1 ? rounds : 1;
    if (rq > 1) {
        uint32_t best = rq, cost = ~0u;
        for (uint32_t r = rq; r <= 2 * rq; r++) {
            const uint32_t wgs = groups * ((nqk1 + r - 1) / r);
            const uint32_t cc = (wgs + cus - 1) / cus * r;
            if (cc < cost) {
                cost = cc;
                best = r;
            }
        }
        rq = best;
    }
    a.past = past;
    a.n = n;
    a.keys_qk = static_cast<int>(kDecodeKeysQK * rq);
    a.nwg_qk = static_cast<int>((n + static_cast<uint32_t>(a.keys_qk) - 1) / static_cast<uint32_t>(a.keys_qk));
    if (a.f_loop) {
        const uint32_t per = cus / groups > 0 ? cus / groups : 1;
        const uint32_t tiles = (n + kKeyTile - 1) / kKeyTile;
        const uint32_t run_keys = kKeyTile * ((tiles + per - 1) / per);
        a.keys_pv = static_cast<int>(run_keys > 4 * kKeyTile ? run_keys : 4 * kKeyTile);
    } else {
        a.keys_pv = kDecodeKeysPV;
    }
    a.nwg_pv = static_cast<int>((n + static_cast<uint32_t>(a.keys_pv) - 1) / static_cast<uint32_t>(a.keys_pv));
    return HSDPA_OK;
}

// The step's configuration in the workspace: status, run, past (low, high),
// keys_qk, nwg_qk, keys_pv, nwg_pv (32 bytes, 16-byte aligned).
__device__ __forceinline__ void frame_cfg_store(const DecodeArgs &a, uint32_t status, bool run)
{
    uint4 *c = reinterpret_cast<uint4 *>(a.f_cfg);
    c[0] = make_uint4(status, run ? 1u : 0u, static_cast<uint32_t>(a.past), static_cast<uint32_t>(a.past >> 32));
    c[1] = make_uint4(static_cast<uint32_t>(a.keys_qk), static_cast<uint32_t>(a.nwg_qk),
                      static_cast<uint32_t>(a.keys_pv), static_cast<uint32_t>(a.nwg_pv));
}

__device__ __forceinline__ uint32_t frame_cfg_load(DecodeArgs &a, bool &run)
{
    const uint4 *c = reinterpret_cast<const uint4 *>(a.f_cfg);
    const uint4 c0 = c[0], c1 = c[1];
    run = c0.y != 0;
    a.past = static_cast<uint64_t>(c0.z) | (static_cast<uint64_t>(c0.w) << 32);
    a.n = run ? a.past + 1 : 0;
    a.keys_qk = static_cast<int>(c1.x);
    a.nwg_qk = static_cast<int>(c1.y);
    a.keys_pv = static_cast<int>(c1.z);
    a.nwg_pv = static_cast<int>(c1.w);
    return c0.x;
}

// FUSED: also store the maximum of every 16-key block of each column (bmax):
// the Fused form evaluates a block's exponentials at the running maximum of
// the blocks up to it. TWO (with LOOP): exactly two tiles per wave. FRAME:
// rows and past read at run time (frame_args); workgroups past the visible
// keys exit at once.
template <int D, bool LOOP, int MR = 0, bool FUSED = false, bool TWO = false, bool MG = false, bool FRAME = false>
__global__ __launch_bounds__(256) void decode_qk(DecodeArgs a)
{
    static_assert(!FRAME || (LOOP && MR == 0 && !TWO && !MG), "frame calls: one group per workgroup, looped tiles");
    if constexpr (FRAME) {
        bool run;
        const uint32_t st = frame_args(a, run);
        if (blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x == 0) frame_cfg_store(a, st, run);
        if (!run || static_cast<int>(blockIdx.x) >= a.nwg_qk) return;
    }
    constexpr int KS = D / 32;
    constexpr int C = D / 8, KM = swz_group<D>() - 1;          // chunks per row, swizzle mask
    // MG: every group of the KV head in this workgroup (at most kDecodeMaxSub),
    // its Q columns staged in LDS in the lanes' operand layout, so that each K
    // tile is loaded and staged once for all of them (several rows after a
    // cache, or more than 16 query heads per KV head)
    constexpr int NG = MG ? kDecodeMaxSub : 1;
    static_assert(!(MG && FUSED), "the Fused form scores one group per workgroup");
    __shared__ __attribute__((aligned(16))) uint16_t kt[4][kKeyTile * D];
    __shared__ __attribute__((aligned(16))) u32x4 qs[MG ? kDecodeMaxSub * KS * 64 : 1];
    __shared__ float red[NG][4][16];
    // blockIdx.y: the KV head; id.z: which of its a.sub groups of g columns
    // (one unless a KV head has more than 16)
    const DecodeIds<MG ? 1 : MR> id(a);
    if (!MG && MR == 2 && id.wg >= a.nwg_qk) return;       // grid padding
    const int ng = MG ? a.sub : 1;
    const int kvh0 = MG ? static_cast<int>(blockIdx.y) * a.sub
                        : MR == 2 ? static_cast<int>(blockIdx.y) * a.sub + id.z
                                  : static_cast<int>(blockIdx.y * gridDim.z + blockIdx.z);
    const int wg = id.wg;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63, i = l & 15, G = l >> 4;
    const uint64_t j0 = static_cast<uint64_t>(wg) * a.keys_qk;
    const uint64_t j1 = j0 + a.keys_qk < a.n ? j0 + a.keys_qk : a.n;
    const bool colv = i < a.g;
    // Rows past the visible keys (loaded from row 0) and columns past g are
    // computed and discarded: an MFMA output element depends only on its own
    // A row and B column. Column i of group z: its Q row and the keys visible
    // to it (keys below lim).
    auto qsrc = [&](int z, uint64_t &lim) {
        lim = a.n;
        if constexpr (MR) {
            // a padded column (past rows * G) computes column 0's scores, never stored
            const int cg = z * a.g + (colv ? i : 0), c = cg < a.cols ? cg : 0, row = c / a.G;
            lim = a.past + static_cast<uint64_t>(row) + 1;
            return a.q + static_cast<uint64_t>(row) * a.q_row +
                   static_cast<uint64_t>(static_cast<int>(blockIdx.y) * a.G + c - row * a.G) * a.q_head + 8 * G;
        } else {
            return a.q + static_cast<uint64_t>((MG ? kvh0 + z : kvh0) * a.g + (colv ? i : 0)) * a.q_head + 8 * G;
        }
    };
    u32x4 qb[KS];
    uint64_t lim1 = a.n;
    if constexpr (MG) {
        for (int z = wave; z < ng; z += 4) {
            uint64_t lz;
            const uint16_t *qp = qsrc(z, lz);
#pragma unroll
            for (int s = 0; s < KS; s++) qs[(z * KS + s) * 64 + l] = load16(qp + 32 * s);
        }
        __syncthreads();
    } else {
        const uint16_t *qp = MR ? qsrc(id.z, lim1) : qsrc(0, lim1);
#pragma unroll
        for (int s = 0; s < KS; s++) qb[s] = load16(qp + 32 * s);
    }
    const uint16_t *kbase = a.k + static_cast<uint64_t>(blockIdx.y) * a.kv_stride;
    uint16_t *my = kt[wave];
    // MG with MR: the row of column z g + i, stepped by g columns from column
    // i's (g = gq G + gr), instead of a division per group and tile
    int qrow0 = 0, qrem0 = 0, gq = 0, gr = 0;
    if constexpr (MG && MR) {
        const int c = colv ? i : 0;
        qrow0 = c / a.G;
        qrem0 = c - qrow0 * a.G;
        gq = a.g / a.G;
        gr = a.g - gq * a.G;
    }
    float m[NG];
#pragma unroll
    for (int z = 0; z < NG; z++) m[z] = kNegInf;
    // One 32-key tile of the wave: staged through its LDS rows, scored for
    // each group, stored.
    auto tile = [&](uint64_t t0, const u32x4 (&kr)[Tile<D, 64>::kPer]) {
#pragma unroll
        for (int c0 = 0; c0 < Tile<D, 64>::kPer; c0++) {
            const int c = l + 64 * c0, key = c / C, dc = c % C;
            store16(my + key * D + 8 * (dc ^ (key & KM)), kr[c0]);
        }
        // The rows are this wave's own: LDS operations of one wave complete in
        // order, so only the compiler has to be kept from reordering them.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        u32x4 ka[2][KS];
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int s = 0; s < KS; s++) {
                const int row = 16 * b + i;
                ka[b][s] = load16(my + row * D + 8 * ((4 * s + G) ^ (row & KM)));
            }
        int crow = qrow0, crem = qrem0;
#pragma unroll
        for (int z = 0; z < NG; z++) {
            if (z >= ng) break;
            const int kvh = MG ? kvh0 + z : kvh0;
            uint64_t lim = lim1;
            if constexpr (MG) {
                if constexpr (MR) {
                    // a padded column (past rows * G) takes row 0's limit
                    const int cg = z * a.g + (colv ? i : 0);
                    lim = a.past + static_cast<uint64_t>(cg < a.cols ? crow : 0) + 1;
                    crow += gq;
                    crem += gr;
                    const bool w = crem >= a.G;
                    crem = w ? crem - a.G : crem;
                    crow += w ? 1 : 0;
                }
#pragma unroll
                for (int s = 0; s < KS; s++) qb[s] = qs[(z * KS + s) * 64 + l];
            }
            f32x4 acc[2] = {};
#pragma unroll
            for (int s = 0; s < KS; s++)
#pragma unroll
                for (int b = 0; b < 2; b++) acc[b] = mfma16(ka[b][s], qb[s], acc[b]);
            if (colv && t0 < j1) {
                float *sp = a.scores + static_cast<uint64_t>(kvh * a.g + i) * a.npad + t0 + 4 * G;
#pragma unroll
                for (int b = 0; b < 2; b++) {
                    float4 v4;
                    float *v = reinterpret_cast<float *>(&v4);
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const uint64_t key = t0 + 16 * b + 4 * G + r;
                        const bool valid = key < j1 && (!MR || key < lim);
                        const float s = acc[b][r] * a.scale;
                        v[r] = valid ? s : kNegInf;
                        if (valid) m[z] = s > m[z] ? s : m[z];
                    }
                    *reinterpret_cast<float4 *>(sp + 16 * b) = v4;
                }
            }
            // a frame call's pass 2 reads block maxima only where its
            // workgroups start inside a pass-1 workgroup's keys (the host path
            // launches the Chained pass 1 where none does)
            if (FUSED && (!FRAME || a.keys_pv % a.keys_qk != 0)) {
                // block b of the tile: keys t0 + 16 b + 4 G + r over the four lane
                // groups G of column i (the same scaled values as stored above)
#pragma unroll
                for (int b = 0; b < 2; b++) {
                    float bm = kNegInf;
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const uint64_t key = t0 + 16 * b + 4 * G + r;
                        const float s = acc[b][r] * a.scale;
                        if (key < j1 && (!MR || key < lim)) bm = s > bm ? s : bm;
                    }
                    const float o16 = __shfl_xor(bm, 16);
                    bm = o16 > bm ? o16 : bm;
                    const float o32 = __shfl_xor(bm, 32);
                    bm = o32 > bm ? o32 : bm;
                    if (colv && G == 0 && t0 + 16 * b < j1)
                        a.bmax[static_cast<uint64_t>(kvh * a.g + i) * a.nblk + (t0 + 16 * b) / 16] = bm;
                }
            }
        }
    };
    constexpr bool NT = MG || MR != 2;     // streams no other workgroup rereads
    if constexpr (!LOOP) {
        u32x4 kr[Tile<D, 64>::kPer];
        tile_gload<D, 64, NT>(kbase, j0 + kKeyTile * wave, j1, l, kr);
        // Every load is in flight before the first use waits on one: left to
        // itself the scheduler interleaves them and keeps only a few outstanding.
        __builtin_amdgcn_sched_barrier(0);
        tile(j0 + kKeyTile * wave, kr);
    } else if (TWO || (FRAME && a.keys_qk == 8 * kKeyTile)) {
        // exactly two rounds of one tile per wave (keys_qk = 256): both tiles
        // requested before the first is scored. In the loop below the second
        // is requested at the top of the loop and waits behind the first
        // (32K keys on 2 KV heads: 21.3 -> 20.6 us); for more rounds the loop
        // runs faster with one tile in flight (two: 0.8 us slower at 64K and
        // 128K). A frame call takes this form whenever its step's keys_qk is
        // 256.
        u32x4 kr0[Tile<D, 64>::kPer], kr1[Tile<D, 64>::kPer];
        tile_gload<D, 64, NT>(kbase, j0 + kKeyTile * wave, j1, l, kr0);
        tile_gload<D, 64, NT>(kbase, j0 + 4 * kKeyTile + kKeyTile * wave, j1, l, kr1);
        __builtin_amdgcn_sched_barrier(0);
        tile(j0 + kKeyTile * wave, kr0);
        __builtin_amdgcn_sched_barrier(0);
        tile(j0 + 4 * kKeyTile + kKeyTile * wave, kr1);
    } else {
        // keys_qk / 128 rounds of one tile per wave, the next round's tile in
        // flight while this one is scored; the prefetch after the last round
        // falls past j1 and reads row 0 (clamped, unused)
        const int rounds = a.keys_qk / (4 * kKeyTile);
        u32x4 kr0[Tile<D, 64>::kPer], kr1[Tile<D, 64>::kPer];
        tile_gload<D, 64, NT>(kbase, j0 + kKeyTile * wave, j1, l, kr0);
        for (int it = 0; it < rounds; it += 2) {
            const uint64_t t0 = j0 + 4 * kKeyTile * it + kKeyTile * wave;
            tile_gload<D, 64, NT>(kbase, t0 + 4 * kKeyTile, j1, l, kr1);
            __builtin_amdgcn_sched_barrier(0);
            tile(t0, kr0);
            if (it + 1 < rounds) {
                tile_gload<D, 64, NT>(kbase, t0 + 8 * kKeyTile, j1, l, kr0);
                __builtin_amdgcn_sched_barrier(0);
                tile(t0 + 4 * kKeyTile, kr1);
            }
        }
    }
#pragma unroll
    for (int z = 0; z < NG; z++) {
        float mz = m[z];
        float mo = __shfl_xor(mz, 16);
        mz = mo > mz ? mo : mz;
        mo = __shfl_xor(mz, 32);
        mz = mo > mz ? mo : mz;
        if (G == 0) red[z][wave][i] = mz;
    }
    __syncthreads();
    // thread z 16 + i: column i of group z
    const int z = static_cast<int>(threadIdx.x) / 16, ic = static_cast<int>(threadIdx.x) % 16;
    if (z < ng && ic < a.g) {
        float r = red[z][0][ic];
#pragma unroll
        for (int w = 1; w < 4; w++) r = red[z][w][ic] > r ? red[z][w][ic] : r;
        a.wgmax[(static_cast<uint64_t>(kvh0 + (MG ? z : 0)) * a.g + ic) * a.nwg_qk + wg] = r;
    }
}

// ---------------------------------------------------------------------------
// Decode pass 2: exponentials at the exact maximum and P.V partial sums.
// grid (nwg_pv, kv_heads), 64 W threads, keys_pv = 32 W (W tiles of 32).
//  1. wave w loads V tile w (whole rows) into registers;
//  2. the exact maximum per query head is reduced from the pass-1 maxima;
//  3. the g x 256 exponentials are computed once, split into hi + lo bf16 and
//     stored in LDS as P columns: with g <= 8, columns 0..7 hold hi and 8..15
//     lo, so one v_mfma_f32_16x16x32_bf16 covers both halves; with g > 8 the
//     hi and lo halves are two 16-column blocks;
//  4. the V tiles go to LDS (swizzled for the 16-row transpose reads);
//  5. wave w reads all its P and V^T operands from LDS, then computes
//     O^T = V^T . P^T for its dimension blocks over its share of the tiles;
//     O = O(hi columns) + O(lo columns).
// NCB: P column blocks, 1 for g <= 8, 2 for g <= 16.
// W waves (and W tiles of keys) per workgroup: W = 8 holds 131 072 + 16 896 +
// ~2 600 bytes of LDS at D = 256, one workgroup per CU; W = 4 half of that, two
// per CU, so that one workgroup's work after its last load overlaps another's
// stream when the grid takes several rounds.
// LOOP: the workgroup covers keys_pv keys (any multiple of 32) in chunks of
// W tiles, one round of workgroups over the cache instead of several: steps
// 3-5 per chunk, the next chunk's scores and V tiles loaded as soon as this
// chunk's V is in LDS (its registers are free then), O accumulated over the
// chunks in the MFMA registers.
// FUSED (the reference's Fused form, src/jit/target/x86/emit_sdpa/x86/decode.rs:
// 501-669): the keys are blocks of 16, each evaluated at the running maximum
// M_b of the blocks up to it instead of the row maximum, and weighted by the
// product C_b of the corrections P(M_{b'-1} - M_b') of the later blocks b' of
// the chunk: e = fl(P(s - M_b) * C_b). The running maximum entering the
// workgroup comes from the pass-1 maxima of the keys before it; a chunk
// rescales what came before it by its corrections' product X (O and l, in
// LOOP), and part_x receives the workgroup's product for the combine.
// ---------------------------------------------------------------------------
template <int D, int W, int NCB, bool LOOP = false, int MR = 0, bool FUSED = false, bool FRAME = false>
__global__ __launch_bounds__(64 * W, D > 256 ? 1 : 8 / W) void decode_pv(DecodeArgs a)
{
    static_assert(!FRAME || MR == 0, "frame calls: one group per workgroup");
    if constexpr (FRAME) {
        bool run;
        frame_cfg_load(a, run);
        if (!run || static_cast<int>(blockIdx.x) >= a.nwg_pv) return;
    }
    constexpr int THREADS = 64 * W;
    constexpr int KEYS = W * kKeyTile;                          // 256 or 128
    constexpr int PS = KEYS + 8;                                // P column stride, bf16
    constexpr int DB = D / 16;                                  // 16-dimension blocks
    constexpr int DBW = DB >= W ? (DB + W - 1) / W : 1;         // blocks per wave
    constexpr int PARTS = DB >= W ? 1 : W / DB;                 // waves per block
    static_assert(DB >= W || W % DB == 0, "the waves split each dimension block evenly");
    // blocks dgi * DBW + db past DB (D/16 not a multiple of W) read block 0 and
    // store nothing
    constexpr bool ALL = DB % W == 0 || DB < W;
    constexpr int WPP = W / PARTS;                              // waves per part
    constexpr int TPP = W / PARTS;                              // tiles per wave
    static_assert(THREADS / KEYS == 2, "two head parities per workgroup");
    __shared__ __attribute__((aligned(16))) uint16_t vt[W][kKeyTile * D];
    __shared__ __attribute__((aligned(16))) uint16_t pc[2 * kDecodeMaxGroup * PS];
    __shared__ float smax[kDecodeMaxGroup];
    __shared__ float lpart[W][kDecodeMaxGroup];
    __shared__ __attribute__((aligned(16))) float ored[PARTS > 1 ? (PARTS - 1) * WPP * NCB * DBW * 4 * 64 : 1];
    // FUSED: per (column, block of the chunk): block maximum, running maximum,
    // product of the later blocks' corrections; per column: the chunk's and
    // the workgroup's products
    constexpr int NB = KEYS / 16;
    constexpr int FN = FUSED ? kDecodeMaxGroup * NB : 1, FH = FUSED ? kDecodeMaxGroup : 1;
    __shared__ float fbm[FN], fmb[FN], fcf[FN], fx[FH], fxw[FH];
    const DecodeIds<MR> id(a);
    if (MR == 2 && id.wg >= a.nwg_pv) return;              // grid padding
    const int kvh = MR == 2 ? static_cast<int>(blockIdx.y) * a.sub + id.z       // as in decode_qk
                            : static_cast<int>(blockIdx.y * gridDim.z + blockIdx.z);
    const int wg = id.wg, tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, j = l & 15, G = l >> 4;
    const uint64_t span = LOOP ? static_cast<uint64_t>(a.keys_pv) : static_cast<uint64_t>(KEYS);
    const uint64_t j0 = static_cast<uint64_t>(wg) * span;
    const uint64_t j1 = j0 + span < a.n ? j0 + span : a.n;
    const uint16_t *vbase = a.v + static_cast<uint64_t>(blockIdx.y) * a.kv_stride;
    constexpr int nh = 8 * NCB;                                 // lo columns start here
    // The small loads go first: the vector-memory counter completes in order,
    // so anything issued after the V tile would wait for all of it.
    const int key_e = tid % KEYS;
    const int hq = __builtin_amdgcn_readfirstlane(tid / KEYS);  // the same in a whole wave
    float sv[kDecodeMaxGroup / 2];
    // this thread's scores of the chunk starting at key c0, columns hq + 2 i
    // (their addresses are the same in a whole wave)
    auto load_scores = [&](uint64_t c0) {
        const uint64_t gk = c0 + key_e, key = gk < j1 ? gk : 0;
#pragma unroll
        for (int i = 0; i < nh / 2; i++) {
            const int h = hq + 2 * i;
            const float *col = a.scores + static_cast<uint64_t>(kvh * a.g + (h < a.g ? h : 0)) * a.npad;
            sv[i] = col[key];
        }
    };
    load_scores(j0);
    // Pass-1 maxima: T lanes per head (THREADS / 8 for g <= 8, THREADS / 16
    // for g <= 16); lane u reads entries u, u + T, .. of head t / T. The first
    // batch is loaded before the V tile, later batches (more than 8 T
    // workgroups in pass 1) after it.
    constexpr int T = THREADS / nh;
    const int jh = tid / T, u = tid % T;
    const float *msrc = a.wgmax + (static_cast<uint64_t>(kvh) * a.g + (jh < a.g ? jh : 0)) * a.nwg_qk;
    constexpr int BATCH = 8;
    // FUSED: only the pass-1 workgroups wholly before this workgroup's keys
    const int wlim = FUSED ? static_cast<int>(j0 / static_cast<uint64_t>(a.keys_qk)) : a.nwg_qk;
    float mx[BATCH];
#pragma unroll
    for (int b = 0; b < BATCH; b++) {
        const int w = u + b * T;
        mx[b] = msrc[w < a.nwg_qk ? w : 0];
    }
    u32x4 vr[Tile<D, 64>::kPer];
    tile_gload<D, 64, MR != 2>(vbase, j0 + kKeyTile * wave, j1, l, vr);
    __builtin_amdgcn_sched_barrier(0);                          // all loads issued first
    float m = kNegInf;
#pragma unroll
    for (int b = 0; b < BATCH; b++) m = (u + b * T < wlim && mx[b] > m) ? mx[b] : m;
    for (int w0 = u + BATCH * T; w0 < wlim; w0 += BATCH * T) {
#pragma unroll
        for (int b = 0; b < BATCH; b++) {
            const int w = w0 + b * T;
            mx[b] = msrc[w < a.nwg_qk ? w : 0];
        }
#pragma unroll
        for (int b = 0; b < BATCH; b++) m = (w0 + b * T < wlim && mx[b] > m) ? mx[b] : m;
    }
    if constexpr (FUSED) {
        // the blocks between the last whole pass-1 workgroup and j0
        const uint64_t b1 = j0 / 16;
        const float *bsrc = a.bmax + (static_cast<uint64_t>(kvh) * a.g + (jh < a.g ? jh : 0)) * a.nblk;
        for (uint64_t b = static_cast<uint64_t>(wlim) * (a.keys_qk / 16) + u; b < b1; b += T) {
            const float x = bsrc[b];
            m = x > m ? x : m;
        }
    }

    // 2. exact maximum per query head (FUSED: the running maximum entering the
    //    workgroup): a DPP reduction over the head's lanes
    m = group_max_hi(m, T);
    // the sink joins the maximum (the Fused form declines it)
    if (!FUSED && a.sink_on) m = m > a.sink ? m : a.sink;
    if (u == T - 1 && jh < a.g) smax[jh] = m;
    __syncthreads();

    const int dgi = wave % WPP, part = wave / WPP;
    f32x4 o[NCB][DBW] = {};
    // steps 3-5 for the chunk of keys [c0, c1); one chunk unless LOOP
    for (uint64_t c0 = j0;; c0 += KEYS) {
        const uint64_t c1 = c0 + KEYS < j1 ? c0 + KEYS : j1;
        const bool kv_e = c0 + key_e < c1;
        // whether key c0 + key_e is visible to column h
        auto visible = [&](int h) {
            bool vis = kv_e;
            if constexpr (MR) {
                // column h's row sees keys [0, past + row]
                const int row = (id.z * a.g + h) / a.G;
                vis = vis && c0 + key_e <= a.past + static_cast<uint64_t>(row);
            }
            return vis;
        };
        if constexpr (FUSED) {
            // (a) the maxima of the chunk's 16-key blocks: a row of 16 lanes
            //     holds one block of one column
#pragma unroll
            for (int i = 0; i < kDecodeMaxGroup / 2; i++) {
                const int h = tid / KEYS + 2 * i;
                if (h >= a.g) break;
                float x = visible(h) ? sv[i] : kNegInf;
                x = group_max_hi(x, 16);
                if ((l & 15) == 0) fbm[h * NB + key_e / 16] = x;
            }
            __syncthreads();
            // (b) per (column, block), in the NB lanes of each column: the
            //     running maximum M_b (a prefix maximum, exact in any order;
            //     M_{-1} the maximum entering the chunk), the correction
            //     P(M_{b-1} - M_b), and C_b = the product of the later blocks'
            //     corrections, multiplied left to right from the column's lanes
            //     (from LDS one after another these scans waited out a read
            //     each); the chunk's product X rescales what came before it
            if (tid < a.g * NB) {
                const int h = tid / NB, b = tid - h * NB;
                const float m0 = smax[h];
                float mb = fbm[tid] > m0 ? fbm[tid] : m0;
                // with 16 blocks a column is one 16-lane DPP row: the shifts
                // and broadcasts are row_shr and row_newbcast moves instead of
                // LDS permutes, each of which the next step waited out (the
                // 15 broadcasts of the product)
                constexpr bool ROW = NB == 16;
#pragma unroll
                for (int off = 1; off < NB; off *= 2) {
                    const float o = ROW ? row_shr_n(mb, off, kNegInf) : __shfl_up(mb, off, NB);
                    if (b >= off && o > mb) mb = o;
                }
                const float mprev = ROW ? row_shr_n(mb, 1, m0) : __shfl_up(mb, 1, NB);
                const float mp = b > 0 ? mprev : m0;
                const float cor = exp_poly(mp - mb);
                float c = 1.0f;
#pragma unroll
                for (int k = 1; k < NB; k++) {
                    const float ck = ROW ? row_lane(cor, k) : __shfl(cor, k, NB);
                    c = k > b ? c * ck : c;
                }
                const float mlast = ROW ? row_lane(mb, NB - 1) : __shfl(mb, NB - 1, NB);
                fmb[tid] = mb;
                fcf[tid] = c;
                if (b == 0) {
                    const float x = cor * c;
                    fx[h] = x;
                    fxw[h] = c0 == j0 ? x : fxw[h] * x;
                    smax[h] = mlast;
                }
            }
            __syncthreads();
        }
        // 3. dense exponentials: thread t owns key c0 + t % KEYS for heads
        //    t / KEYS, t / KEYS + 2, ...; a wave covers 64 consecutive keys of
        //    one head set. Every column slot at once, with no branch between
        //    them, so that the slots' exponentials and sums overlap (taken one
        //    after another, each waited out its own chain); slots past g get
        //    zeros, read only by columns that are never stored.
        constexpr int HC = nh / 2;                              // slots per thread
        float ev[HC];
        ColumnRows rows(id.z * a.g + hq, MR ? a.G : 1);         // MR: column h's row, by steps of two
#pragma unroll
        for (int i = 0; i < HC; i++) {
            const int h = hq + 2 * i;
            if (MR && i > 0) rows.next2();
            // column h's row sees keys [0, past + row]
            const bool vis = (h < a.g) & kv_e & (!MR || c0 + key_e <= a.past + static_cast<uint64_t>(rows.row));
            // computed in every lane, then selected
            float x;
            if constexpr (FUSED) {
                const int fb = h * NB + key_e / 16;
                x = exp_poly(sv[i] - fmb[fb]) * fcf[fb];
            } else {
                x = exp_poly(sv[i] - smax[h]);
            }
            ev[i] = vis ? x : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < HC; i += 2) {
            const int h = hq + 2 * i;                           // slots i and i + 1: columns h, h + 2
            uint32_t hb, lb;
            split2(ev[i], ev[i + 1], hb, lb);
            pc[h * PS + key_e] = static_cast<uint16_t>(hb);
            pc[(h + 2) * PS + key_e] = static_cast<uint16_t>(hb >> 16);
            pc[(nh + h) * PS + key_e] = static_cast<uint16_t>(lb);
            pc[(nh + h + 2) * PS + key_e] = static_cast<uint16_t>(lb >> 16);
        }
        float esum[HC];
#pragma unroll
        for (int i = 0; i < HC; i++) esum[i] = wave_sum_hi(ev[i]);
        if (l == 63) {
#pragma unroll
            for (int i = 0; i < HC; i++) {
                const int h = hq + 2 * i;
                if constexpr (FUSED) lpart[wave][h] = (LOOP && c0 != j0 ? lpart[wave][h] * fx[h] : 0.0f) + esum[i];
                else lpart[wave][h] = (LOOP && c0 != j0 ? lpart[wave][h] : 0.0f) + esum[i];
            }
        }
        // 4. V tile to LDS; with LOOP the next chunk's scores and V tiles are
        //    requested right behind it
        tile_mask_lstore_v16<D, 64>(vt[wave], c0 + kKeyTile * wave, c1, l, vr);
        const bool more = LOOP && c1 < j1;
        if (more) {
            // the stores above read vr first: the loads below reuse its registers
            __builtin_amdgcn_sched_barrier(0);
            load_scores(c0 + KEYS);
            tile_gload<D, 64, MR != 2>(vbase, c0 + KEYS + kKeyTile * wave, j1, l, vr);
        }
        __syncthreads();
        if constexpr (FUSED && LOOP) {
            // what the earlier chunks accumulated, rescaled by this chunk's
            // corrections; lane j holds column j (j % 8 with g <= 8: hi and lo)
            if (c0 != j0) {
                const int hc = NCB == 1 ? (j & 7) : j;
                const float x = fx[hc < a.g ? hc : 0];
#pragma unroll
                for (int c = 0; c < NCB; c++)
#pragma unroll
                    for (int db = 0; db < DBW; db++)
#pragma unroll
                        for (int r = 0; r < 4; r++) o[c][db][r] = o[c][db][r] * x;
            }
        }

        // 5. P.V for this wave's dimension blocks. Columns that hold no head
        //    read whatever the LDS holds; their outputs are never used. Every
        //    operand read is issued before the first MFMA: reading each just
        //    before its MFMA waits out the LDS latency once per MFMA. With
        //    LOOP the next chunk's V registers are live here, so the operands
        //    come in two halves of the tiles, in quarters at D = 256 (the
        //    halves spilled 29 registers under the Fused form: 128K keys on
        //    16/2 heads 77.5 -> 71.2 us Fused, 48K 30.0 -> 29.2 us Chained),
        //    in eighths under the Fused form at D = 256 (quarters spilled 9
        //    registers there, and each reload waited for the next chunk's V
        //    loads: 128K keys 69.8 -> 68.5 us).
        constexpr int PH = FUSED && LOOP && D == 256 && TPP % 8 == 0 ? 8 : LOOP && D == 256 && TPP % 4 == 0 ? 4 : LOOP && TPP % 2 == 0 ? 2 : 1, TPH = TPP / PH;
#pragma unroll
        for (int ph = 0; ph < PH; ph++) {
            u32x4 bp[TPH][NCB], av[TPH][DBW];
#pragma unroll
            for (int tt = 0; tt < TPH; tt++) {
                const int t = part * TPP + ph * TPH + tt;
#pragma unroll
                for (int c = 0; c < NCB; c++) bp[tt][c] = load16(pc + (16 * c + j) * PS + kKeyTile * t + 8 * G);
#pragma unroll
                for (int db = 0; db < DBW; db++) {
                    const int blk = dgi * DBW + db;
                    av[tt][db] = vt16_operand<D>(vt[t], 16 * (ALL || blk < DB ? blk : 0), l);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int tt = 0; tt < TPH; tt++)
#pragma unroll
                for (int db = 0; db < DBW; db++)
#pragma unroll
                    for (int c = 0; c < NCB; c++) o[c][db] = mfma16(av[tt][db], bp[tt][c], o[c][db]);
        }
        if (!more) break;
        __syncthreads();                        // pc and vt are rewritten by the next chunk
    }
    if (PARTS > 1) {
        if (part > 0) {
            float *dst = ored + ((part - 1) * WPP + dgi) * (NCB * DBW * 4 * 64);
#pragma unroll
            for (int c = 0; c < NCB; c++)
#pragma unroll
                for (int db = 0; db < DBW; db++)
#pragma unroll
                    for (int r = 0; r < 4; r++) dst[((c * DBW + db) * 4 + r) * 64 + l] = o[c][db][r];
        }
        __syncthreads();
        if (part == 0)
            for (int p = 1; p < PARTS; p++) {
                const float *src = ored + ((p - 1) * WPP + dgi) * (NCB * DBW * 4 * 64);
#pragma unroll
                for (int c = 0; c < NCB; c++)
#pragma unroll
                    for (int db = 0; db < DBW; db++)
#pragma unroll
                        for (int r = 0; r < 4; r++) o[c][db][r] += src[((c * DBW + db) * 4 + r) * 64 + l];
            }
    }
    // O(head) = O(hi column) + O(lo column): lane j + 8 holds the lo column
    // of head j when g <= 8, the second block when g > 8.
    const uint64_t pbase = (static_cast<uint64_t>(kvh) * a.nwg_pv + wg) * a.g;
#pragma unroll
    for (int db = 0; db < DBW; db++) {
        f32x4 s;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            if constexpr (NCB == 1) s[r] = o[0][db][r] + row_xor8(o[0][db][r]);
            else s[r] = o[0][db][r] + o[NCB - 1][db][r];
        }
        if (part == 0 && j < 8 * NCB && j < a.g && (ALL || dgi * DBW + db < DB)) {
            float *dst = a.part_o + (pbase + j) * D + 16 * (dgi * DBW + db) + 4 * G;
            *reinterpret_cast<float4 *>(dst) = float4{s[0], s[1], s[2], s[3]};
        }
    }
    if (tid < a.g) {
        // heads of parity p were summed by waves p KEYS/64 .., 64 keys each
        const int p0 = (tid % (THREADS / KEYS)) * (KEYS / 64);
        float L = 0.0f;
        for (int w = 0; w < KEYS / 64; w++) L += lpart[p0 + w][tid];
        // the sink's exponential, once per column: in workgroup 0's sum
        if (!FUSED && a.sink_on && wg == 0) L += exp_poly(a.sink - smax[tid]);
        a.part_l[pbase + tid] = L;
        if constexpr (FUSED) a.part_x[pbase + tid] = fxw[tid];
    }
}

// ---------------------------------------------------------------------------
// Decode pass 2 over every group of a KV head in one workgroup (2 to
// kDecodeMaxSub groups of 9 to 16 columns; 8 waves, 256 keys, as decode_pv's
// 8-wave form with two P column blocks). The V tiles are loaded and staged in
// LDS once, and each wave reads its V^T operands into registers once; then,
// for each group in turn, the exact maximum of its columns, the exponentials
// (hi + lo P columns in LDS) and P.V, the scores and maxima of the group
// after next requested before this group's products (two groups in flight). The partials go where decode_pv
// puts them, so the combine is the same. Every column carries its row's
// causal limit (a few rows; one row sees all keys). Grid (nwg_pv, kv_heads).
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(512, 1) void decode_pv_all(DecodeArgs a)
{
    constexpr int W = 8, NCB = 2, THREADS = 64 * W, KEYS = W * kKeyTile, PS = KEYS + 8;
    constexpr int DB = D / 16, DBW = DB / W, nh = 8 * NCB;
    static_assert(DB % W == 0, "each wave takes whole dimension blocks");
    constexpr int T = THREADS / nh, BATCH = 8;                  // lanes per column's maxima
    __shared__ __attribute__((aligned(16))) uint16_t vt[W][kKeyTile * D];
    __shared__ __attribute__((aligned(16))) uint16_t pc[2 * kDecodeMaxGroup * PS];
    __shared__ float smax[kDecodeMaxGroup];
    __shared__ float lpart[W][kDecodeMaxGroup];
    const int wg = static_cast<int>(blockIdx.x), tid = threadIdx.x;
    const int kvh0 = static_cast<int>(blockIdx.y) * a.sub, ng = a.sub;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, j = l & 15, G = l >> 4;
    const uint64_t j0 = static_cast<uint64_t>(wg) * KEYS;
    const uint64_t j1 = j0 + KEYS < a.n ? j0 + KEYS : a.n;
    const uint16_t *vbase = a.v + static_cast<uint64_t>(blockIdx.y) * a.kv_stride;
    const int key_e = tid % KEYS;
    const uint64_t gk = j0 + key_e;
    const bool kv_e = gk < j1;
    const int jh = tid / T, u = tid % T;
    // two groups' loads in flight: group z's scores and maxima arrive while
    // group z - 1 is computed (buffer z % 2)
    float sva[kDecodeMaxGroup / 2], mxa[BATCH], svb[kDecodeMaxGroup / 2], mxb[BATCH];
    const int hq = __builtin_amdgcn_readfirstlane(tid / KEYS);  // the same in a whole wave
    // group z's scores of this thread's key (columns hq + 2 i, whose addresses
    // are the same in a whole wave) and the first batch of its columns'
    // pass-1 maxima
    auto load_group = [&](int z, float(&sv)[kDecodeMaxGroup / 2], float(&mx)[BATCH]) {
        const int kvh = kvh0 + z;
        const uint64_t key = kv_e ? gk : 0;
#pragma unroll
        for (int i = 0; i < nh / 2; i++) {
            const int h = hq + 2 * i;
            const float *col = a.scores + static_cast<uint64_t>(kvh * a.g + (h < a.g ? h : 0)) * a.npad;
            sv[i] = col[key];
        }
        const float *msrc = a.wgmax + (static_cast<uint64_t>(kvh) * a.g + (jh < a.g ? jh : 0)) * a.nwg_qk;
#pragma unroll
        for (int b = 0; b < BATCH; b++) {
            const int w = u + b * T;
            mx[b] = msrc[w < a.nwg_qk ? w : 0];
        }
    };
    load_group(0, sva, mxa);
    if (ng > 1) load_group(1, svb, mxb);
    u32x4 vr[Tile<D, 64>::kPer];
    tile_gload<D, 64, true>(vbase, j0 + kKeyTile * wave, j1, l, vr);
    __builtin_amdgcn_sched_barrier(0);                          // all loads issued first
    u32x4 av[W][DBW];                                           // this wave's V^T operands, all tiles
    // one group: FIRST also stages V and reads the V^T operands; ODD takes
    // buffer b
    auto group = [&](int z, auto first_t, auto odd_t) {
        constexpr bool FIRST = decltype(first_t)::value, ODD = decltype(odd_t)::value;
        float(&sv)[kDecodeMaxGroup / 2] = ODD ? svb : sva;
        float(&mx)[BATCH] = ODD ? mxb : mxa;
        const int kvh = kvh0 + z;
        float m = kNegInf;
#pragma unroll
        for (int b = 0; b < BATCH; b++) m = (u + b * T < a.nwg_qk && mx[b] > m) ? mx[b] : m;
        const float *msrc = a.wgmax + (static_cast<uint64_t>(kvh) * a.g + (jh < a.g ? jh : 0)) * a.nwg_qk;
        for (int w0 = u + BATCH * T; w0 < a.nwg_qk; w0 += BATCH * T) {
#pragma unroll
            for (int b = 0; b < BATCH; b++) {
                const int w = w0 + b * T;
                mx[b] = msrc[w < a.nwg_qk ? w : 0];
            }
#pragma unroll
            for (int b = 0; b < BATCH; b++) m = (w0 + b * T < a.nwg_qk && mx[b] > m) ? mx[b] : m;
        }
        m = group_max_hi(m, T);
        if (a.sink_on) m = m > a.sink ? m : a.sink;             // the sink joins the maximum
        // the previous group's P operand reads and partial sums are done
        // before this barrier, so its slots may be rewritten after it
        if (u == T - 1 && jh < a.g) smax[jh] = m;
        __syncthreads();
        // column tid's maximum, for the sink's term (smax is rewritten by the
        // next group once every wave has passed this group's second barrier)
        const float mcol = tid < a.g ? smax[tid] : 0.0f;
        // every column slot at once, with no branch between them (as in
        // decode_pv); slots past g get zeros
        float ev[nh / 2];
        // column h's row sees keys [0, past + row], row = (z g + h) / G, by
        // steps of two columns
        ColumnRows rows(z * a.g + hq, a.G);
#pragma unroll
        for (int i = 0; i < nh / 2; i++) {
            const int h = hq + 2 * i;
            if (i > 0) rows.next2();
            const bool vis = (h < a.g) & kv_e & (gk <= a.past + static_cast<uint64_t>(rows.row));
            const float x = exp_poly(sv[i] - smax[h]);          // computed in every lane, then selected
            ev[i] = vis ? x : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < nh / 2; i += 2) {
            const int h = hq + 2 * i;                           // slots i and i + 1: columns h, h + 2
            uint32_t hb, lb;
            split2(ev[i], ev[i + 1], hb, lb);
            pc[h * PS + key_e] = static_cast<uint16_t>(hb);
            pc[(h + 2) * PS + key_e] = static_cast<uint16_t>(hb >> 16);
            pc[(nh + h) * PS + key_e] = static_cast<uint16_t>(lb);
            pc[(nh + h + 2) * PS + key_e] = static_cast<uint16_t>(lb >> 16);
        }
        float esum[nh / 2];
#pragma unroll
        for (int i = 0; i < nh / 2; i++) esum[i] = wave_sum_hi(ev[i]);
        if (l == 63) {
#pragma unroll
            for (int i = 0; i < nh / 2; i++) lpart[wave][hq + 2 * i] = esum[i];
        }
        if (z + 2 < ng) load_group(z + 2, sv, mx);
        if constexpr (FIRST) tile_mask_lstore_v16<D, 64>(vt[wave], j0 + kKeyTile * wave, j1, l, vr);
        __syncthreads();
        if constexpr (FIRST) {
#pragma unroll
            for (int t = 0; t < W; t++)
#pragma unroll
                for (int db = 0; db < DBW; db++) av[t][db] = vt16_operand<D>(vt[t], 16 * (wave * DBW + db), l);
        }
        u32x4 bp[W][NCB];
#pragma unroll
        for (int t = 0; t < W; t++)
#pragma unroll
            for (int c = 0; c < NCB; c++) bp[t][c] = load16(pc + (16 * c + j) * PS + kKeyTile * t + 8 * G);
        __builtin_amdgcn_sched_barrier(0);
        f32x4 o[NCB][DBW] = {};
#pragma unroll
        for (int t = 0; t < W; t++)
#pragma unroll
            for (int db = 0; db < DBW; db++)
#pragma unroll
                for (int c = 0; c < NCB; c++) o[c][db] = mfma16(av[t][db], bp[t][c], o[c][db]);
        // O(column) = O(hi block) + O(lo block)
        const uint64_t pbase = (static_cast<uint64_t>(kvh) * a.nwg_pv + wg) * a.g;
#pragma unroll
        for (int db = 0; db < DBW; db++) {
            if (j < a.g) {
                float *dst = a.part_o + (pbase + j) * D + 16 * (wave * DBW + db) + 4 * G;
                *reinterpret_cast<float4 *>(dst) = float4{o[0][db][0] + o[1][db][0], o[0][db][1] + o[1][db][1],
                                                          o[0][db][2] + o[1][db][2], o[0][db][3] + o[1][db][3]};
            }
        }
        if (tid < a.g) {
            // columns of parity p were summed by waves 4 p .. 4 p + 3, 64 keys each
            const int p0 = (tid % (THREADS / KEYS)) * (KEYS / 64);
            float L = 0.0f;
            for (int w = 0; w < KEYS / 64; w++) L += lpart[p0 + w][tid];
            if (a.sink_on && wg == 0) L += exp_poly(a.sink - mcol);  // once per column
            a.part_l[pbase + tid] = L;
        }
    };
    group(0, std::true_type{}, std::false_type{});
    for (int z = 1; z < ng; z += 2) {
        group(z, std::false_type{}, std::true_type{});
        if (z + 1 < ng) group(z + 1, std::false_type{}, std::false_type{});
    }
}

// ---------------------------------------------------------------------------
// Decode pass 2 over every group of a KV head in one workgroup that walks a
// run of keys in 256-key chunks (up to kDecodeLoopMaxSub groups of at most 16
// columns: a few rows over a long cache, one round of (nwg_pv, kv_heads)
// workgroups). First the exact maxima of every group's columns (two groups'
// pass-1 maxima in flight). Then per chunk: the V tiles staged in LDS once for
// all the groups; for each group in turn the exponentials (hi + lo P columns
// in LDS, the column sums added up per wave in LDS), the next group's scores
// requested, and P.V into the group's accumulator (the hi and the lo block
// into one), which stays in registers over the whole run, the V^T operands
// read from LDS for each group in parts of two tiles; the next chunk's V
// tiles are requested after the last group (held in registers during the
// groups, they spilled). The partials and column sums go where decode_pv
// puts them, so the combine is the same. Each column carries its row's
// causal limit.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(512, 1) void decode_pv_all_loop(DecodeArgs a)
{
    constexpr int W = 8, NCB = 2, THREADS = 64 * W, KEYS = W * kKeyTile, PS = KEYS + 8;
    constexpr int DB = D / 16, DBW = DB / W, nh = 8 * NCB, HC = nh / 2, MS = kDecodeLoopMaxSub;
    static_assert(DB % W == 0, "each wave takes whole dimension blocks");
    static_assert(MS * W * kDecodeMaxGroup <= THREADS, "one thread per column sum to clear");
    constexpr int T = THREADS / nh, BATCH = 8;                  // lanes per column's maxima
    __shared__ __attribute__((aligned(16))) uint16_t vt[W][kKeyTile * D];
    __shared__ __attribute__((aligned(16))) uint16_t pc[2 * kDecodeMaxGroup * PS];
    __shared__ float smax[MS][kDecodeMaxGroup];
    __shared__ float lsum[MS][W][kDecodeMaxGroup];
    __shared__ int crow[MS][kDecodeMaxGroup];                   // the row of group z's column h
    const int wg = static_cast<int>(blockIdx.x), tid = threadIdx.x;
    const int kvh0 = static_cast<int>(blockIdx.y) * a.sub, ng = a.sub;     // 2 <= ng <= MS
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, j = l & 15, G = l >> 4;
    const uint64_t j0 = static_cast<uint64_t>(wg) * static_cast<uint64_t>(a.keys_pv);
    const uint64_t j1 = j0 + static_cast<uint64_t>(a.keys_pv) < a.n ? j0 + static_cast<uint64_t>(a.keys_pv) : a.n;
    const uint16_t *vbase = a.v + static_cast<uint64_t>(blockIdx.y) * a.kv_stride;
    const int key_e = tid % KEYS;
    const int hq = __builtin_amdgcn_readfirstlane(tid / KEYS);  // the same in a whole wave
    const int jh = tid / T, u = tid % T;
    // group z's scores of this thread's key of the chunk at c0 (columns hq + 2 i),
    // in buffer z % 2, requested one group ahead
    float sva[HC], svb[HC];
    auto load_scores = [&](int z, uint64_t c0, float(&sv)[HC]) {
        const uint64_t gk = c0 + key_e, key = gk < j1 ? gk : 0;
        const int kvh = kvh0 + z;
#pragma unroll
        for (int i = 0; i < HC; i++) {
            const int h = hq + 2 * i;
            const float *col = a.scores + static_cast<uint64_t>(kvh * a.g + (h < a.g ? h : 0)) * a.npad;
            sv[i] = col[key];
        }
    };
    // group z's first batch of pass-1 maxima, in buffer z % 2 (two groups' in
    // flight)
    auto load_max = [&](int z, float(&mx)[BATCH]) {
        const float *msrc = a.wgmax + (static_cast<uint64_t>(kvh0 + z) * a.g + (jh < a.g ? jh : 0)) * a.nwg_qk;
#pragma unroll
        for (int b = 0; b < BATCH; b++) {
            const int w = u + b * T;
            mx[b] = msrc[w < a.nwg_qk ? w : 0];
        }
    };
    // the first two groups' maxima, the first chunk's scores of group 0 and
    // its V tiles
    float mxa[BATCH], mxb[BATCH];
    load_max(0, mxa);
    load_max(1, mxb);
    load_scores(0, j0, sva);
    u32x4 vr[Tile<D, 64>::kPer];
    tile_gload<D, 64, true>(vbase, j0 + kKeyTile * wave, j1, l, vr);
    __builtin_amdgcn_sched_barrier(0);                          // all loads issued first
    // the exact maxima, group by group (the sink joins them)
#pragma unroll
    for (int z = 0; z < MS; z++) {
        if (z < ng) {
            float(&mx)[BATCH] = (z & 1) ? mxb : mxa;
            float m = kNegInf;
#pragma unroll
            for (int b = 0; b < BATCH; b++) m = (u + b * T < a.nwg_qk && mx[b] > m) ? mx[b] : m;
            if (z + 2 < ng) load_max(z + 2, mx);
            const float *msrc = a.wgmax + (static_cast<uint64_t>(kvh0 + z) * a.g + (jh < a.g ? jh : 0)) * a.nwg_qk;
            for (int w0 = u + BATCH * T; w0 < a.nwg_qk; w0 += BATCH * T) {
                float xb[BATCH];
#pragma unroll
                for (int b = 0; b < BATCH; b++) {
                    const int w = w0 + b * T;
                    xb[b] = msrc[w < a.nwg_qk ? w : 0];
                }
#pragma unroll
                for (int b = 0; b < BATCH; b++) m = (w0 + b * T < a.nwg_qk && xb[b] > m) ? xb[b] : m;
            }
            m = group_max_hi(m, T);
            if (a.sink_on) m = m > a.sink ? m : a.sink;
            if (u == T - 1 && jh < a.g) smax[z][jh] = m;
        }
    }
    if (tid < MS * W * kDecodeMaxGroup) (&lsum[0][0][0])[tid] = 0.0f;
    if (tid < MS * kDecodeMaxGroup) (&crow[0][0])[tid] = ((tid / kDecodeMaxGroup) * a.g + tid % kDecodeMaxGroup) / a.G;
    f32x4 o[MS][DBW] = {};                                      // hi and lo P blocks into one accumulator
    for (uint64_t c0 = j0; c0 < j1; c0 += KEYS) {
        const uint64_t c1 = c0 + KEYS < j1 ? c0 + KEYS : j1;
        const uint64_t gk = c0 + key_e;
        const bool kv_e = gk < c1, more = c1 < j1;
        // every wave's P.V of the previous chunk has read the V tiles (first:
        // the maxima and the cleared sums are visible)
        __syncthreads();
        tile_mask_lstore_v16<D, 64>(vt[wave], c0 + kKeyTile * wave, c1, l, vr);
        auto group = [&](auto zt) {
            constexpr int z = decltype(zt)::value;
            float(&sv)[HC] = (z & 1) ? svb : sva;
            // column h's row sees keys [0, past + row]: key c0 + key_e while
            // key_e <= past + row - c0, a limit in [-1, KEYS] in a scalar
            // register; the rows are read from LDS in the chunk loop (held
            // in registers for every group and column over the loop, they
            // spilled)
            float ev[HC];
            const int64_t rel0 = static_cast<int64_t>(a.past) - static_cast<int64_t>(c0);
#pragma unroll
            for (int i = 0; i < HC; i++) {
                const int h = hq + 2 * i;
                const int64_t rel = rel0 + __builtin_amdgcn_readfirstlane(crow[z][h]);
                const int lim = __builtin_amdgcn_readfirstlane(static_cast<int>(rel < 0 ? -1 : rel > KEYS ? KEYS : rel));
                const bool vis = (h < a.g) & kv_e & (key_e <= lim);
                const float x = exp_poly(sv[i] - smax[z][h]);   // computed in every lane, then selected
                ev[i] = vis ? x : 0.0f;
            }
            // the next group's scores, or the next chunk's of group 0 (this
            // buffer's scores are used above)
            if (z + 1 < ng) load_scores(z + 1, c0, ((z + 1) & 1) ? svb : sva);
            else if (more) load_scores(0, c1, sva);
#pragma unroll
            for (int i = 0; i < HC; i += 2) {
                const int h = hq + 2 * i;                       // slots i and i + 1: columns h, h + 2
                uint32_t hb, lb;
                split2(ev[i], ev[i + 1], hb, lb);
                pc[h * PS + key_e] = static_cast<uint16_t>(hb);
                pc[(h + 2) * PS + key_e] = static_cast<uint16_t>(hb >> 16);
                pc[(nh + h) * PS + key_e] = static_cast<uint16_t>(lb);
                pc[(nh + h + 2) * PS + key_e] = static_cast<uint16_t>(lb >> 16);
            }
            float esum[HC];
#pragma unroll
            for (int i = 0; i < HC; i++) esum[i] = wave_sum_hi(ev[i]);
            if (l == 63) {
#pragma unroll
                for (int i = 0; i < HC; i++) lsum[z][wave][hq + 2 * i] += esum[i];
            }
            __syncthreads();                                    // the P columns (and V tiles) are in LDS
            // P.V in parts of TP tiles, each part's P and V^T operands read
            // from LDS before its MFMAs; the last part's are read before the
            // barrier after which pc is written again
            constexpr int TP = 2;
            auto part = [&](auto pt) {
                constexpr int t0 = decltype(pt)::value * TP;
                constexpr bool LAST = t0 + TP == W;
                u32x4 bp[TP][NCB], av[TP][DBW];
#pragma unroll
                for (int t = 0; t < TP; t++) {
#pragma unroll
                    for (int c = 0; c < NCB; c++) bp[t][c] = load16(pc + (16 * c + j) * PS + kKeyTile * (t0 + t) + 8 * G);
#pragma unroll
                    for (int db = 0; db < DBW; db++) av[t][db] = vt16_operand<D>(vt[t0 + t], 16 * (wave * DBW + db), l);
                }
                if constexpr (LAST) __syncthreads();
#pragma unroll
                for (int t = 0; t < TP; t++)
#pragma unroll
                    for (int db = 0; db < DBW; db++)
#pragma unroll
                        for (int c = 0; c < NCB; c++) o[z][db] = mfma16(av[t][db], bp[t][c], o[z][db]);
                __builtin_amdgcn_sched_barrier(0);
            };
            part(std::integral_constant<int, 0>{});
            part(std::integral_constant<int, 1>{});
            part(std::integral_constant<int, 2>{});
            part(std::integral_constant<int, 3>{});
        };
        group(std::integral_constant<int, 0>{});
        group(std::integral_constant<int, 1>{});
        if constexpr (MS > 2) { if (ng > 2) group(std::integral_constant<int, 2>{}); }
        if constexpr (MS > 3) { if (ng > 3) group(std::integral_constant<int, 3>{}); }
        // the next chunk's V tiles (requested here, where the P.V operands
        // are no longer held)
        if (more) tile_gload<D, 64, true>(vbase, c1 + kKeyTile * wave, j1, l, vr);
    }
    __syncthreads();                                            // the column sums are complete
#pragma unroll
    for (int z = 0; z < MS; z++) {
        if (z < ng) {
            const uint64_t pbase = (static_cast<uint64_t>(kvh0 + z) * a.nwg_pv + wg) * a.g;
#pragma unroll
            for (int db = 0; db < DBW; db++) {
                if (j < a.g) {
                    float *dst = a.part_o + (pbase + j) * D + 16 * (wave * DBW + db) + 4 * G;
                    *reinterpret_cast<float4 *>(dst) = float4{o[z][db][0], o[z][db][1], o[z][db][2], o[z][db][3]};
                }
            }
            if (tid < a.g) {
                // columns of parity p were summed by waves 4 p .. 4 p + 3
                const int p0 = (tid % (THREADS / KEYS)) * (KEYS / 64);
                float L = 0.0f;
                for (int w = 0; w < KEYS / 64; w++) L += lsum[z][p0 + w][tid];
                if (a.sink_on && wg == 0) L += exp_poly(a.sink - smax[z][tid]);  // once per column
                a.part_l[pbase + tid] = L;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Decode pass 2 and the combine in one launch for short caches (one group of
// g <= 8 NCB columns per KV head: the query heads of one row, or MR the (row,
// head) columns of a few rows, each with its row's causal limit; n <=
// kDirectKeys). Workgroup (s, kvh) computes dimensions [DS s, DS s + DS) of
// the g outputs over all n keys (DS = kDirectSlice). Every load is issued
// first: the columns' scores and pass-1 maxima, and the V slice (n rows of 2 DS
// bytes). Then the exact maxima (wave w reduces columns w and w + 8, 32 lanes
// each), the g x n exponentials as P columns in LDS (as decode_pv: [hi of 8 |
// lo of 8] for NCB = 1, a hi and a lo block of 16 for NCB = 2; each slice's
// workgroup computes all of them), the V slice to LDS, P.V with the 32-key
// tiles dealt to the 8 waves, the waves' partial outputs summed in LDS in wave
// order, and out = bf16(O / l), gated like the combine's. Grid (D / DS,
// kv_heads).
// FUSED (the Fused form, one row, NCB = 1, as decode_pv's FUSED over one chunk
// of all the keys): wave h takes head h's block maxima from pass 1, one 16-key
// block per lane, their running maxima M_b by a prefix maximum (exact in any
// order), the corrections P(M_{b-1} - M_b) and each block's product C_b of the
// later blocks' corrections (left to right, from lane broadcasts);
// e = P(s - M_b) * C_b, and out = bf16(O * fl(1/l)).
// ---------------------------------------------------------------------------
template <int D, bool FUSED = false, int NCB = 1, bool MR = false, int DS = kDirectSlice>
__global__ __launch_bounds__(512, 1) void decode_direct(DecodeArgs a)
{
    constexpr int W = 8, THREADS = 64 * W, DBS = DS / 16, NK = kDirectKeys, PS = NK + 8;
    constexpr int R = NK / 256, CH = NK * DS / 8 / THREADS, NT = NK / kKeyTile, NB = NK / 16;
    constexpr int CM = 8 * NCB, HI = CM / 2;                     // columns; per thread parity
    static_assert(D % DS == 0 && NK % 512 == 0 && CH * THREADS * 8 == NK * DS, "slices, rounds, key pairs");
    static_assert(!FUSED || (NB == 64 && NCB == 1 && !MR), "the Fused form: one row, one block of 16 keys per lane");
    __shared__ __attribute__((aligned(16))) uint16_t vs[NK * DS];
    __shared__ __attribute__((aligned(16))) uint16_t pc[2 * CM * PS];
    __shared__ float smax[CM];
    __shared__ float lpart[W][CM];
    __shared__ float ored[W][NCB][DBS][4][64];
    constexpr int FB = FUSED ? 8 * NB : 1;
    __shared__ float fmb[FB], fcf[FB];
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, j = l & 15, G = l >> 4;
    const int kvh = static_cast<int>(blockIdx.y), d0 = static_cast<int>(blockIdx.x) * DS;
    const uint64_t n = a.n;
    const int g = a.g;
    // thread t: keys t % 256 + 256 r, columns t / 256 + 2 i (the same for a
    // whole wave, so the column loops end alike in every lane)
    const int kb = tid % 256, hp = tid / 256;
    float sv[R][HI];
#pragma unroll
    for (int i = 0; i < HI; i++) {
        const int h = hp + 2 * i;
        if (h >= g) break;
        const float *src = a.scores + static_cast<uint64_t>(kvh * g + h) * a.npad;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint64_t key = static_cast<uint64_t>(kb + 256 * r);
            sv[r][i] = src[key < n ? key : 0];
        }
    }
    // the pass-1 maxima of column wave + 8 (l / 32), lane l % 32 taking entry
    // l % 32 (nwg_qk <= NK / 128 <= 32), or (FUSED) head `wave`'s block maxima,
    // one 16-key block per lane (blocks past the cache: -inf, leaving the
    // running maximum as it is)
    const int mcol = wave + 8 * (l >> 5), ml = l & 31;
    const int nbv = static_cast<int>((n + 15) / 16);
    const float mxv = FUSED ? (wave < g && l < nbv ? a.bmax[static_cast<uint64_t>(kvh * g + wave) * a.nblk + l]
                                                   : kNegInf)
                            : (mcol < g && ml < a.nwg_qk
                                   ? a.wgmax[static_cast<uint64_t>(kvh * g + mcol) * a.nwg_qk + ml]
                                   : kNegInf);
    // the V slice: chunk c = tid + THREADS i is key c / (DS / 8), bytes
    // 16 (c % (DS / 8)).. of the slice; keys past the cache read row 0 and are
    // stored as zeros
    const uint16_t *vbase = a.v + static_cast<uint64_t>(kvh) * a.kv_stride + d0;
    u32x4 vr[CH];
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int idx = tid + THREADS * c, key = idx / (DS / 8), part = idx % (DS / 8);
        vr[c] = load16(vbase + static_cast<uint64_t>(static_cast<uint64_t>(key) < n ? key : 0) * D + 8 * part);
    }
    __builtin_amdgcn_sched_barrier(0);                          // all loads issued first
    if constexpr (FUSED) {
        // running maxima: an inclusive prefix maximum over the wave's lanes,
        // by DPP moves (within each 16-lane row by row_shr 1, 2, 4, 8, then
        // row_bcast:15 into rows 1 and 3, row_bcast:31 into rows 2 and 3),
        // and the previous lane's by wave_shr:1; LDS permutes, each waited
        // out by the next step, took longer
        float mb = mxv;
#pragma unroll
        for (int off = 1; off < 16; off *= 2) mb = fmaxnn(mb, row_shr_n(mb, off, kNegInf));
        mb = fmaxnn(mb, dpp<0x142, 0xA>(mb, kNegInf));
        mb = fmaxnn(mb, dpp<0x143, 0xC>(mb, kNegInf));
        const float mprev = dpp<0x138, 0xF>(mb, kNegInf);
        const float cor = l > 0 ? exp_poly(mprev - mb) : 1.0f;
        // C_l = the corrections of blocks l + 1 .. NB - 1 multiplied left to
        // right, each broadcast from its lane in turn
        float c = 1.0f;
#pragma unroll
        for (int k = 1; k < NB; k++) {
            const float ck = lane_value(cor, k);
            c = k > l ? c * ck : c;
        }
        if (wave < g) {
            fmb[wave * NB + l] = mb;
            fcf[wave * NB + l] = c;
        }
    } else {
        float m = group_max_hi(mxv, 32);
        if (a.sink_on) m = m > a.sink ? m : a.sink;             // the sink joins the maximum
        if (ml == 31 && mcol < g) smax[mcol] = m;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < HI; i++) {
        const int h = hp + 2 * i;
        if (h >= g) break;
        // column h's row sees keys [0, past + row] (one row: all n)
        const uint64_t lim = MR ? a.past + static_cast<uint64_t>(h / a.G) + 1 : n;
        float le = 0.0f, er[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int key = kb + 256 * r;
            const bool vis = static_cast<uint64_t>(key) < n && static_cast<uint64_t>(key) < lim;
            float e;
            if constexpr (FUSED) {
                const int fb = h * NB + key / 16;
                e = vis ? exp_poly(sv[r][i] - fmb[fb]) * fcf[fb] : 0.0f;
            } else {
                e = vis ? exp_poly(sv[r][i] - smax[h]) : 0.0f;
            }
            er[r] = e;
            le += e;
        }
        // keys kb + 256 r and kb + 256 (r + 1) split as one pair
#pragma unroll
        for (int r = 0; r < R; r += 2) {
            const int key = kb + 256 * r;
            uint32_t hb, lb;
            split2(er[r], er[r + 1], hb, lb);
            pc[h * PS + key] = static_cast<uint16_t>(hb);
            pc[h * PS + key + 256] = static_cast<uint16_t>(hb >> 16);
            pc[(CM + h) * PS + key] = static_cast<uint16_t>(lb);
            pc[(CM + h) * PS + key + 256] = static_cast<uint16_t>(lb >> 16);
        }
        const float sum = wave_sum_hi(le);
        if (l == 63) lpart[wave][h] = sum;
    }
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int idx = tid + THREADS * c, key = idx / (DS / 8), part = idx % (DS / 8), kk = key % kKeyTile;
        store16(vs + (key / kKeyTile) * (kKeyTile * DS) + kk * DS + 8 * swz16<DS>(kk, part),
                static_cast<uint64_t>(key) < n ? vr[c] : u32x4{0, 0, 0, 0});
    }
    __syncthreads();
    // O^T = V^T . P^T over the tiles t = wave, wave + 8, ..; lane (j, G)
    // holds P column j of each block (NCB = 1: hi of column j, lo of column
    // j - 8; NCB = 2: block 0 hi, block 1 lo of column j), dimensions
    // 4 G .. 4 G + 3 of each 16-dimension block
    const int nt = static_cast<int>((n + kKeyTile - 1) / kKeyTile);
    f32x4 o[NCB][DBS] = {};
#pragma unroll
    for (int k = 0; k < NT / W; k++) {
        const int t = wave + W * k;
        if (t < nt) {
            u32x4 bp[NCB];
#pragma unroll
            for (int c = 0; c < NCB; c++) bp[c] = load16(pc + (16 * c + j) * PS + kKeyTile * t + 8 * G);
#pragma unroll
            for (int db = 0; db < DBS; db++) {
                const u32x4 av = vt16_operand<DS>(vs + t * (kKeyTile * DS), 16 * db, l);
#pragma unroll
                for (int c = 0; c < NCB; c++) o[c][db] = mfma16(av, bp[c], o[c][db]);
            }
        }
    }
#pragma unroll
    for (int c = 0; c < NCB; c++)
#pragma unroll
        for (int db = 0; db < DBS; db++)
#pragma unroll
            for (int r = 0; r < 4; r++) ored[wave][c][db][r][l] = o[c][db][r];
    __syncthreads();
    if (wave == 0) {
        const int h = NCB == 1 ? (j & 7) : j;                   // this lane's column
        const int hc = h < g ? h : 0;
        float L = 0.0f;
        // columns of parity p were summed by waves 4 p .. 4 p + 3
#pragma unroll
        for (int w = 0; w < 4; w++) L += lpart[4 * (hc & 1) + w][hc];
        if (!FUSED && a.sink_on) L += exp_poly(a.sink - smax[hc]);
        // the column's (row, head) and where its output goes
        const int row = MR ? hc / a.G : 0, head = kvh * a.G + hc - row * a.G;
        const uint64_t obase = static_cast<uint64_t>(row) * a.out_row + static_cast<uint64_t>(head) * D + d0 + 4 * G;
        const uint64_t gbase = static_cast<uint64_t>(row) * a.gate_row + static_cast<uint64_t>(head) * D + d0 + 4 * G;
#pragma unroll
        for (int db = 0; db < DBS; db++) {
            f32x4 sum[NCB] = {};
#pragma unroll
            for (int w = 0; w < W; w++)
#pragma unroll
                for (int c = 0; c < NCB; c++)
#pragma unroll
                    for (int r = 0; r < 4; r++) sum[c][r] += ored[w][c][db][r][l];
            uint16_t ob[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                // hi column + lo column
                const float os = NCB == 1 ? sum[0][r] + row_xor8(sum[0][r]) : sum[0][r] + sum[NCB - 1][r];
                ob[r] = static_cast<uint16_t>(cvt_out(FUSED || a.sink_on ? os * (1.0f / L) : os / L));
            }
            if (j < CM && h < g) {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    if (a.gate) ob[r] = gate_bf16(ob[r], a.gate[gbase + 16 * db + r]);
                    a.out[obase + 16 * db + r] = ob[r];
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Decode pass 3: out[h] = bf16(sum_w O_w / sum_w l_w).
// grid (heads, D/64), 512 threads: 64 dimensions x 8 interleaved partial
// subsets; every thread issues all its loads before adding (one round trip
// for up to 8 * 16 partials), and the subsets are summed in a fixed order.
// FUSED: the partials of workgroup w are relative to the running maximum at
// its end; the product S_w of the later workgroups' correction products
// brings them to the last one's (out = sum S_w O_w / sum S_w l_w). S_w comes
// from a suffix product over segments of kFusedMaxSeg workgroups (one per
// thread: lane shuffles within each wave, then the later waves' totals), the
// last segment first. The output is the sum times its reciprocal, as the
// Fused form normalises (decode.rs:653-659).
// ---------------------------------------------------------------------------
constexpr int kCombineSubs = 8;

template <int D, bool MR = false, bool FUSED = false, bool FRAME = false>
__global__ __launch_bounds__(512) void decode_combine(DecodeArgs a)
{
    static_assert(!FRAME || !MR, "frame calls: one row");
    if constexpr (FRAME) {
        bool run;
        const uint32_t st = frame_cfg_load(a, run);
        if (a.f_status && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *a.f_status = st;
        if (!run) return;
    }
    __shared__ float ored[kCombineSubs][64];
    __shared__ float lred[kCombineSubs];
    __shared__ float xs[FUSED ? kFusedMaxSeg : 1];
    __shared__ float wt[FUSED ? kCombineSubs : 1];              // the waves' suffix totals
    static_assert(!FUSED || kFusedMaxSeg == 64 * kCombineSubs, "one scan element per thread");
    const int h = blockIdx.x, kvh = h / a.g, jh = h % a.g;
    const int t = threadIdx.x & 63, sub = threadIdx.x >> 6;
    // D not a multiple of 64: lanes past D in the last block read dimension 0
    // and store nothing
    const bool dok = D % 64 == 0 || static_cast<int>(blockIdx.y * 64 + t) < D;
    const int dim = dok ? blockIdx.y * 64 + t : 0;
    float o = 0.0f, L = 0.0f;
    const uint64_t base = static_cast<uint64_t>(kvh) * a.nwg_pv * a.g + jh;
    constexpr int BATCH = 16;
    if constexpr (FUSED) {
        const int tid = threadIdx.x;
        float carry = 1.0f;                 // product over the workgroups after the segment
        for (int s1 = a.nwg_pv; s1 > 0; s1 -= kFusedMaxSeg) {
            const int s0 = s1 > kFusedMaxSeg ? s1 - kFusedMaxSeg : 0, cnt = s1 - s0;
            // the segment's products first, then its first batch of partials,
            // so that the partials arrive while the products are scanned (one
            // round trip instead of two)
            const float xv = tid < cnt ? a.part_x[base + static_cast<uint64_t>(s0 + tid) * a.g] : 1.0f;
            float xo[BATCH], xl[BATCH];
            auto load_batch = [&](int w0) {
#pragma unroll
                for (int b = 0; b < BATCH; b++) {
                    const int w = w0 + kCombineSubs * b;
                    const uint64_t part = base + static_cast<uint64_t>(w < s1 ? w : s0) * a.g;
                    xo[b] = a.part_o[part * D + dim];
                    xl[b] = a.part_l[part];
                }
            };
            int w0 = s0 + sub;
            load_batch(w0);
            // xs[i] <- the product of the segment's products i .. cnt-1 (the
            // threads past cnt hold 1): a suffix product within each wave by
            // lane shuffles, then times the later waves' totals; a doubling
            // scan in LDS took two barriers per step
            const int lane = tid & 63;
            float p = xv;
#pragma unroll
            for (int off = 1; off < 64; off *= 2) {
                const float y = __shfl_down(p, off);
                p = lane + off < 64 ? p * y : p;
            }
            __syncthreads();                // the previous segment's xs and wt are read
            if (lane == 0) wt[sub] = p;
            __syncthreads();
            float later = 1.0f;
            for (int u = kCombineSubs - 1; u > sub; u--) later = later * wt[u];
            xs[tid] = p * later;
            __syncthreads();
            for (; w0 < s1; w0 += kCombineSubs * BATCH) {
                if (w0 != s0 + sub) load_batch(w0);
#pragma unroll
                for (int b = 0; b < BATCH; b++) {
                    const int i = w0 + kCombineSubs * b - s0;
                    if (i < cnt) {
                        const float S = (i + 1 < cnt ? xs[i + 1] : 1.0f) * carry;
                        o += S * xo[b];
                        L += S * xl[b];
                    }
                }
            }
            carry = carry * xs[0];
        }
    }
    for (int w0 = sub; !FUSED && w0 < a.nwg_pv; w0 += kCombineSubs * BATCH) {
        float xo[BATCH], xl[BATCH];
#pragma unroll
        for (int b = 0; b < BATCH; b++) {
            const int w = w0 + kCombineSubs * b;
            const uint64_t part = base + static_cast<uint64_t>(w < a.nwg_pv ? w : 0) * a.g;
            xo[b] = a.part_o[part * D + dim];
            xl[b] = a.part_l[part];
        }
#pragma unroll
        for (int b = 0; b < BATCH; b++)
            if (w0 + kCombineSubs * b < a.nwg_pv) {
                o += xo[b];
                L += xl[b];
            }
    }
    ored[sub][t] = o;
    if (t == 0) lred[sub] = L;
    __syncthreads();
    if (sub == 0 && dok) {
        float os = 0.0f, ls = 0.0f;
#pragma unroll
        for (int i = 0; i < kCombineSubs; i++) {
            os += ored[i][t];
            ls += lred[i];
        }
        // the Fused form and the sink normalise by the reciprocal (decode.rs:653-659, 280-290)
        uint16_t ob = static_cast<uint16_t>(cvt_out(FUSED || a.sink_on ? os * (1.0f / ls) : os / ls));
        uint64_t oat = static_cast<uint64_t>(h) * D + dim, gat = oat;
        if constexpr (MR) {
            // group kvh = y sub + z; its column jh is column z g + jh of KV head y
            const int y = kvh / a.sub, c = (kvh - y * a.sub) * a.g + jh, row = c / a.G;
            if (c >= a.cols) return;                            // a padded column
            const uint64_t head = static_cast<uint64_t>(y * a.G + c - row * a.G);
            oat = static_cast<uint64_t>(row) * a.out_row + head * D + dim;
            gat = static_cast<uint64_t>(row) * a.gate_row + head * D + dim;
        }
        if (a.gate) ob = gate_bf16(ob, a.gate[gat]);
        a.out[oat] = ob;
    }
}

// ---------------------------------------------------------------------------
// Prefill: the causal attention of a chunk, two passes over the keys in one
// workgroup: the exact row maxima, then exponentials and P.V.
// grid (row groups, heads / HPW), 64 NW threads: NW = 8 waves, two per SIMD
// (D <= 256), or 4, one per SIMD with twice the registers (D > 256). Wave w
// serves query head blockIdx.y * HPW + w % HPW and rows r0 + 32 (w / HPW) ..
// +32, r0 the group's first row; the HPW heads of a workgroup share one KV
// head (HPW = 8 when g is a multiple of 8), so all waves read the same K and V
// tiles from LDS. Tiles are double-buffered: the global loads of tile t+1 are
// in flight while tile t is computed. Tiles below the diagonal of all of a
// wave's rows skip the causal mask.
// POW2 (the scale is a positive power of two): fl(fl(dot * scale) - M) equals
// fl(dot - Mraw) * scale exactly, Mraw being the maximum of the unscaled
// dot products, and the scale folds exactly into the exponential's clamp
// (-87.33654 / scale) and multiplier (log2(e) * scale). Otherwise every score
// is scaled first, as in the reference.
// ---------------------------------------------------------------------------
struct ExpArgs {
    float m;        // POW2: Mraw; otherwise the scaled maximum M
    float scale;    // otherwise: the scale
    float clamp;    // POW2: -87.33654 / scale; otherwise -87.33654
    float mul;      // POW2: 1.442695 * scale; otherwise 1.442695
};

template <bool POW2>
__device__ __forceinline__ float exp_score(float acc, const ExpArgs &x)
{
    const float d = POW2 ? acc - x.m : acc * x.scale - x.m;
    const float t1 = __builtin_fmaxf(d, x.clamp) * x.mul;
    const float t2 = __builtin_rintf(t1);
    const float f = t1 - t2;
    float p = __builtin_fmaf(f, 0.00967248f, 0.05550411f);
    p = __builtin_fmaf(f, p, 0.2402265f);
    p = __builtin_fmaf(f, p, 0.6931472f);
    p = __builtin_fmaf(f, p, 1.0f);
    return __builtin_ldexpf(p, static_cast<int>(t2));
}

// The sink joins a causal row's maximum m (under POW2 the maximum of the
// unscaled dot products, as the kernels keep it): the scaled maximum becomes
// the larger of M and the sink (vmaxss, decode.rs:239-290), returned in ms;
// the result is the maximum the exponentials take, ms / scale under POW2
// (exact for a power of two; a quotient past the f32 range is infinite, and
// every exponential then clamps as the reference's does).
template <bool POW2>
__device__ __forceinline__ float sink_max(float m, const PrefillArgs &a, float &ms)
{
    const float s = POW2 ? m * a.scale : m;
    ms = s > a.sink ? s : a.sink;
    return POW2 ? ms / a.scale : ms;
}

// A row's normalisation: the division by its sum, or (the sink) the
// product with the sum's reciprocal.
struct div_norm {
    float l;
    __device__ __forceinline__ float operator()(float x) const { return x / l; }
};
struct rcp_norm {
    float inv;
    __device__ __forceinline__ float operator()(float x) const { return x * inv; }
};

// The outputs of one row held in the 32x32 accumulators o (lane: row
// col, dimensions 32 dt + 8 c + 4 grp ..), normalised, gated, stored.
template <int D, typename N>
__device__ __forceinline__ void store_rows(const f32x16 *o, uint16_t *op, const uint16_t *gp, int grp, N nrm)
{
#pragma unroll
    for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
        for (int c = 0; c < 4; c++) {
            uint32_t b0 = cvt_out(nrm(o[dt][4 * c])), b1 = cvt_out(nrm(o[dt][4 * c + 1]));
            uint32_t b2 = cvt_out(nrm(o[dt][4 * c + 2])), b3 = cvt_out(nrm(o[dt][4 * c + 3]));
            const int at = 32 * dt + 8 * c + 4 * grp;
            if (gp) {
                const uint2 g = *reinterpret_cast<const uint2 *>(gp + at);
                b0 = gate_bf16(static_cast<uint16_t>(b0), static_cast<uint16_t>(g.x));
                b1 = gate_bf16(static_cast<uint16_t>(b1), static_cast<uint16_t>(g.x >> 16));
                b2 = gate_bf16(static_cast<uint16_t>(b2), static_cast<uint16_t>(g.y));
                b3 = gate_bf16(static_cast<uint16_t>(b3), static_cast<uint16_t>(g.y >> 16));
            }
            *reinterpret_cast<uint2 *>(op + at) = uint2{b0 | (b1 << 16), b2 | (b3 << 16)};
        }
}

template <int D, int HPW, bool POW2, int NW = 8, bool SINK = false>
__global__ __launch_bounds__(64 * NW, 1) void prefill_attn(PrefillArgs a)
{
    constexpr int RB = NW / HPW, THREADS = 64 * NW;
    constexpr int SK = Pad<D>::K, SV = Pad<D>::V;
    __shared__ __attribute__((aligned(16))) uint16_t kb[2][kKeyTile * SK];
    __shared__ __attribute__((aligned(16))) uint16_t vb[2][kKeyTile * SV];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, col = l & 31, grp = l >> 5;
    const int head = blockIdx.y * HPW + (wave % HPW);
    const int kvh = head / a.gqa;
    const uint64_t rgroup = gridDim.x - 1 - blockIdx.x;       // heaviest rows first
    const uint64_t wg_r0 = rgroup * (32 * RB);
    const uint64_t w_r0 = wg_r0 + 32 * (wave / HPW);
    const uint64_t row = w_r0 + col;
    const bool rowv = row < a.rows;
    const bool wact = w_r0 < a.rows;
    const uint64_t wg_rend = wg_r0 + 32 * RB < a.rows ? wg_r0 + 32 * RB : a.rows;
    const int ntiles = static_cast<int>((a.past + wg_rend + kKeyTile - 1) / kKeyTile);
    const int nfull = wact ? static_cast<int>((a.past + w_r0 + 1) / kKeyTile) : 0;  // no mask needed
    const uint64_t lim = a.past + row;                         // last visible key of this row

    const uint16_t *kg = a.k + static_cast<uint64_t>(kvh) * a.kv_stride;
    const uint16_t *vg = a.v + static_cast<uint64_t>(kvh) * a.kv_stride;
    u32x4 kr[Tile<D, THREADS>::kPer], vr[Tile<D, THREADS>::kPer];
    u32x4 qb[D / 16];
    const uint16_t *qp = a.q + (rowv ? row : 0) * a.q_row + static_cast<uint64_t>(head) * a.q_head;
#pragma unroll
    for (int s = 0; s < D / 16; s++) {
        const u32x4 v = load16(qp + 16 * s + 8 * grp);
        qb[s] = rowv ? v : u32x4{0, 0, 0, 0};
    }
    tile_gload<D, THREADS, false>(kg, 0, a.n, tid, kr);
    const int arow = swap23(col) * SK + 8 * grp;
    // One accumulation chain: a second one would not fit the 256 registers
    // of two waves per SIMD; the other wave on the SIMD fills the gaps.
    auto qk = [&](const uint16_t *kt) {
        f32x16 acc = {};
#pragma unroll
        for (int s = 0; s < D / 16; s += 2) {
            // two K operands requested before their MFMAs
            const u32x4 k0 = load16(kt + arow + 16 * s), k1 = load16(kt + arow + 16 * (s + 1));
            acc = mfma(k0, qb[s], acc);
            acc = mfma(k1, qb[s + 1], acc);
        }
        return acc;
    };

    // Every wave computes every tile of the workgroup's key range: tiles past
    // a wave's last visible key take the masked path and contribute nothing.
    // With no wave-dependent branches around them, the loads of the next
    // tiles stay in flight across the compute.

    // pass 1: exact row maxima (of the unscaled dot products when POW2).
    // Out-of-range keys of the last tile read row 0 and are never visible.
    tile_lstore_padded<D, THREADS>(kb[0], SK, tid, kr);
    __syncthreads();
    float m = kNegInf;
    for (int t = 0; t < ntiles; t++) {
        const uint64_t t0 = static_cast<uint64_t>(t) * kKeyTile;
        const bool last = t + 1 == ntiles;
        tile_gload<D, THREADS, false>(kg, last ? 0 : t0 + kKeyTile, a.n, tid, kr);   // after the last: pass 2's first tile
        if (last) tile_gload<D, THREADS, false>(vg, 0, a.n, tid, vr);
        __builtin_amdgcn_sched_barrier(0);
        const f32x16 acc = qk(kb[t & 1]);
        if (t < nfull) {
#pragma unroll
            for (int r = 0; r < 16; r++) m = __builtin_fmaxf(m, POW2 ? acc[r] : acc[r] * a.scale);
        } else {
            // keys t0 + k with k <= vis are visible to this row
            const int vis = static_cast<int>(static_cast<int64_t>(lim) - static_cast<int64_t>(t0));
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float s = POW2 ? acc[r] : acc[r] * a.scale;
                if (key_of(r, grp) <= vis) m = __builtin_fmaxf(m, s);
            }
        }
        if (!last) tile_lstore_padded<D, THREADS>(kb[(t + 1) & 1], SK, tid, kr);
        __syncthreads();
    }
    m = __builtin_fmaxf(m, __shfl_xor(m, 32));
    float ms = 0.0f;                                            // the scaled maximum, with the sink
    if constexpr (SINK) m = sink_max<POW2>(m, a, ms);
    ExpArgs ex;
    ex.m = m;
    ex.scale = a.scale;
    ex.clamp = POW2 ? -87.33654f / a.scale : -87.33654f;
    ex.mul = POW2 ? 1.442695f * a.scale : 1.442695f;

    // pass 2: exponentials at the exact maximum, P.V with P = hi + lo. The
    // next K tile is loaded first, the next V tile after the first half's
    // softmax, so that their staging registers are not live at the peak.
    tile_lstore_padded<D, THREADS>(kb[0], SK, tid, kr);
    tile_mask<D, THREADS>(0, a.n, tid, vr);
    tile_lstore_padded<D, THREADS>(vb[0], SV, tid, vr);
    __syncthreads();
    f32x16 o[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; dt++) o[dt] = f32x16{};
    // the sink's exponential starts the row's sum (in one of its two lanes),
    // so that nothing of it stays live across the tiles
    float lsum = SINK && grp == 0 ? exp_poly(a.sink - ms) : 0.0f;
    for (int t = 0; t < ntiles; t++) {
        const uint64_t t0 = static_cast<uint64_t>(t) * kKeyTile;
        const int b = t & 1;
        tile_gload<D, THREADS, false>(kg, t0 + kKeyTile, a.n, tid, kr);  // past the end: row 0, unused
        __builtin_amdgcn_sched_barrier(0);
        const f32x16 acc = qk(kb[b]);
        const bool full = t < nfull;
        const int vis = static_cast<int>(static_cast<int64_t>(lim) - static_cast<int64_t>(t0));
        // exponentials of one half of the tile's keys as hi and lo operands
        auto half = [&](int h, auto masked, u32x4 &hi, u32x4 &lo) {
            constexpr bool MASKED = decltype(masked)::value;
            float ev[8];
#pragma unroll
            for (int r = 0; r < 8; r++) {
                const float e = exp_score<POW2>(acc[8 * h + r], ex);
                ev[r] = !MASKED || key_of(8 * h + r, grp) <= vis ? e : 0.0f;
                lsum += ev[r];
            }
            split_pack_hw(ev, hi, lo);
        };
        auto pv = [&](int h, const u32x4 &hi, const u32x4 &lo) {
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int dt = 0; dt < D / 32; dt++) {
                const u32x4 av = vt_operand_padded<D>(vb[b], 16 * h, 32 * dt, l);
                o[dt] = mfma(av, hi, o[dt]);
                o[dt] = mfma(av, lo, o[dt]);
            }
            __builtin_amdgcn_s_setprio(0);
        };
        u32x4 hi, lo;
        if (full) half(0, std::false_type{}, hi, lo);
        else half(0, std::true_type{}, hi, lo);
        tile_gload<D, THREADS, false>(vg, t0 + kKeyTile, a.n, tid, vr);
        __builtin_amdgcn_sched_barrier(0);
        pv(0, hi, lo);
        if (full) half(1, std::false_type{}, hi, lo);
        else half(1, std::true_type{}, hi, lo);
        pv(1, hi, lo);
        if (t + 1 < ntiles) {
            tile_lstore_padded<D, THREADS>(kb[b ^ 1], SK, tid, kr);
            tile_mask<D, THREADS>(t0 + kKeyTile, a.n, tid, vr);
            tile_lstore_padded<D, THREADS>(vb[b ^ 1], SV, tid, vr);
        }
        __syncthreads();
    }
    lsum += __shfl_xor(lsum, 32);
    if (rowv) {
        uint16_t *op = a.out + row * a.out_row + static_cast<uint64_t>(head) * D;
        const uint16_t *gp = a.gate ? a.gate + row * a.gate_row + static_cast<uint64_t>(head) * D : nullptr;
        // O / l, or with the sink O times 1 / l
        if constexpr (SINK) store_rows<D>(o, op, gp, grp, rcp_norm{1.0f / lsum});
        else store_rows<D>(o, op, gp, grp, div_norm{lsum});
    }
}

// ---------------------------------------------------------------------------
// Causal prefill of a short chunk, the keys of each row block split among the
// waves of its workgroup: grid (row blocks of 32, heads), KS waves (one per
// SIMD); wave k takes key tiles k, k + KS, ... (at most TPW) of its row block.
// Pass 1 computes their scores once and keeps them in registers (TPW tiles of
// 16 f32 per lane) with the wave's partial row maxima; the waves exchange
// those through LDS into the exact row maximum; pass 2 takes the
// exponentials of the kept scores (P = hi + lo) against V tiles into a
// partial O and l. Each wave then posts its O to LDS and finishes a share of
// the dimensions over all waves' partials, in a fixed order. Numerics follow
// prefill_attn's (exponentials at the exact row maximum, P = hi + lo), with
// Q.K^T in two accumulation chains and each row normalised by its
// reciprocal: other f32 roundings, far below a bf16 ulp.
// Where the one-workgroup causal kernel runs a row block's tiles one after
// the other in every wave, so that the longest row block's tiles are its
// critical path, and the split kernels pass f32 partials through memory,
// this keeps the split inside the workgroup and computes Q.K^T once: for 512
// rows with no cache, at most 4 tiles per wave, in one launch. Each wave
// stages its own tiles (K rows padded to D + 8, V rows to D + 32) and loads
// the next tile while computing this one.
// ---------------------------------------------------------------------------
template <int D, int KS, int TPW, bool POW2>
__global__ __launch_bounds__(64 * KS, 1) void prefill_ks(PrefillArgs a)
{
    constexpr int SK = Pad<D>::K, SV = Pad<D>::V;
    constexpr int TILE_U16 = kKeyTile * (SK + SV);               // one wave's K and V tile
    constexpr int OFLOATS = (D / 32) * 16 * 64;                   // one wave's O partial
    static_assert(KS * TILE_U16 * 2 >= KS * OFLOATS * 4, "the O partials fit the tile buffers");
    __shared__ __attribute__((aligned(16))) uint16_t tiles[KS * TILE_U16];
    __shared__ float mred[KS][32];
    __shared__ float lred[KS][32];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63, col = l & 31, grp = l >> 5;
    const int head = blockIdx.y, kvh = head / a.gqa;
    const uint64_t rb = gridDim.x - 1 - blockIdx.x;             // heaviest row blocks first
    const uint64_t r0 = rb * 32, row = r0 + col;
    const bool rowv = row < a.rows;
    const uint64_t rend = r0 + 32 < a.rows ? r0 + 32 : a.rows;
    const int ntiles = static_cast<int>((a.past + rend + kKeyTile - 1) / kKeyTile);
    const int nfull = static_cast<int>((a.past + r0 + 1) / kKeyTile);   // no mask needed below
    const uint64_t lim = a.past + row;                          // last visible key of this row
    uint16_t *kt = tiles + wave * TILE_U16;
    uint16_t *vt = kt + kKeyTile * SK;

    const uint16_t *kg = a.k + static_cast<uint64_t>(kvh) * a.kv_stride;
    const uint16_t *vg = a.v + static_cast<uint64_t>(kvh) * a.kv_stride;
    // this wave's tiles are its own LDS rows: LDS operations of one wave
    // complete in order, so only the compiler has to be kept from reordering
    auto wave_sync = [&]() {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    u32x4 kr[Tile<D, 64>::kPer], vr[Tile<D, 64>::kPer];
    tile_gload<D, 64, false>(kg, static_cast<uint64_t>(wave) * kKeyTile, a.n, l, kr);

    // pass 1: the scores of this wave's tiles (unscaled dot products when
    // POW2), kept, and their row maxima
    f32x16 sc[TPW];
    float m = kNegInf;
    {
        u32x4 qb[D / 16];
        const uint16_t *qp = a.q + (rowv ? row : 0) * a.q_row + static_cast<uint64_t>(head) * a.q_head;
#pragma unroll
        for (int s = 0; s < D / 16; s++) {
            const u32x4 v = load16(qp + 16 * s + 8 * grp);
            qb[s] = rowv ? v : u32x4{0, 0, 0, 0};
        }
        const int arow = swap23(col) * SK + 8 * grp;
#pragma unroll
        for (int i = 0; i < TPW; i++) {
            const int t = wave + KS * i;
            if (t < ntiles) {
                const uint64_t t0 = static_cast<uint64_t>(t) * kKeyTile;
                tile_lstore_padded<D, 64>(kt, SK, l, kr);
                wave_sync();
                // the next tile's K, or after the last one the first pass-2 V tile
                if (t + KS < ntiles) tile_gload<D, 64, false>(kg, t0 + KS * kKeyTile, a.n, l, kr);
                else tile_gload<D, 64, false>(vg, static_cast<uint64_t>(wave) * kKeyTile, a.n, l, vr);
                // every K operand read issued before the first MFMA: with one
                // wave per SIMD nothing else hides an LDS round trip per MFMA
                u32x4 ka[D / 16];
#pragma unroll
                for (int s = 0; s < D / 16; s++) ka[s] = load16(kt + arow + 16 * s);
                __builtin_amdgcn_sched_barrier(0);
                // two accumulation chains: one wave per SIMD has no other wave
                // to fill a dependent chain's gaps
                f32x16 acc0 = {}, acc1 = {};
#pragma unroll
                for (int s = 0; s < D / 16; s += 2) {
                    acc0 = mfma(ka[s], qb[s], acc0);
                    acc1 = mfma(ka[s + 1], qb[s + 1], acc1);
                }
                const f32x16 acc = acc0 + acc1;
                sc[i] = acc;
                if (t < nfull) {
#pragma unroll
                    for (int r = 0; r < 16; r++) m = __builtin_fmaxf(m, POW2 ? acc[r] : acc[r] * a.scale);
                } else {
                    const int vis = static_cast<int>(static_cast<int64_t>(lim) - static_cast<int64_t>(t0));
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const float x = POW2 ? acc[r] : acc[r] * a.scale;
                        if (key_of(r, grp) <= vis) m = __builtin_fmaxf(m, x);
                    }
                }
                wave_sync();
            }
        }
    }
    // a wave with no tile still loads its (clamped, unused) first V tile
    if (wave >= ntiles) tile_gload<D, 64, false>(vg, 0, a.n, l, vr);
    m = __builtin_fmaxf(m, __shfl_xor(m, 32));
    if (grp == 0) mred[wave][col] = m;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < KS; w++) m = __builtin_fmaxf(m, mred[w][col]);
    // rows past the chunk: a finite maximum, their outputs are never stored
    if (!rowv) m = 0.0f;
    ExpArgs ex;
    ex.m = m;
    ex.scale = a.scale;
    ex.clamp = POW2 ? -87.33654f / a.scale : -87.33654f;
    ex.mul = POW2 ? 1.442695f * a.scale : 1.442695f;

    // pass 2: exponentials of the kept scores at the exact maximum, P.V with
    // P = hi + lo
    f32x16 o[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; dt++) o[dt] = f32x16{};
    float lsum = 0.0f;
#pragma unroll
    for (int i = 0; i < TPW; i++) {
        const int t = wave + KS * i;
        if (t < ntiles) {
            const uint64_t t0 = static_cast<uint64_t>(t) * kKeyTile;
            tile_mask<D, 64>(t0, a.n, l, vr);
            tile_lstore_padded<D, 64>(vt, SV, l, vr);
            wave_sync();
            if (t + KS < ntiles) tile_gload<D, 64, false>(vg, t0 + KS * kKeyTile, a.n, l, vr);
            const bool full = t < nfull;
            const int vis = static_cast<int>(static_cast<int64_t>(lim) - static_cast<int64_t>(t0));
#pragma unroll
            for (int h = 0; h < 2; h++) {
                // the V^T operands of this half are read while its exponentials are computed
                u32x4 av[D / 32];
#pragma unroll
                for (int dt = 0; dt < D / 32; dt++) av[dt] = vt_operand_padded<D>(vt, 16 * h, 32 * dt, l);
                float ev[8];
#pragma unroll
                for (int r = 0; r < 8; r++) {
                    const float e = exp_score<POW2>(sc[i][8 * h + r], ex);
                    ev[r] = full || key_of(8 * h + r, grp) <= vis ? e : 0.0f;
                    lsum += ev[r];
                }
                u32x4 hi, lo;
                split_pack_hw(ev, hi, lo);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int dt = 0; dt < D / 32; dt++) {
                    o[dt] = mfma(av[dt], hi, o[dt]);
                    o[dt] = mfma(av[dt], lo, o[dt]);
                }
            }
            wave_sync();
        }
    }
    lsum += __shfl_xor(lsum, 32);
    if (grp == 0) lred[wave][col] = lsum;
    // every wave posts its O partial; wave w then finishes dimension blocks
    // w, w + KS, ... over the partials of waves 0 .. KS-1 in that order
    float *ox = reinterpret_cast<float *>(tiles);
    __syncthreads();
    {
        float *dst = ox + wave * OFLOATS;
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
            for (int r = 0; r < 16; r++) dst[(dt * 16 + r) * 64 + l] = o[dt][r];
    }
    __syncthreads();
    if (rowv) {
        float L = 0.0f;
#pragma unroll
        for (int w = 0; w < KS; w++) L += lred[w][col];
        // one division per row, then products (one more rounding, far below a
        // bf16 ulp)
        const float inv = 1.0f / L;
        uint16_t *op = a.out + row * a.out_row + static_cast<uint64_t>(head) * D;
        const uint16_t *gp = a.gate ? a.gate + row * a.gate_row + static_cast<uint64_t>(head) * D : nullptr;
        for (int dt = wave; dt < D / 32; dt += KS) {
            float f[16];
#pragma unroll
            for (int r = 0; r < 16; r++) {
                float x = ox[(dt * 16 + r) * 64 + l];
#pragma unroll
                for (int w = 1; w < KS; w++) x += ox[w * OFLOATS + (dt * 16 + r) * 64 + l];
                f[r] = x;
            }
#pragma unroll
            for (int c = 0; c < 4; c++) {
                uint32_t b0 = cvt_out(f[4 * c] * inv), b1 = cvt_out(f[4 * c + 1] * inv);
                uint32_t b2 = cvt_out(f[4 * c + 2] * inv), b3 = cvt_out(f[4 * c + 3] * inv);
                const int at = 32 * dt + 8 * c + 4 * grp;
                if (gp) {
                    const uint2 g = *reinterpret_cast<const uint2 *>(gp + at);
                    b0 = gate_bf16(static_cast<uint16_t>(b0), static_cast<uint16_t>(g.x));
                    b1 = gate_bf16(static_cast<uint16_t>(b1), static_cast<uint16_t>(g.x >> 16));
                    b2 = gate_bf16(static_cast<uint16_t>(b2), static_cast<uint16_t>(g.y));
                    b3 = gate_bf16(static_cast<uint16_t>(b3), static_cast<uint16_t>(g.y >> 16));
                }
                *reinterpret_cast<uint2 *>(op + at) = uint2{b0 | (b1 << 16), b2 | (b3 << 16)};
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Causal prefill of a short chunk, keys split among the waves for the scores
// and dimensions split among them for P.V: grid (row blocks of 32, heads), KS
// waves: 4 (one per SIMD, D >= 128) or 8 (two per SIMD, D = 256). The row
// block's Q is loaded once, a share per wave, and shared through LDS. Pass 1
// is prefill_ks's: wave k computes and keeps the scores of key tiles k,
// k + KS, ... (the next tile's load in flight). After the row maxima are
// exchanged, pass 2 runs in rounds of KS tiles: wave w accumulates O for its
// D / KS dimensions over the round's tiles,
// staging its V slices through its own LDS rows (VPF tiles loaded ahead, the
// next tile's operands read after this one's MFMAs are issued), while the
// exponentials of the next round's tiles (each wave its own, split hi + lo in
// the lanes' operand layout) are computed between those MFMAs and posted to
// LDS for all waves. Every workgroup runs MT tiles (the launch's largest
// count, in whole rounds), the ones past its own fully masked: nothing
// branches on the count. No partial outputs pass between the waves, only the
// row sums (added in wave order). Numerics as prefill_ks.
// ---------------------------------------------------------------------------
template <int S>
__device__ __forceinline__ u32x4 vt_operand_stride(const uint16_t *vtile, int kb, int d0, int l)
{
    const int j = l & 15, G = l >> 4;
    const int key = kb + 8 * (G >> 1) + (j >> 2);
    const int dim = d0 + 16 * (G & 1) + 4 * (j & 3);
    const u32x2 a = tr_read(vtile + key * S + dim);
    const u32x2 b = tr_read(vtile + (key + 4) * S + dim);
    return u32x4{a.x, a.y, b.x, b.y};
}

// DW dimensions [d0, d0 + DW) of a 32-key V tile: 32 * DW/8 chunks of 16
// bytes, lanes on consecutive chunks (each instruction reads whole 2*DW-byte
// row pieces). Keys at or past lim read the tile's first row (or row 0) and are
// zeroed when stored.
template <int DW> struct Slice {
    static constexpr int kPer = kKeyTile * (DW / 8) / 64;
    static_assert(kKeyTile * (DW / 8) % 64 == 0, "whole chunks per lane");
};

template <int D, int DW>
__device__ __forceinline__ void slice_gload(const uint16_t *base, uint64_t t0, uint64_t lim, int d0, int l,
                                            u32x4 (&r)[Slice<DW>::kPer])
{
    const bool any = t0 < lim;
    const uint16_t *tb = base + (any ? t0 : 0) * D + d0;
    const uint32_t nvalid = any ? static_cast<uint32_t>(lim - t0 < kKeyTile ? lim - t0 : kKeyTile) : 0u;
#pragma unroll
    for (int i = 0; i < Slice<DW>::kPer; i++) {
        const int c = l + 64 * i, key = c / (DW / 8), dc = c % (DW / 8);
        const uint32_t off = static_cast<uint32_t>(key) < nvalid ? static_cast<uint32_t>(key * D + 8 * dc) : 0u;
        r[i] = *reinterpret_cast<const u32x4 *>(tb + off);
    }
}

template <int DW, int S>
__device__ __forceinline__ void slice_mask_lstore(uint16_t *st, uint64_t t0, uint64_t lim, int l,
                                                  const u32x4 (&r)[Slice<DW>::kPer])
{
    const uint32_t nvalid = t0 < lim ? static_cast<uint32_t>(lim - t0 < kKeyTile ? lim - t0 : kKeyTile) : 0u;
#pragma unroll
    for (int i = 0; i < Slice<DW>::kPer; i++) {
        const int c = l + 64 * i, key = c / (DW / 8), dc = c % (DW / 8);
        store16(st + key * S + 8 * dc, static_cast<uint32_t>(key) < nvalid ? r[i] : u32x4{0, 0, 0, 0});
    }
}

template <int D, int KS, int MT, int VPF, bool POW2>
__global__ __launch_bounds__(64 * KS, 1) void prefill_kd(PrefillArgs a)
{
    static_assert(KS == 4 || KS == 8, "a round's exponentials are spread over its tiles' products");
    static_assert(MT % KS == 0 && VPF <= MT, "whole rounds");
    static_assert(D / 32 >= KS, "every wave accumulates O for a share of the dimensions");
    constexpr int TPW = MT / KS;                                // rounds; one tile per wave each
    constexpr int SK = Pad<D>::K;
    constexpr int EPT = 16 / KS;                                // next-round exponentials per tile of a round
    constexpr int DW = D / KS;                                  // dimensions per wave
    constexpr int DPW = DW / 32;                                // 32-dimension blocks per wave
    constexpr int SVS = DW + 32;                                // V slice row stride (bf16)
    constexpr int QS = D / 16 / KS;                             // Q chunks each wave loads
    constexpr int KT_U16 = kKeyTile * SK;                       // one wave's K tile
    constexpr int Q_U16 = (D / 16) * 64 * 8;                    // Q in the lanes' operand layout
    // the P operands of two rounds at a time (the round being multiplied and
    // the one being posted): [tile % PR][half][hi, lo][lane] x 8 bf16
    constexpr int PR = MT < 2 * KS ? MT : 2 * KS;
    constexpr int P_U16 = PR * 4 * 64 * 8;
    constexpr int VS_U16 = 2 * kKeyTile * SVS;                  // one wave's two V slices
    constexpr int PASS1 = KS * KT_U16 + Q_U16, PASS2 = P_U16 + KS * VS_U16;
    __shared__ __attribute__((aligned(16))) uint16_t lds[PASS1 > PASS2 ? PASS1 : PASS2];
    __shared__ float mred[KS][32];
    __shared__ float lred[KS][32];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63, col = l & 31, grp = l >> 5;
    const int head = blockIdx.y, kvh = head / a.gqa;
    const uint64_t rb = gridDim.x - 1 - blockIdx.x;             // heaviest row blocks first
    const uint64_t r0 = rb * 32, row = r0 + col;
    const bool rowv = row < a.rows;
    const uint64_t rend = r0 + 32 < a.rows ? r0 + 32 : a.rows;
    // the block's key tiles; every workgroup runs MT (the launch's largest),
    // the ones past its own fully masked, so that nothing branches on the
    // count (a branch makes the later waits wait for every load in flight)
    const uint64_t nblk_keys = a.past + rend;
    const uint64_t nblk = nblk_keys < a.n ? nblk_keys : a.n;   // loads at or past: one clamped address
    const int nfull = static_cast<int>((a.past + r0 + 1) / kKeyTile);   // no mask needed below
    const uint64_t lim = a.past + row;                          // last visible key of this row
    uint16_t *kt = lds + wave * KT_U16;
    uint16_t *qs = lds + KS * KT_U16;
    uint16_t *pbuf = lds;
    uint16_t *vs = lds + P_U16 + wave * VS_U16;
    const int d0 = wave * DW;

    const uint16_t *kg = a.k + static_cast<uint64_t>(kvh) * a.kv_stride;
    const uint16_t *vg = a.v + static_cast<uint64_t>(kvh) * a.kv_stride;
    auto wave_sync = [&]() {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    u32x4 kr[Tile<D, 64>::kPer];
    tile_gload<D, 64, false>(kg, static_cast<uint64_t>(wave) * kKeyTile, nblk, l, kr);
    {
        const uint16_t *qp = a.q + (rowv ? row : 0) * a.q_row + static_cast<uint64_t>(head) * a.q_head;
#pragma unroll
        for (int j = 0; j < QS; j++) {
            const int sq = wave * QS + j;
            const u32x4 v = load16(qp + 16 * sq + 8 * grp);
            store16(qs + (sq * 64 + l) * 8, rowv ? v : u32x4{0, 0, 0, 0});
        }
    }
    lds_barrier();

    // pass 1: the scores of this wave's tiles (unscaled dot products when
    // POW2), kept, and their row maxima
    f32x16 sc[TPW];
    float m = kNegInf;
    {
        u32x4 qb[D / 16];
#pragma unroll
        for (int sq = 0; sq < D / 16; sq++) qb[sq] = load16(qs + (sq * 64 + l) * 8);
        const int arow = swap23(col) * SK + 8 * grp;
#pragma unroll
        for (int i = 0; i < TPW; i++) {
            const int t = wave + KS * i;
            const uint64_t t0 = static_cast<uint64_t>(t) * kKeyTile;
            tile_lstore_padded<D, 64>(kt, SK, l, kr);
            wave_sync();
            if (i + 1 < TPW) tile_gload<D, 64, false>(kg, t0 + KS * kKeyTile, nblk, l, kr);
            // the tile's K operands read before its MFMAs: all at once into two
            // accumulation chains, or, where more than 16 tiles' scores are
            // kept, in two halves into one chain (registers)
            constexpr bool WIDE = MT > 16;
            constexpr int KA = WIDE ? D / 32 : D / 16;
            f32x16 acc0 = {}, acc1 = {};
#pragma unroll
            for (int s0 = 0; s0 < D / 16; s0 += KA) {
                u32x4 ka[KA];
#pragma unroll
                for (int sq = 0; sq < KA; sq++) ka[sq] = load16(kt + arow + 16 * (s0 + sq));
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int sq = 0; sq < KA; sq += 2) {
                    acc0 = mfma(ka[sq], qb[s0 + sq], acc0);
                    if constexpr (WIDE) acc0 = mfma(ka[sq + 1], qb[s0 + sq + 1], acc0);
                    else acc1 = mfma(ka[sq + 1], qb[s0 + sq + 1], acc1);
                }
            }
            const f32x16 acc = WIDE ? acc0 : acc0 + acc1;
            sc[i] = acc;
            const bool full = t < nfull;
            const int vis = static_cast<int>(static_cast<int64_t>(lim) - static_cast<int64_t>(t0));
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float x = POW2 ? acc[r] : acc[r] * a.scale;
                m = __builtin_fmaxf(m, full || key_of(r, grp) <= vis ? x : kNegInf);
            }
            wave_sync();
        }
    }
    // the first VPF V slices of this wave's dimensions, in flight across the
    // exchange and the first round's exponentials
    u32x4 vq[VPF][Slice<DW>::kPer];
#pragma unroll
    for (int j = 0; j < VPF; j++) slice_gload<D, DW>(vg, static_cast<uint64_t>(j) * kKeyTile, nblk, d0, l, vq[j]);
    __builtin_amdgcn_sched_barrier(0);
    m = __builtin_fmaxf(m, __shfl_xor(m, 32));
    if (grp == 0) mred[wave][col] = m;
    lds_barrier();                                              // also: every wave is done with its K tile
#pragma unroll
    for (int w = 0; w < KS; w++) m = __builtin_fmaxf(m, mred[w][col]);
    // rows past the chunk: a finite maximum, their outputs are never stored
    if (!rowv) m = 0.0f;
    ExpArgs ex;
    ex.m = m;
    ex.scale = a.scale;
    ex.clamp = POW2 ? -87.33654f / a.scale : -87.33654f;
    ex.mul = POW2 ? 1.442695f * a.scale : 1.442695f;

    // pass 2. exps_q(r, q): the exponentials of scores 4q .. 4q+3 of this
    // wave's tile of round r at the exact maximum, masked by bits (so that the
    // exponential is not made conditional); after quarters 1 and 3 the half's
    // hi and lo are posted in the lanes' B-operand layout
    float lsum = 0.0f;
    float ev[16];
    // one exponential: score k of this wave's tile of round r
    auto exp_k = [&](int r, int k) {
        const int t = wave + KS * r;
        const uint64_t t0 = static_cast<uint64_t>(t) * kKeyTile;
        const bool full = t < nfull;
        const int vis = static_cast<int>(static_cast<int64_t>(lim) - static_cast<int64_t>(t0));
        const float e = exp_score<POW2>(sc[r][k], ex);
        const uint32_t keep = full || key_of(k, grp) <= vis ? 0xFFFFFFFFu : 0u;
        ev[k] = __uint_as_float(__float_as_uint(e) & keep);
        lsum += ev[k];
    };
    // half h of that tile's exponentials (8 of them), posted
    auto post_half = [&](int r, int h) {
        const int t = wave + KS * r;
        u32x4 hi, lo;
        split_pack_hw(ev + 8 * h, hi, lo);
        store16(pbuf + (((t % PR) * 2 + h) * 2 + 0) * 512 + 8 * l, hi);
        store16(pbuf + (((t % PR) * 2 + h) * 2 + 1) * 512 + 8 * l, lo);
    };
    auto exps_q = [&](int r, int q) {
#pragma unroll
        for (int k = 4 * q; k < 4 * q + 4; k++) exp_k(r, k);
        if (q & 1) post_half(r, q >> 1);
    };
    u32x4 p[4], av[2][DPW];
    auto read_p = [&](int t) {
#pragma unroll
        for (int j = 0; j < 4; j++) p[j] = load16(pbuf + ((t % PR) * 4 + j) * 512 + 8 * l);
    };
    // tile t's V slice (vq[t % VPF]) to its staging rows, its V^T operands
    // read back, the slice VPF tiles on requested in its registers
    auto stage = [&](int t) {
        uint16_t *st = vs + (t & 1) * kKeyTile * SVS;
        slice_mask_lstore<DW, SVS>(st, static_cast<uint64_t>(t) * kKeyTile, nblk, l, vq[t % VPF]);
        wave_sync();
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int dt = 0; dt < DPW; dt++) av[h][dt] = vt_operand_stride<SVS>(st, 16 * h, 32 * dt, l);
        if (t + VPF < MT) slice_gload<D, DW>(vg, static_cast<uint64_t>(t + VPF) * kKeyTile, nblk, d0, l, vq[t % VPF]);
    };
#pragma unroll
    for (int q = 0; q < 4; q++) exps_q(0, q);
    stage(0);
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();                                              // round 0's P posted
    read_p(0);
    f32x16 o[DPW];
#pragma unroll
    for (int dt = 0; dt < DPW; dt++) o[dt] = f32x16{};
#pragma unroll
    for (int r = 0; r < TPW; r++) {
#pragma unroll
        for (int j = 0; j < KS; j++) {
            const int t = KS * r + j;
            // this tile's products, one exponential of the next round issued
            // after each of the first EPT, while the matrix core runs it (the
            // order pinned: the scheduler would group them)
            __builtin_amdgcn_sched_barrier(0);
            int e_at = 0;
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int hl = 0; hl < 2; hl++)
#pragma unroll
                    for (int dt = 0; dt < DPW; dt++) {
                        o[dt] = mfma(av[h][dt], p[2 * h + hl], o[dt]);
                        __builtin_amdgcn_sched_barrier(0);
                        if (r + 1 < TPW && e_at < EPT) {
                            exp_k(r + 1, EPT * j + e_at);
                            __builtin_amdgcn_sched_barrier(0);
                        }
                        e_at++;
                    }
#pragma unroll
            for (; e_at < EPT; e_at++)
                if (r + 1 < TPW) exp_k(r + 1, EPT * j + e_at);
            // a half's eight exponentials are complete after tiles KS/2 - 1 and KS - 1
            if (r + 1 < TPW && (j + 1) % (KS / 2) == 0) post_half(r + 1, j / (KS / 2));
            __builtin_amdgcn_sched_barrier(0);
            if (t + 1 < MT) {
                stage(t + 1);
                if (j + 1 < KS) read_p(t + 1);
            }
        }
        if (r + 1 < TPW) {
            __builtin_amdgcn_sched_barrier(0);
            lds_barrier();                                      // round r + 1's P posted
            read_p(KS * (r + 1));
        }
    }
    lsum += __shfl_xor(lsum, 32);
    if (grp == 0) lred[wave][col] = lsum;
    lds_barrier();
    if (!rowv) return;
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < KS; w++) L += lred[w][col];
    const float inv = 1.0f / L;
    uint16_t *op = a.out + row * a.out_row + static_cast<uint64_t>(head) * D + d0;
    const uint16_t *gp = a.gate ? a.gate + row * a.gate_row + static_cast<uint64_t>(head) * D + d0 : nullptr;
#pragma unroll
    for (int dt = 0; dt < DPW; dt++)
#pragma unroll
        for (int c = 0; c < 4; c++) {
            uint32_t b0 = cvt_out(o[dt][4 * c] * inv), b1 = cvt_out(o[dt][4 * c + 1] * inv);
            uint32_t b2 = cvt_out(o[dt][4 * c + 2] * inv), b3 = cvt_out(o[dt][4 * c + 3] * inv);
            const int at = 32 * dt + 8 * c + 4 * grp;
            if (gp) {
                const uint2 g = *reinterpret_cast<const uint2 *>(gp + at);
                b0 = gate_bf16(static_cast<uint16_t>(b0), static_cast<uint16_t>(g.x));
                b1 = gate_bf16(static_cast<uint16_t>(b1), static_cast<uint16_t>(g.x >> 16));
                b2 = gate_bf16(static_cast<uint16_t>(b2), static_cast<uint16_t>(g.y));
                b3 = gate_bf16(static_cast<uint16_t>(b3), static_cast<uint16_t>(g.y >> 16));
            }
            *reinterpret_cast<uint2 *>(op + at) = uint2{b0 | (b1 << 16), b2 | (b3 << 16)};
        }
}

// ---------------------------------------------------------------------------
// Causal prefill split over the keys, for chunks whose grid of (row group,
// head group) workgroups leaves compute units idle (a short chunk after a long
// cache): gridDim.z workgroups share a row group's key tiles, tile range
// [z per, (z + 1) per) of its ntiles, per = ceil(ntiles / gridDim.z).
//   prefill_split_max     pass 1 over the range: partial row maxima
//                         smax[z][head][row] (-inf where the range holds no
//                         visible key)
//   prefill_split_pv      the exact row maximum (the largest partial: max is
//                         exact in any order, so the exponentials are those of
//                         the one-workgroup kernel), then pass 2 over the range:
//                         unnormalised so[z][row][head][D] and sl[z][row][head]
//   prefill_split_combine out = bf16(sum_z O / sum_z l), z ascending (+ gate)
// Same waves, tiles and numerics as prefill_attn.
// The paired form (PAIRED, grid (R row groups, head groups), one round of
// the compute units; prefill_pairs): in the P.V pass workgroup i < j = R - 1 -
// i walks the whole of row group i (output written directly), then the last h
// tiles of row group j (slot 1); workgroup j walks the rest of row group j
// (slot 0). Its maxima pass runs as the even split in two (grid (R, head
// groups, 2)). The combine serves the rows of the split row groups only.
// ---------------------------------------------------------------------------
struct SplitArgs {
    float *smax;            // [slots][heads][rows]
    float *so;              // [slots][srows][heads][D]: rows r0 .. r0 + srows - 1
    float *sl;              // [slots][srows][heads]
    int heads;
    uint64_t r0, srows;     // the rows with partials (the even split: all rows)
};

// The split kernels' workgroup (row group x, head group y, split z). When the
// (head group, split) pairs are a multiple of 8, the row groups of one pair go
// to one XCD (workgroup i runs on XCD i % 8), where they walk the same key
// tiles and its L2 serves all but the first (256 rows after 32K: 5 % faster).
struct SplitIds {
    int x, y, z;
    __device__ __forceinline__ SplitIds()
    {
        const int gx = gridDim.x, gy = gridDim.y, gz = gridDim.z, C = gy * gz;
        x = blockIdx.x; y = blockIdx.y; z = blockIdx.z;
        if (C % 8 == 0) {
            const int L = x + gx * (y + gy * z), xcd = L & 7, k = L >> 3, c = xcd + 8 * (k / gx);
            x = k % gx; y = c % gy; z = c / gy;
        }
    }
};

// A split workgroup's key ranges, walked in turn: row group rg, tiles
// [tb, te), partial slot (-1: the row group's whole range, its output
// written directly). One range under the even split, one or two paired.
struct SplitSeg {
    int rg, tb, te, slot;
};

template <bool PAIRED>
struct SplitSegs {
    int n;
    SplitSeg s0, s1;
    __device__ __forceinline__ SplitSegs(const PrefillArgs &a, const SplitIds &sid, uint64_t rpw)
    {
        const int R = static_cast<int>(gridDim.x);
        s1 = SplitSeg{0, 0, 0, -1};
        if constexpr (!PAIRED) {
            const int rg = R - 1 - sid.x;                          // heaviest rows first
            const int ntiles = static_cast<int>(causal_tiles(a.past, a.rows, rg, rpw));
            const int nz = static_cast<int>(gridDim.z), per = (ntiles + nz - 1) / nz;
            const int tb = sid.z * per < ntiles ? sid.z * per : ntiles;
            n = 1;
            s0 = SplitSeg{rg, tb, tb + per < ntiles ? tb + per : ntiles, sid.z};
        } else {
            // every workgroup starts at tile 0, so that the workgroups of a KV
            // head on one XCD walk the same tiles at about the same time and
            // its L2 serves all but the first; the light ones then walk the
            // last tiles of their partners' row groups
            const int i = sid.x < R - 1 - sid.x ? sid.x : R - 1 - sid.x, j = R - 1 - i;
            const int ti = static_cast<int>(causal_tiles(a.past, a.rows, i, rpw));
            const int tj = static_cast<int>(causal_tiles(a.past, a.rows, j, rpw));
            const int h = i < j ? static_cast<int>(pair_share(ti, tj)) : 0;
            if (sid.x == i) {
                n = h > 0 ? 2 : 1;
                s0 = SplitSeg{i, 0, ti, -1};
                s1 = SplitSeg{j, tj - h, tj, 1};
            } else {
                n = 1;
                s0 = SplitSeg{j, 0, tj - h, h > 0 ? 0 : -1};
            }
        }
    }
};

template <int D, int HPW, bool POW2, int NW, bool PAIRED = false>
__global__ __launch_bounds__(64 * NW, 1) void prefill_split_max(PrefillArgs a, SplitArgs sp)
{
    constexpr int RB = NW / HPW, THREADS = 64 * NW;
    constexpr int SK = Pad<D>::K;
    __shared__ __attribute__((aligned(16))) uint16_t kb[2][kKeyTile * SK];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, col = l & 31, grp = l >> 5;
    const SplitIds sid;
    const int head = sid.y * HPW + (wave % HPW);
    const int kvh = head / a.gqa;
    const SplitSegs<PAIRED> segs(a, sid, 32 * RB);
    const uint16_t *kg = a.k + static_cast<uint64_t>(kvh) * a.kv_stride;
    const int arow = swap23(col) * SK + 8 * grp;
    // one key range, then (paired) the second: the body is instantiated for
    // each, so that no register stays live from one to the other
    auto run = [&](const SplitSeg sg) {
        const uint64_t wg_r0 = static_cast<uint64_t>(sg.rg) * (32 * RB);
        const uint64_t w_r0 = wg_r0 + 32 * (wave / HPW);
        const uint64_t row = w_r0 + col;
        const bool rowv = row < a.rows;
        const bool wact = w_r0 < a.rows;
        const int nfull = wact ? static_cast<int>((a.past + w_r0 + 1) / kKeyTile) : 0;
        const uint64_t lim = a.past + row;
        const int tb = sg.tb, te = sg.te;

        u32x4 kr[Tile<D, THREADS>::kPer];
        u32x4 qb[D / 16];
        const uint16_t *qp = a.q + (rowv ? row : 0) * a.q_row + static_cast<uint64_t>(head) * a.q_head;
#pragma unroll
        for (int s = 0; s < D / 16; s++) {
            const u32x4 v = load16(qp + 16 * s + 8 * grp);
            qb[s] = rowv ? v : u32x4{0, 0, 0, 0};
        }
        float m = kNegInf;
        if (tb < te) {
            tile_gload<D, THREADS, false>(kg, static_cast<uint64_t>(tb) * kKeyTile, a.n, tid, kr);
            tile_lstore_padded<D, THREADS>(kb[0], SK, tid, kr);
            __syncthreads();
            // as prefill_attn's pass 1: the next tile's load is not branched
            // around (past the cache it reads row 0, unused)
            for (int t = tb; t < te; t++) {
                const uint64_t t0 = static_cast<uint64_t>(t) * kKeyTile;
                tile_gload<D, THREADS, false>(kg, t0 + kKeyTile, a.n, tid, kr);
                __builtin_amdgcn_sched_barrier(0);
                const uint16_t *kt = kb[(t - tb) & 1];
                f32x16 acc = {};
#pragma unroll
                for (int s = 0; s < D / 16; s += 2) {
                    // two K operands requested before their MFMAs
                    const u32x4 k0 = load16(kt + arow + 16 * s), k1 = load16(kt + arow + 16 * (s + 1));
                    acc = mfma(k0, qb[s], acc);
                    acc = mfma(k1, qb[s + 1], acc);
                }
                if (t < nfull) {
#pragma unroll
                    for (int r = 0; r < 16; r++) m = __builtin_fmaxf(m, POW2 ? acc[r] : acc[r] * a.scale);
                } else {
                    const int vis = static_cast<int>(static_cast<int64_t>(lim) - static_cast<int64_t>(t0));
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const float s = POW2 ? acc[r] : acc[r] * a.scale;
                        if (key_of(r, grp) <= vis) m = __builtin_fmaxf(m, s);
                    }
                }
                if (t + 1 < te) tile_lstore_padded<D, THREADS>(kb[(t - tb + 1) & 1], SK, tid, kr);
                __syncthreads();
            }
        }
        m = __builtin_fmaxf(m, __shfl_xor(m, 32));
        const int slot = sg.slot < 0 ? 0 : sg.slot;
        if (rowv && grp == 0) sp.smax[(static_cast<uint64_t>(slot) * sp.heads + head) * a.rows + row] = m;
    };
    run(segs.s0);
    if (PAIRED && segs.n > 1) run(segs.s1);
}

template <int D, int HPW, bool POW2, int NW, bool PAIRED = false, bool SINK = false>
__global__ __launch_bounds__(64 * NW, 1) void prefill_split_pv(PrefillArgs a, SplitArgs sp)
{
    constexpr int RB = NW / HPW, THREADS = 64 * NW;
    constexpr int SK = Pad<D>::K, SV = Pad<D>::V;
    __shared__ __attribute__((aligned(16))) uint16_t kb[2][kKeyTile * SK];
    __shared__ __attribute__((aligned(16))) uint16_t vb[2][kKeyTile * SV];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, col = l & 31, grp = l >> 5;
    const SplitIds sid;
    const int head = sid.y * HPW + (wave % HPW);
    const int kvh = head / a.gqa;
    const SplitSegs<PAIRED> segs(a, sid, 32 * RB);
    const uint16_t *kg = a.k + static_cast<uint64_t>(kvh) * a.kv_stride;
    const uint16_t *vg = a.v + static_cast<uint64_t>(kvh) * a.kv_stride;
    const int arow = swap23(col) * SK + 8 * grp;
    auto run = [&](const SplitSeg sg, auto direct_t) {
        constexpr bool DIRECT = decltype(direct_t)::value;   // a whole row group: output written directly
        const uint64_t wg_r0 = static_cast<uint64_t>(sg.rg) * (32 * RB);
        const uint64_t w_r0 = wg_r0 + 32 * (wave / HPW);
        const uint64_t row = w_r0 + col;
        const bool rowv = row < a.rows;
        const bool wact = w_r0 < a.rows;
        const int nfull = wact ? static_cast<int>((a.past + w_r0 + 1) / kKeyTile) : 0;
        const uint64_t lim = a.past + row;
        const int tb = sg.tb, te = sg.te;

        // the exact row maximum: the largest of the partial maxima (rows past
        // the chunk take 0: computed, never stored); paired, every row's two
        // halves are in slots 0 and 1
        float m = rowv ? kNegInf : 0.0f;
        if (rowv) {
            const int nz = PAIRED ? 2 : static_cast<int>(gridDim.z);   // paired: the maxima pass's two halves
            for (int z = 0; z < nz; z++)
                m = __builtin_fmaxf(m, sp.smax[(static_cast<uint64_t>(z) * sp.heads + head) * a.rows + row]);
        }
        float ms = 0.0f;                                        // the scaled maximum, with the sink
        if constexpr (SINK) m = sink_max<POW2>(m, a, ms);
        ExpArgs ex;
        ex.m = m;
        ex.scale = a.scale;
        ex.clamp = POW2 ? -87.33654f / a.scale : -87.33654f;
        ex.mul = POW2 ? 1.442695f * a.scale : 1.442695f;

        u32x4 kr[Tile<D, THREADS>::kPer], vr[Tile<D, THREADS>::kPer];
        u32x4 qb[D / 16];
        const uint16_t *qp = a.q + (rowv ? row : 0) * a.q_row + static_cast<uint64_t>(head) * a.q_head;
#pragma unroll
        for (int s = 0; s < D / 16; s++) {
            const u32x4 v = load16(qp + 16 * s + 8 * grp);
            qb[s] = rowv ? v : u32x4{0, 0, 0, 0};
        }
        f32x16 o[D / 32];
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++) o[dt] = f32x16{};
        // the sink's exponential, once per row: it starts the sum of the whole
        // range's or of slot 0's (in one lane of two)
        float lsum = SINK && (DIRECT || sg.slot == 0) && grp == 0 ? exp_poly(a.sink - ms) : 0.0f;
        if (tb < te) {
            tile_gload<D, THREADS, false>(kg, static_cast<uint64_t>(tb) * kKeyTile, a.n, tid, kr);
            tile_gload<D, THREADS, false>(vg, static_cast<uint64_t>(tb) * kKeyTile, a.n, tid, vr);
            tile_lstore_padded<D, THREADS>(kb[0], SK, tid, kr);
            tile_mask<D, THREADS>(static_cast<uint64_t>(tb) * kKeyTile, a.n, tid, vr);
            tile_lstore_padded<D, THREADS>(vb[0], SV, tid, vr);
            __syncthreads();
            // as prefill_attn's pass 2: loads not branched around, the masked
            // and unmasked halves of a tile instantiated apart, the P.V MFMAs
            // at raised priority
            for (int t = tb; t < te; t++) {
                const uint64_t t0 = static_cast<uint64_t>(t) * kKeyTile;
                const int b = (t - tb) & 1;
                tile_gload<D, THREADS, false>(kg, t0 + kKeyTile, a.n, tid, kr);  // past the cache: row 0, unused
                __builtin_amdgcn_sched_barrier(0);
                f32x16 acc = {};
#pragma unroll
                for (int s = 0; s < D / 16; s += 2) {
                    // two K operands requested before their MFMAs
                    const u32x4 k0 = load16(kb[b] + arow + 16 * s), k1 = load16(kb[b] + arow + 16 * (s + 1));
                    acc = mfma(k0, qb[s], acc);
                    acc = mfma(k1, qb[s + 1], acc);
                }
                const bool full = t < nfull;
                const int vis = static_cast<int>(static_cast<int64_t>(lim) - static_cast<int64_t>(t0));
                auto half = [&](int h, auto masked, u32x4 &hi, u32x4 &lo) {
                    constexpr bool MASKED = decltype(masked)::value;
                    float ev[8];
#pragma unroll
                    for (int r = 0; r < 8; r++) {
                        const float e = exp_score<POW2>(acc[8 * h + r], ex);
                        ev[r] = !MASKED || key_of(8 * h + r, grp) <= vis ? e : 0.0f;
                        lsum += ev[r];
                    }
                    split_pack_hw(ev, hi, lo);
                };
                auto pv = [&](int h, const u32x4 &hi, const u32x4 &lo) {
                    __builtin_amdgcn_s_setprio(1);
#pragma unroll
                    for (int dt = 0; dt < D / 32; dt++) {
                        const u32x4 av = vt_operand_padded<D>(vb[b], 16 * h, 32 * dt, l);
                        o[dt] = mfma(av, hi, o[dt]);
                        o[dt] = mfma(av, lo, o[dt]);
                    }
                    __builtin_amdgcn_s_setprio(0);
                };
                u32x4 hi, lo;
                if (full) half(0, std::false_type{}, hi, lo);
                else half(0, std::true_type{}, hi, lo);
                tile_gload<D, THREADS, false>(vg, t0 + kKeyTile, a.n, tid, vr);
                __builtin_amdgcn_sched_barrier(0);
                pv(0, hi, lo);
                if (full) half(1, std::false_type{}, hi, lo);
                else half(1, std::true_type{}, hi, lo);
                pv(1, hi, lo);
                if (t + 1 < te) {
                    tile_lstore_padded<D, THREADS>(kb[b ^ 1], SK, tid, kr);
                    tile_mask<D, THREADS>(t0 + kKeyTile, a.n, tid, vr);
                    tile_lstore_padded<D, THREADS>(vb[b ^ 1], SV, tid, vr);
                }
                __syncthreads();
            }
        }
        lsum += __shfl_xor(lsum, 32);
        if (!rowv) return;
        if constexpr (DIRECT) {
            // a whole row group: its output, as prefill_attn writes it
            uint16_t *op = a.out + row * a.out_row + static_cast<uint64_t>(head) * D;
            const uint16_t *gp = a.gate ? a.gate + row * a.gate_row + static_cast<uint64_t>(head) * D : nullptr;
            if constexpr (SINK) store_rows<D>(o, op, gp, grp, rcp_norm{1.0f / lsum});
            else store_rows<D>(o, op, gp, grp, div_norm{lsum});
        } else {
            const uint64_t cell = (static_cast<uint64_t>(sg.slot) * sp.srows + (row - sp.r0)) * sp.heads + head;
            float *op = sp.so + cell * D;
#pragma unroll
            for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
                for (int c = 0; c < 4; c++)
                    *reinterpret_cast<f32x4 *>(op + 32 * dt + 8 * c + 4 * grp) =
                        f32x4{o[dt][4 * c], o[dt][4 * c + 1], o[dt][4 * c + 2], o[dt][4 * c + 3]};
            if (grp == 0) sp.sl[cell] = lsum;
        }
    };
    if constexpr (PAIRED) {
        // a light workgroup: its row group whole, then its partner's tail
        if (segs.s0.slot < 0) run(segs.s0, std::true_type{});
        else run(segs.s0, std::false_type{});
        if (segs.n > 1) run(segs.s1, std::false_type{});
    } else {
        run(segs.s0, std::false_type{});
    }
}

// grid (rows with partials, heads), D threads: one output element each.
template <int D>
__global__ __launch_bounds__(D) void prefill_split_combine(PrefillArgs a, SplitArgs sp, int splits);
// The wide combine's shape: DL lanes of 4 dimensions each, SUBS subsets of
// the splits; it takes more than kCombineNarrowSplits splits (2 splits of the
// paired form: 21.0 us with a thread per dimension, 35.6 us this way).
template <int D> struct CombineShape {
    static constexpr int DL = D / 4, SUBS = 256 / DL > 0 ? 256 / DL : 1, THREADS = DL * SUBS;
};
constexpr int kCombineNarrowSplits = 4;
template <int D>
__global__ __launch_bounds__(CombineShape<D>::THREADS) void prefill_split_combine_wide(PrefillArgs a, SplitArgs sp,
                                                                                       int splits);

// A positive power of two in [2^-20, 2^20]: scaling by it is exact for the
// scores and for the folded exponential constants.
static bool scale_is_pow2(float s)
{
    const uint32_t b = __builtin_bit_cast(uint32_t, s);
    const uint32_t e = (b >> 23) & 0xFF;
    return (b & 0x807FFFFFu) == 0 && e >= 127 - 20 && e <= 127 + 20;
}

// The three split kernels on grid (row groups, head groups, splits). POW2:
// whether a power-of-two scale takes the folded form (the general form rounds
// identically).
template <int D, int HPW, int NW, bool POW2_FORM = true, bool SINK = false>
static hipError_t launch_prefill_split(const PrefillArgs &a, int heads, const PrefillSplit &ps, dim3 grid, int splits,
                                       hipStream_t s)
{
    const SplitArgs sp{ps.smax, ps.so, ps.sl, heads, 0, a.rows};
    const dim3 gs(grid.x, grid.y, static_cast<unsigned>(splits));
    hipError_t e;
    if (POW2_FORM && scale_is_pow2(a.scale)) {
        e = launch(prefill_split_max<D, HPW, POW2_FORM, NW>, gs, dim3(64 * NW), s, a, sp);
        if (e == hipSuccess) e = launch(prefill_split_pv<D, HPW, POW2_FORM, NW, false, SINK>, gs, dim3(64 * NW), s, a, sp);
    } else {
        e = launch(prefill_split_max<D, HPW, false, NW>, gs, dim3(64 * NW), s, a, sp);
        if (e == hipSuccess) e = launch(prefill_split_pv<D, HPW, false, NW, false, SINK>, gs, dim3(64 * NW), s, a, sp);
    }
    if (e != hipSuccess) return e;
    const dim3 gc(static_cast<unsigned>(a.rows), heads);
    return splits > kCombineNarrowSplits
               ? launch(prefill_split_combine_wide<D>, gc, dim3(CombineShape<D>::THREADS), s, a, sp, splits)
               : launch(prefill_split_combine<D>, gc, dim3(D), s, a, sp, splits);
}

// The paired form on the causal kernel's grid (row groups, head groups); pr
// from prefill_pairs.
template <int D, int HPW, int NW, bool POW2_FORM = true, bool SINK = false>
static hipError_t launch_prefill_paired(const PrefillArgs &a, int heads, const PrefillSplit &ps, dim3 grid,
                                        const PairRows &pr, hipStream_t s)
{
    const SplitArgs sp{ps.smax, ps.so, ps.sl, heads, pr.r0, pr.srows};
    // the maxima pass takes every row group's tiles in two halves (slots 0
    // and 1 of every row), twice the workgroups of the pairs: two per CU, four
    // waves per SIMD, where the pairs' one per CU left the K operand reads'
    // latency exposed; the P.V pass takes the larger of the two
    const dim3 gmax(grid.x, grid.y, 2);
    hipError_t e;
    if (POW2_FORM && scale_is_pow2(a.scale)) {
        e = launch(prefill_split_max<D, HPW, POW2_FORM, NW, false>, gmax, dim3(64 * NW), s, a, sp);
        if (e == hipSuccess)
            e = launch(prefill_split_pv<D, HPW, POW2_FORM, NW, true, SINK>, grid, dim3(64 * NW), s, a, sp);
    } else {
        e = launch(prefill_split_max<D, HPW, false, NW, false>, gmax, dim3(64 * NW), s, a, sp);
        if (e == hipSuccess) e = launch(prefill_split_pv<D, HPW, false, NW, true, SINK>, grid, dim3(64 * NW), s, a, sp);
    }
    if (e != hipSuccess) return e;
    return launch(prefill_split_combine<D>, dim3(static_cast<unsigned>(pr.srows), heads), dim3(D), s, a, sp, 2);
}

template <int D>
__global__ __launch_bounds__(D) void prefill_split_combine(PrefillArgs a, SplitArgs sp, int splits)
{
    const uint64_t row = sp.r0 + blockIdx.x, head = blockIdx.y;
    const int dim = threadIdx.x;
    float o = 0.0f, ls = 0.0f;
    for (int z = 0; z < splits; z++) {
        const uint64_t cell = (static_cast<uint64_t>(z) * sp.srows + blockIdx.x) * sp.heads + head;
        o += sp.so[cell * D + dim];
        ls += sp.sl[cell];
    }
    uint16_t ob = static_cast<uint16_t>(cvt_out(a.sink_on ? o * (1.0f / ls) : o / ls));   // the sink: O times 1 / l
    if (a.gate) ob = gate_bf16(ob, a.gate[row * a.gate_row + head * D + dim]);
    a.out[row * a.out_row + head * D + dim] = ob;
}

// The combine for many splits (more than kCombineNarrowSplits).
template <int D>
__global__ __launch_bounds__(CombineShape<D>::THREADS) void prefill_split_combine_wide(PrefillArgs a, SplitArgs sp,
                                                                                       int splits)
{
    // lane t of subset u: dimensions 4 t .. 4 t + 3 of the splits u, u + SUBS,
    // .., B of them requested at a time; the subsets' sums then added in
    // subset order (with at most SUBS splits, the plain split order). One
    // 4-byte load per split in turn left too few bytes in flight: 128 splits
    // of 17 rows after 32K keys (36 MB of partials) took 36.6 us.
    constexpr int DL = CombineShape<D>::DL, SUBS = CombineShape<D>::SUBS, B = 8;
    __shared__ float4 ored[SUBS][DL];
    __shared__ float lred[SUBS];
    const uint64_t row = sp.r0 + blockIdx.x, head = blockIdx.y;
    const int t = static_cast<int>(threadIdx.x) % DL, u = static_cast<int>(threadIdx.x) / DL;
    float o[4] = {0.0f, 0.0f, 0.0f, 0.0f}, ls = 0.0f;
    for (int z0 = u; z0 < splits; z0 += SUBS * B) {
        float4 xo[B];
        float xl[B];
#pragma unroll
        for (int b = 0; b < B; b++) {
            const int z = z0 + SUBS * b;
            if (z < splits) {
                const uint64_t cell = (static_cast<uint64_t>(z) * sp.srows + blockIdx.x) * sp.heads + head;
                xo[b] = *reinterpret_cast<const float4 *>(sp.so + cell * D + 4 * t);
                xl[b] = sp.sl[cell];
            }
        }
#pragma unroll
        for (int b = 0; b < B; b++)
            if (z0 + SUBS * b < splits) {
                o[0] += xo[b].x;
                o[1] += xo[b].y;
                o[2] += xo[b].z;
                o[3] += xo[b].w;
                ls += xl[b];
            }
    }
    ored[u][t] = float4{o[0], o[1], o[2], o[3]};
    if (t == 0) lred[u] = ls;
    __syncthreads();
    if (u != 0) return;
    float4 sum = ored[0][t];
    float L = lred[0];
    for (int v = 1; v < SUBS; v++) {
        const float4 x = ored[v][t];
        sum.x += x.x;
        sum.y += x.y;
        sum.z += x.z;
        sum.w += x.w;
        L += lred[v];
    }
    const float sv[4] = {sum.x, sum.y, sum.z, sum.w};
    uint16_t ob[4];
    if (a.sink_on) {
        const float inv = 1.0f / L;                             // the sink: O times 1 / l
#pragma unroll
        for (int r = 0; r < 4; r++) ob[r] = static_cast<uint16_t>(cvt_out(sv[r] * inv));
    } else {
#pragma unroll
        for (int r = 0; r < 4; r++) ob[r] = static_cast<uint16_t>(cvt_out(sv[r] / L));
    }
    if (a.gate) {
        const uint2 gw = *reinterpret_cast<const uint2 *>(a.gate + row * a.gate_row + head * D + 4 * t);
        const uint16_t gv[4] = {static_cast<uint16_t>(gw.x), static_cast<uint16_t>(gw.x >> 16),
                                static_cast<uint16_t>(gw.y), static_cast<uint16_t>(gw.y >> 16)};
#pragma unroll
        for (int r = 0; r < 4; r++) ob[r] = gate_bf16(ob[r], gv[r]);
    }
    *reinterpret_cast<uint2 *>(a.out + row * a.out_row + head * D + 4 * t) =
        uint2{ob[0] | (static_cast<uint32_t>(ob[1]) << 16), ob[2] | (static_cast<uint32_t>(ob[3]) << 16)};
}

}  // namespace hsdpa
