// hsdpa_kernels.hip — gfx950 kernels of the attention step: the attention
// kernels for head dimensions 64, 128 and 256 (templates in
// hsdpa_attn_kernels.h), the element kernels around them, and the launchers.

#include "hsdpa_attn_kernels.h"

namespace hsdpa {

// ---------------------------------------------------------------------------
// KV append (src/jit/target/x86/execution/kv.rs:15-69): row r of KV head h of
// the token-major block, (r*heads + h)*head_dim, to position past + r of head
// h, h*stride + (past + r)*head_dim. The source is one contiguous run, so
// element e of it maps to (r, h, d) = (e / (heads*hd), e / hd % heads, e % hd).
// Vector path: 16 bytes per lane (head_dim and stride multiples of 8, pointers
// 16-byte aligned); otherwise one bf16 per lane. Grid-stride over the block.
// ---------------------------------------------------------------------------
template <bool VEC>
__global__ __launch_bounds__(256) void kv_append(KvAppendArgs a)
{
    constexpr uint64_t W = VEC ? 8 : 1;                          // elements per lane
    const uint64_t per_row = a.heads * a.head_dim;
    const uint64_t total = a.rows * per_row / W;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const uint64_t e = i * W;
        const uint64_t r = e / per_row, rem = e - r * per_row;
        const uint64_t h = rem / a.head_dim, d = rem - h * a.head_dim;
        const uint64_t dst = h * a.stride + (a.past + r) * a.head_dim + d;
        if (VEC) {
            const u32x4 kv = *reinterpret_cast<const u32x4 *>(a.in_keys + e);
            const u32x4 vv = *reinterpret_cast<const u32x4 *>(a.in_values + e);
            *reinterpret_cast<u32x4 *>(a.keys + dst) = kv;
            *reinterpret_cast<u32x4 *>(a.values + dst) = vv;
        } else {
            a.keys[dst] = a.in_keys[e];
            a.values[dst] = a.in_values[e];
        }
    }
}

// ---------------------------------------------------------------------------
// Head RMS norm + RoPE (the head-norm-rope node, transforms.rs:32-81), one wave
// per (row, head), restating the AVX-512 element kernels bit for bit:
//  * sum of squares (emit_elem.rs:251-271): vdpbf16ps(x, x) per block of 32
//    into chain c % min(4, blocks), 16 f32 lanes per chain; chain c lives in
//    lanes 16c .. 16c+15, lane L of a chain takes elements 2L+1 then 2L of each
//    block (bf16 inputs denormals-as-zero, each product exact, one rounding per
//    add, results flushed to zero); chains added in order, then the hsum tree;
//  * scalar: * fl(1/dim), + eps, correctly rounded sqrt, 1 / that;
//  * y = bf16((x * inv) * w'), w' = w or w + 1 (emit_elem.rs:302-334);
//  * rotate_half RoPE on the normalised bf16 values (emit_elem.rs:479-520):
//    a' = fma(-b, s, a c), b' = fma(b, c, a s).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_daz(uint16_t b)
{
    return __uint_as_float((b & 0x7F80u) ? static_cast<uint32_t>(b) << 16 : static_cast<uint32_t>(b & 0x8000u) << 16);
}

__device__ __forceinline__ float ftz(float x)
{
    const uint32_t b = __float_as_uint(x);
    return (b & 0x7F800000u) ? x : __uint_as_float(b & 0x80000000u);
}

__device__ __forceinline__ float bf16f(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }

// One (row, head), one wave: x (dim bf16) normalised and rotated in place;
// `copy`, when not null, receives the same dim values. cs and sn are the
// table rows of the position (read only when rotary > 0).
__device__ __forceinline__ void norm_rope_head(uint16_t *x, uint16_t *copy, const uint16_t *w, const uint16_t *cs,
                                               const uint16_t *sn, int dim, int rotary, int plus_one, float eps,
                                               uint16_t *ybuf, int l)
{
    const int c = l >> 4, L = l & 15;
    const int nb = dim / 32, nacc = nb < 4 ? nb : 4;
    float acc = 0.0f;
    if (c < nacc)
        for (int b = c; b < nb; b += nacc) {
            const float x1 = bf16_daz(x[32 * b + 2 * L + 1]), x0 = bf16_daz(x[32 * b + 2 * L]);
            acc = ftz(__builtin_fmaf(x1, x1, acc));
            acc = ftz(__builtin_fmaf(x0, x0, acc));
        }
    // chains 1..3 added in order into chain 0
    const float c1 = __shfl(acc, L + 16), c2 = __shfl(acc, L + 32), c3 = __shfl(acc, L + 48);
    float s = acc;
    if (nacc > 1) s = s + c1;
    if (nacc > 2) s = s + c2;
    if (nacc > 3) s = s + c3;
    // the hsum tree over the 16 lanes of chain 0, in every lane
    float lv[16];
#pragma unroll
    for (int i = 0; i < 16; i++) lv[i] = __shfl(s, i);
    float h8[8], h4[4];
#pragma unroll
    for (int i = 0; i < 8; i++) h8[i] = lv[i] + lv[i + 8];
#pragma unroll
    for (int i = 0; i < 4; i++) h4[i] = h8[i] + h8[i + 4];
    const float u0 = h4[0] + h4[1], u1 = h4[2] + h4[3];
    float ms = u0 + u1;
    ms = ms * (1.0f / static_cast<float>(dim));
    ms = ms + eps;
    const float inv = 1.0f / __builtin_sqrtf(ms);
    for (int i = l; i < dim; i += 64) {
        float ww = bf16f(w[i]);
        if (plus_one) ww = ww + 1.0f;
        float v = bf16f(x[i]) * inv;
        v = v * ww;
        ybuf[i] = static_cast<uint16_t>(cvt_out(v));
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int half = rotary / 2;
    for (int i = l; i < dim; i += 64) {
        uint16_t out = ybuf[i];
        if (i < rotary) {
            const int j = i < half ? i : i - half;
            const float av = bf16f(ybuf[j]), bv = bf16f(ybuf[j + half]);
            const float cv = bf16f(cs[j]), sv = bf16f(sn[j]);
            const float r = i < half ? __builtin_fmaf(-bv, sv, av * cv) : __builtin_fmaf(bv, cv, av * sv);
            out = static_cast<uint16_t>(cvt_out(r));
        }
        x[i] = out;
        if (copy) copy[i] = out;
    }
}

// norm_rope_head for a compile-time dim (64, 128, 256): the same operations in
// the same order, with every global load (the sum-of-squares elements, x and w
// in output order, the table entries) issued before the first use, so that the
// wave waits on one round trip instead of three.
template <int DIM>
__device__ __forceinline__ void norm_rope_head_d(uint16_t *x, uint16_t *copy, const uint16_t *w, const uint16_t *cs,
                                                 const uint16_t *sn, int rotary, int plus_one, float eps,
                                                 uint16_t *ybuf, int l)
{
    constexpr int NB = DIM / 32, NACC = NB < 4 ? NB : 4, PB = (NB + NACC - 1) / NACC, PE = DIM / 64;
    const int c = l >> 4, L = l & 15, half = rotary / 2;
    uint16_t s1[PB], s0[PB], xe[PE], we[PE], ce[PE] = {}, se[PE] = {};
#pragma unroll
    for (int p = 0; p < PB; p++) {
        const int b = c + NACC * p, bb = (c < NACC && b < NB) ? b : 0;
        s1[p] = x[32 * bb + 2 * L + 1];
        s0[p] = x[32 * bb + 2 * L];
    }
#pragma unroll
    for (int p = 0; p < PE; p++) {
        xe[p] = x[l + 64 * p];
        we[p] = w[l + 64 * p];
    }
    if (rotary) {
#pragma unroll
        for (int p = 0; p < PE; p++) {
            const int i = l + 64 * p, j = i < rotary ? (i < half ? i : i - half) : 0;
            ce[p] = cs[j];
            se[p] = sn[j];
        }
    }
    float acc = 0.0f;
    if (c < NACC) {
#pragma unroll
        for (int p = 0; p < PB; p++)
            if (c + NACC * p < NB) {
                const float x1 = bf16_daz(s1[p]), x0 = bf16_daz(s0[p]);
                acc = ftz(__builtin_fmaf(x1, x1, acc));
                acc = ftz(__builtin_fmaf(x0, x0, acc));
            }
    }
    // chains 1..3 added in order into chain 0
    const float c1 = __shfl(acc, L + 16), c2 = __shfl(acc, L + 32), c3 = __shfl(acc, L + 48);
    float s = acc;
    if (NACC > 1) s = s + c1;
    if (NACC > 2) s = s + c2;
    if (NACC > 3) s = s + c3;
    // the hsum tree over the 16 lanes of chain 0, in every lane
    float lv[16];
#pragma unroll
    for (int i = 0; i < 16; i++) lv[i] = __shfl(s, i);
    float h8[8], h4[4];
#pragma unroll
    for (int i = 0; i < 8; i++) h8[i] = lv[i] + lv[i + 8];
#pragma unroll
    for (int i = 0; i < 4; i++) h4[i] = h8[i] + h8[i + 4];
    const float u0 = h4[0] + h4[1], u1 = h4[2] + h4[3];
    float ms = u0 + u1;
    ms = ms * (1.0f / static_cast<float>(DIM));
    ms = ms + eps;
    const float inv = 1.0f / __builtin_sqrtf(ms);
#pragma unroll
    for (int p = 0; p < PE; p++) {
        float ww = bf16f(we[p]);
        if (plus_one) ww = ww + 1.0f;
        float v = bf16f(xe[p]) * inv;
        v = v * ww;
        ybuf[l + 64 * p] = static_cast<uint16_t>(cvt_out(v));
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int p = 0; p < PE; p++) {
        const int i = l + 64 * p;
        uint16_t out = ybuf[i];
        if (i < rotary) {
            const int j = i < half ? i : i - half;
            const float av = bf16f(ybuf[j]), bv = bf16f(ybuf[j + half]);
            const float cv = bf16f(ce[p]), sv = bf16f(se[p]);
            const float r = i < half ? __builtin_fmaf(-bv, sv, av * cv) : __builtin_fmaf(bv, cv, av * sv);
            out = static_cast<uint16_t>(cvt_out(r));
        }
        x[i] = out;
        if (copy) copy[i] = out;
    }
}

// One (row, head) of the node by the wave: the compile-time routine for the
// engine's head dims, the general one otherwise.
__device__ __forceinline__ void norm_rope_any(uint16_t *x, uint16_t *copy, const uint16_t *w, const uint16_t *cs,
                                              const uint16_t *sn, int dim, int rotary, int plus_one, float eps,
                                              uint16_t *ybuf, int l)
{
    switch (dim) {
    case 64: norm_rope_head_d<64>(x, copy, w, cs, sn, rotary, plus_one, eps, ybuf, l); break;
    case 128: norm_rope_head_d<128>(x, copy, w, cs, sn, rotary, plus_one, eps, ybuf, l); break;
    case 256: norm_rope_head_d<256>(x, copy, w, cs, sn, rotary, plus_one, eps, ybuf, l); break;
    default: norm_rope_head(x, copy, w, cs, sn, dim, rotary, plus_one, eps, ybuf, l); break;
    }
}

__global__ __launch_bounds__(64) void head_norm_rope(NormRopeArgs a)
{
    __shared__ uint16_t ybuf[512];
    const uint64_t row = blockIdx.x;
    uint16_t *x = a.data + row * a.row_stride + static_cast<uint64_t>(blockIdx.y) * a.head_stride;
    norm_rope_any(x, nullptr, a.w, a.cos + (a.past + row) * a.table_row, a.sin + (a.past + row) * a.table_row, a.dim,
                  a.rotary, a.plus_one, a.eps, ybuf, static_cast<int>(threadIdx.x));
}

// The layer chain's element work before the attention (the head-norm-rope
// node for q then k, and the kv-append node, lowering.rs:549-592) in one
// launch: grid (rows, heads + kv_heads), one wave per (row, head). A KV
// head's wave writes the normalised k row both in place and into the cache,
// then copies the v row; the results equal the three nodes run in order.
__global__ __launch_bounds__(64) void layer_prep(LayerPrepArgs a)
{
    __shared__ uint16_t ybuf[512];
    const uint64_t row = blockIdx.x, pos = a.past + row;
    const int y = static_cast<int>(blockIdx.y), l = static_cast<int>(threadIdx.x);
    const uint16_t *cs = a.cos + pos * a.table_row, *sn = a.sin + pos * a.table_row;
    if (y < a.heads) {
        norm_rope_any(a.q + row * a.q_row + static_cast<uint64_t>(y) * a.q_head, nullptr, a.q_norm, cs, sn, a.dim,
                      a.rotary, a.plus_one, a.eps, ybuf, l);
        return;
    }
    const uint64_t h = static_cast<uint64_t>(y - a.heads);
    const uint64_t dst = h * a.kv_stride + pos * a.dim, src = row * a.kv_row + h * a.dim;
    norm_rope_any(a.k + src, a.keys + dst, a.k_norm, cs, sn, a.dim, a.rotary, a.plus_one, a.eps, ybuf, l);
    for (int i = l; i < a.dim; i += 64) a.values[dst + i] = a.v[src + i];
}

// ---------------------------------------------------------------------------
// Output gate (the attention-output-gate node): gate_bf16 per element,
// grid-stride over rows x width.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void output_gate(GateArgs a)
{
    const uint64_t total = a.rows * a.width;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const uint64_t r = i / a.width, c = i - r * a.width;
        uint16_t *ap = a.attn + r * a.attn_row + c;
        *ap = gate_bf16(*ap, a.gate[r * a.gate_row + c]);
    }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
bool head_dim_supported(int d) { return d >= 32 && d <= 512 && d % 32 == 0; }


// MR: 1 for a few rows after a cache, one column per (row, head) pair; 2 for
// several groups numbered onto one XCD per key range (DecodeIds), a few rows or
// one row (row 0 of every column).
template <int D, int MR>
static hipError_t decode_dm(const DecodeArgs &a, int kv_heads, hipStream_t s)
{
    // MR = 2: the groups of a key range on one XCD (DecodeIds)
    constexpr bool xcd = MR == 2;
    const auto pad8 = [](int n) { return static_cast<unsigned>((n + 7) / 8 * 8); };
    const dim3 gqk = xcd ? dim3(pad8(a.nwg_qk) * a.sub, kv_heads, 1) : dim3(a.nwg_qk, kv_heads, a.sub);
    const dim3 gpv = xcd ? dim3(pad8(a.nwg_pv) * a.sub, kv_heads, 1) : dim3(a.nwg_pv, kv_heads, a.sub);
    hipError_t e;
    if (a.qk_all) {
        // pass 1 scores all the KV head's groups in one workgroup, two or more
        // tiles per wave (decode_qk_groups)
        const dim3 g1(a.nwg_qk, kv_heads, 1);
        if (a.keys_qk <= 4 * kKeyTile) return hipErrorInvalidValue;
        e = a.keys_qk == 8 * kKeyTile ? launch(decode_qk<D, true, MR, false, true, true>, g1, dim3(256), s, a)
                                      : launch(decode_qk<D, true, MR, false, false, true>, g1, dim3(256), s, a);
    } else {
        e = a.keys_qk == 8 * kKeyTile ? launch(decode_qk<D, true, MR, false, true>, gqk, dim3(256), s, a)
            : a.keys_qk > 4 * kKeyTile  ? launch(decode_qk<D, true, MR>, gqk, dim3(256), s, a)
                                        : launch(decode_qk<D, false, MR>, gqk, dim3(256), s, a);
    }
    if (e != hipSuccess) return e;
    if (a.direct) {
        // a short cache: pass 2 writes the outputs (decode_direct_ok); one
        // group, so never the XCD numbering
        if constexpr (MR == 2) {
            return hipErrorInvalidValue;
        } else {
            const dim3 grid(D / kDirectSlice, kv_heads);
            return a.g <= 8 ? launch(decode_direct<D, false, 1, MR == 1>, grid, dim3(512), s, a)
                            : launch(decode_direct<D, false, 2, MR == 1>, grid, dim3(512), s, a);
        }
    }
    if (a.pv_all) {
        // pass 2 over all the KV head's groups in one workgroup: 256 keys
        // each, or a run of chunks each (decode_pv_all_loop_ok)
        if constexpr (D == 256) {
            if (a.keys_pv == kDecodeKeysPV) {
                e = launch(decode_pv_all<D>, dim3(a.nwg_pv, kv_heads, 1), dim3(512), s, a);
            } else {
                if (a.keys_pv < kDecodeKeysPV || a.sub < 2 || a.sub > kDecodeLoopMaxSub) return hipErrorInvalidValue;
                e = launch(decode_pv_all_loop<D>, dim3(a.nwg_pv, kv_heads, 1), dim3(512), s, a);
            }
        } else {
            return hipErrorInvalidValue;
        }
    } else if (a.g <= 8) {
        if (a.keys_pv == 4 * kKeyTile) e = launch(decode_pv<D, 4, 1, false, MR>, gpv, dim3(256), s, a);
        else if (a.keys_pv <= kDecodeKeysPV) e = launch(decode_pv<D, 8, 1, false, MR>, gpv, dim3(512), s, a);
        else e = launch(decode_pv<D, 8, 1, true, MR>, gpv, dim3(512), s, a);
    } else {
        if (a.keys_pv == 4 * kKeyTile) {
            e = launch(decode_pv<D, 4, 2, false, MR>, gpv, dim3(256), s, a);
        } else if (a.keys_pv > kDecodeKeysPV) {
            e = launch(decode_pv<D, 8, 2, true, MR>, gpv, dim3(512), s, a);
        } else {
            e = launch(decode_pv<D, 8, 2, false, MR>, gpv, dim3(512), s, a);
        }
    }
    if (e != hipSuccess) return e;
    return launch(decode_combine<D, MR != 0>, dim3(kv_heads * a.sub * a.g, (D + 63) / 64), dim3(64 * kCombineSubs),
                  s, a);
}

template <int D>
static hipError_t decode_d(const DecodeArgs &a, int kv_heads, hipStream_t s)
{
    if (a.xcd) return decode_dm<D, 2>(a, kv_heads, s);
    // one row in equal groups: the one-row kernels; a few rows, or padded
    // groups: the kernels that map each column to its (row, head)
    return a.rows == 1 && a.g * a.sub == a.cols ? decode_dm<D, 0>(a, kv_heads, s) : decode_dm<D, 1>(a, kv_heads, s);
}

hipError_t launch_decode(const DecodeArgs &a, int head_dim, int kv_heads, hipStream_t s)
{
    switch (head_dim) {
    case 64: return decode_d<64>(a, kv_heads, s);
    case 128: return decode_d<128>(a, kv_heads, s);
    case 256: return decode_d<256>(a, kv_heads, s);
    default: return launch_decode_more(a, head_dim, kv_heads, s);
    }
}

// The causal kernel's grid: (row groups, head groups) of HPW query heads x
// 32 * 8 / HPW rows at the tuned head dimensions (HPW the largest of 8, 4, 2
// that divides the group size), one head x 32 NW rows at the others.
static int prefill_hpw(const PrefillArgs &a, int head_dim)
{
    if (a.sink_on) return 1;                                    // launch_prefill_sink's grid
    if (head_dim == 64 || head_dim == 128 || head_dim == 256)
        return a.gqa % 8 == 0 ? 8 : a.gqa % 4 == 0 ? 4 : a.gqa % 2 == 0 ? 2 : 1;
    return 1;
}

static uint64_t prefill_rows_per_wg(const PrefillArgs &a, int head_dim)
{
    if (head_dim == 64 || head_dim == 128 || head_dim == 256) return 32 * (8 / prefill_hpw(a, head_dim));
    return 32 * (head_dim > 256 ? 4 : 8);
}

static dim3 prefill_grid(const PrefillArgs &a, int head_dim, int heads)
{
    const uint64_t rows_per_wg = prefill_rows_per_wg(a, head_dim);
    return dim3(static_cast<unsigned>((a.rows + rows_per_wg - 1) / rows_per_wg), heads / prefill_hpw(a, head_dim));
}

int prefill_split_count(const PrefillArgs &a, int head_dim, int heads, const PrefillSplit &ps)
{
    const dim3 g = prefill_grid(a, head_dim, heads);
    return prefill_splits(a, static_cast<uint64_t>(g.x) * g.y, heads, ps);
}

PairRows prefill_pair_rows(const PrefillArgs &a, int head_dim, int heads, const PrefillSplit &ps)
{
    const dim3 g = prefill_grid(a, head_dim, heads);
    if (prefill_splits(a, static_cast<uint64_t>(g.x) * g.y, heads, ps) > 1) return PairRows{0, 0};
    return prefill_pairs(a, g.x, static_cast<uint64_t>(g.x) * g.y, prefill_rows_per_wg(a, head_dim), heads, ps);
}

template <int D, int HPW>
static hipError_t prefill_dh(const PrefillArgs &a, int heads, const PrefillSplit &ps, hipStream_t s)
{
    const dim3 grid = prefill_grid(a, D, heads);
    const int splits = prefill_splits(a, static_cast<uint64_t>(grid.x) * grid.y, heads, ps);
    if (splits > 1) return launch_prefill_split<D, HPW, 8>(a, heads, ps, grid, splits, s);
    const PairRows pr = prefill_pairs(a, grid.x, static_cast<uint64_t>(grid.x) * grid.y, 32 * (8 / HPW), heads, ps);
    if (pr.srows) return launch_prefill_paired<D, HPW, 8>(a, heads, ps, grid, pr, s);
    if (scale_is_pow2(a.scale)) return launch(prefill_attn<D, HPW, true>, grid, dim3(512), s, a);
    return launch(prefill_attn<D, HPW, false>, grid, dim3(512), s, a);
}

template <int D>
static hipError_t prefill_d(const PrefillArgs &a, int heads, const PrefillSplit &ps, hipStream_t s)
{
    if (a.gqa % 8 == 0) return prefill_dh<D, 8>(a, heads, ps, s);
    if (a.gqa % 4 == 0) return prefill_dh<D, 4>(a, heads, ps, s);
    if (a.gqa % 2 == 0) return prefill_dh<D, 2>(a, heads, ps, s);
    return prefill_dh<D, 1>(a, heads, ps, s);
}

hipError_t launch_kv_append(const KvAppendArgs &a, bool vec, hipStream_t s)
{
    const uint64_t total = a.rows * a.heads * a.head_dim / (vec ? 8 : 1);
    const uint64_t wgs = (total + 255) / 256;
    const dim3 grid(static_cast<unsigned>(wgs < 16384 ? wgs : 16384));
    return vec ? launch(kv_append<true>, grid, dim3(256), s, a) : launch(kv_append<false>, grid, dim3(256), s, a);
}

hipError_t launch_norm_rope(const NormRopeArgs &a, hipStream_t s)
{
    return launch(head_norm_rope, dim3(static_cast<unsigned>(a.rows), static_cast<unsigned>(a.heads)), dim3(64), s, a);
}

hipError_t launch_layer_prep(const LayerPrepArgs &a, hipStream_t s)
{
    return launch(layer_prep, dim3(static_cast<unsigned>(a.rows), static_cast<unsigned>(a.heads + a.kv_heads)),
                  dim3(64), s, a);
}

hipError_t launch_gate(const GateArgs &a, hipStream_t s)
{
    const uint64_t wgs = (a.rows * a.width + 255) / 256;
    return launch(output_gate, dim3(static_cast<unsigned>(wgs < 16384 ? wgs : 16384)), dim3(256), s, a);
}

hipError_t launch_prefill(const PrefillArgs &a, int head_dim, int heads, const PrefillSplit &ps, hipStream_t s)
{
    if (a.sink_on) return launch_prefill_sink(a, head_dim, heads, ps, s);
    switch (head_dim) {
    case 64: return prefill_d<64>(a, heads, ps, s);
    case 128: return prefill_d<128>(a, heads, ps, s);
    case 256: return prefill_d<256>(a, heads, ps, s);
    default: return launch_prefill_more(a, head_dim, heads, ps, s);
    }
}

}  // namespace hsdpa
