/*
 * sdpa_scalar.c — TEST INFRASTRUCTURE ONLY (the oracle; see sdpa_oracle.h).
 *
 * Exact scalar emulation of the SDPA machine code that herbert-jit-bf16 emits
 * for x86 AVX-512 BF16 at its defaults: Chained decode form, inline exp,
 * QK group 8 (one accumulation chain), prefill block of 8 rows. Every
 * function names the emitter lines it follows. Built with -ffp-contract=off
 * so that no multiply-add is fused unless the emitted code fuses it.
 */
#include "sdpa_oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* src/jit/exp_constants.rs:14-23 */
#define EXP_NEG87 (-87.33654f)
#define EXP_LOG2E (1.442695f)
#define EXP_C4 (0.00967248f)
#define EXP_C3 (0.05550411f)
#define EXP_C2 (0.2402265f)
#define EXP_C1 (0.6931472f)
#define EXP_C0 (1.0f)
#define EXP_ONE_BITS 0x3F800000u

static inline float from_bits(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static inline uint32_t to_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }
static inline int is_denormal(float x) { return (to_bits(x) & 0x7F800000u) == 0 && (to_bits(x) & 0x007FFFFFu) != 0; }
static inline float daz(float x) { return is_denormal(x) ? from_bits(to_bits(x) & 0x80000000u) : x; }

/* src/core/tensor.rs:8-11 */
float oracle_bf16_to_f32(uint16_t b) { return from_bits((uint32_t)b << 16); }

/* src/core/tensor.rs:14-24 */
uint16_t oracle_f32_to_bf16_rne(float x)
{
    uint32_t bits = to_bits(x);
    uint32_t lsb = (bits >> 16) & 1u, round_bit = (bits >> 15) & 1u, sticky = bits & 0x7FFFu;
    uint32_t r = bits >> 16;
    if (round_bit == 1u && (sticky != 0u || lsb == 1u)) r += 1u;
    return (uint16_t)r;
}

/* vcvtneps2bf16 (decode.rs:424, prefill.rs:690): Intel SDM
 * convert_fp32_to_bfloat16. */
uint16_t oracle_cvtneps2bf16(float x)
{
    uint32_t b = to_bits(x);
    uint32_t e = b & 0x7F800000u, m = b & 0x007FFFFFu;
    if (e == 0) return (uint16_t)((b >> 16) & 0x8000u);          /* zero, denormal */
    if (e == 0x7F800000u) {
        if (m == 0) return (uint16_t)(b >> 16);                    /* infinity */
        return (uint16_t)((b >> 16) | 0x0040u);                    /* NaN, quieted */
    }
    return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

/* One lane of vdpbf16ps (prefill.rs:428-433, decode.rs:88-94): odd pair
 * first, then even, each an FP32 FMA with DAZ/FTZ and RNE. An exact product
 * added with one rounding is exactly fmaf. */
float oracle_dpbf16_lane(float acc, uint32_t a, uint32_t b)
{
    float a1 = daz(oracle_bf16_to_f32((uint16_t)(a >> 16)));
    float b1 = daz(oracle_bf16_to_f32((uint16_t)(b >> 16)));
    float a0 = daz(oracle_bf16_to_f32((uint16_t)(a & 0xFFFFu)));
    float b0 = daz(oracle_bf16_to_f32((uint16_t)(b & 0xFFFFu)));
    acc = daz(fmaf(a1, b1, daz(acc)));
    acc = daz(fmaf(a0, b0, acc));
    return acc;
}

/* vmaxps dst, src1, src2: src1 when src1 > src2, else src2. */
static inline float vmax(float a, float b) { return a > b ? a : b; }

/* exp_inline (base.rs:189-212): max, mul, roundscale(RNE), sub, four FMA
 * (Horner, vfmadd213ps), cvtps2dq, shift 23, add 1.0's bits, mul. */
float oracle_exp_poly(float x)
{
    float io = vmax(x, EXP_NEG87);
    float t1 = io * EXP_LOG2E;
    float t2 = nearbyintf(t1);               /* vrndscaleps imm 0: RNE */
    t1 = t1 - t2;
    float t3 = EXP_C4;
    t3 = fmaf(t1, t3, EXP_C3);
    t3 = fmaf(t1, t3, EXP_C2);
    t3 = fmaf(t1, t3, EXP_C1);
    t3 = fmaf(t1, t3, EXP_C0);
    /* vcvtps2dq: an integral value converts exactly; NaN and out-of-range
     * values give the integer indefinite 0x80000000 */
    int32_t k = (t2 != t2 || t2 >= 2147483648.0f || t2 < -2147483648.0f) ? INT32_MIN : (int32_t)t2;
    uint32_t sc = ((uint32_t)k << 23) + EXP_ONE_BITS;
    return t3 * from_bits(sc);
}

/* hsum (base.rs:258-267): l_i + l_{i+8}, then + 4 apart, then two vhaddps. */
static float hsum16(const float l[16])
{
    float s[8], t[4];
    for (int i = 0; i < 8; i++) s[i] = l[i] + l[i + 8];
    for (int i = 0; i < 4; i++) t[i] = s[i] + s[i + 4];
    float u0 = t[0] + t[1], u1 = t[2] + t[3];
    return u0 + u1;
}

float oracle_hsum16(const float *l) { return hsum16(l); }

/* hmax (base.rs:271-282): the same halving, then two vshufps/vmaxps steps;
 * operand order kept (dst first) so signed zeros resolve like the code. */
static float hmax16(const float l[16])
{
    float s[8], t[4];
    for (int i = 0; i < 8; i++) s[i] = vmax(l[i], l[i + 8]);
    for (int i = 0; i < 4; i++) t[i] = vmax(s[i], s[i + 4]);
    /* vshufps 0b01_00_11_10 gives [t2, t3, t0, t1]; lanes 0 and 1 of the max */
    const float u0 = vmax(t[0], t[2]), u1 = vmax(t[1], t[3]);
    /* vshufps 0b10_11_00_01 gives [u1, u0, u3, u2]; lane 0 of the max */
    return vmax(u0, u1);
}

/* The score of one position before the scale: one accumulation chain over
 * the head_dim/32 chunks of vdpbf16ps (emit_qk_group_decode prefill.rs:496-542,
 * emit_qk with one chain decode.rs:59-128), then the hsum tree, which
 * qk_reduce (prefill.rs:302-331) reproduces lane for lane. */
float oracle_qk_dot(const uint16_t *q, const uint16_t *k, int head_dim)
{
    float lanes[16] = {0};
    const int n32 = head_dim / 32;
    for (int c = 0; c < n32; c++) {
        for (int L = 0; L < 16; L++) {
            const uint16_t *qp = q + 32 * c + 2 * L, *kp = k + 32 * c + 2 * L;
            uint32_t a = ((uint32_t)qp[1] << 16) | qp[0];
            uint32_t b = ((uint32_t)kp[1] << 16) | kp[0];
            lanes[L] = oracle_dpbf16_lane(lanes[L], a, b);
        }
    }
    return hsum16(lanes);
}

static inline uint64_t roundup16(uint64_t n) { return (n + 15u) & ~(uint64_t)15u; }

/* emit_softmax (decode.rs:212-293) on `nb` blocks of 16 scores: lane-wise
 * max then hmax; lane-wise exp and sequential lane sums, then hsum; true
 * division by the sum. With the sink (sink_on, decode.rs:239-290): the
 * maximum is vmaxss(hmax, sink), the sum after the hsum gains the
 * exponential of sink - max (vsubss, the exp sequence, vaddss), and the
 * scores are multiplied by 1/sum (vdivss once, then vmulps). */
static void softmax_blocks(float *sc, uint64_t nb, int sink_on, float sink)
{
    float maxv[16];
    for (int L = 0; L < 16; L++) maxv[L] = -INFINITY;
    for (uint64_t b = 0; b < nb; b++)
        for (int L = 0; L < 16; L++) maxv[L] = vmax(maxv[L], sc[16 * b + L]);
    const float hm = hmax16(maxv);
    const float m = sink_on ? vmax(hm, sink) : hm;
    float sumv[16] = {0};
    for (uint64_t b = 0; b < nb; b++)
        for (int L = 0; L < 16; L++) {
            float w = oracle_exp_poly(sc[16 * b + L] - m);
            sumv[L] = sumv[L] + w;
            sc[16 * b + L] = w;
        }
    float sum = hsum16(sumv);
    if (sink_on) {
        sum = sum + oracle_exp_poly(sink - m);
        const float inv = 1.0f / sum;
        for (uint64_t i = 0; i < 16 * nb; i++) sc[i] = sc[i] * inv;
    } else {
        for (uint64_t i = 0; i < 16 * nb; i++) sc[i] = sc[i] / sum;
    }
}

typedef float (*qk_dot_fn)(const uint16_t *, const uint16_t *, int);

/* assembly.rs:116-174: QK pass (then -inf padding to a multiple of 16,
 * decode.rs:113-126), softmax, SV pass (decode.rs:348-428), with the QK
 * summation order `qk` (the knob sdpa_qk_group, src/jit/sdpa.rs:178-202). */
static void sdpa_head_qk(qk_dot_fn qk, const uint16_t *q, const uint16_t *k, const uint16_t *v, float *scores,
                         uint16_t *out, uint64_t n, float scale, int head_dim, int sink_on, float sink)
{
    const size_t d = (size_t)head_dim;
    for (uint64_t j = 0; j < n; j++) scores[j] = qk(q, k + j * d, head_dim) * scale;
    for (uint64_t j = n; j < roundup16(n); j++) scores[j] = -INFINITY;
    softmax_blocks(scores, roundup16(n) / 16, sink_on, sink);
    float acc[512];
    for (size_t c = 0; c < d; c++) acc[c] = 0.0f;
    for (uint64_t j = 0; j < n; j++) {
        const float p = scores[j];
        const uint16_t *vr = v + j * d;
        for (size_t c = 0; c < d; c++) acc[c] = fmaf(oracle_bf16_to_f32(vr[c]), p, acc[c]);
    }
    for (size_t c = 0; c < d; c++) out[c] = oracle_cvtneps2bf16(acc[c]);
}

void oracle_sdpa_head(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                      float *scores, uint16_t *out, uint64_t n, float scale,
                      int head_dim)
{
    sdpa_head_qk(oracle_qk_dot, q, k, v, scores, out, n, scale, head_dim, 0, 0.0f);
}

/* The head with the softmax sink (SdpaShape::sink, src/jit/ir.rs:55-60;
 * emit_softmax with sink_on, decode.rs:239-290). */
void oracle_sdpa_head_sink(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                           float *scores, uint16_t *out, uint64_t n, float scale,
                           int head_dim, float sink)
{
    sdpa_head_qk(oracle_qk_dot, q, k, v, scores, out, n, scale, head_dim, 1, sink);
}

/* sdpa_qk_group = 0 (src/jit/sdpa.rs:178-202): emit_qk with four chains
 * (stash_scale, prefill.rs:558-567; decode.rs:59-128), whose score is the
 * Fused form's (oracle_fused_qk_dot: chunk c into chain c % min(4, n32),
 * (c0 + c1) + (c2 + c3), hsum). */
void oracle_sdpa_head_qk0(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                          float *scores, uint16_t *out, uint64_t n, float scale,
                          int head_dim)
{
    sdpa_head_qk(oracle_fused_qk_dot, q, k, v, scores, out, n, scale, head_dim, 0, 0.0f);
}

/* assemble_prefill (prefill.rs:733-912): the whole rows x N rectangle of
 * scores (N = past + rows), -inf from n_i = past+i+1 to roundup16(n_i), the
 * decode softmax on exactly that many blocks per row, +0.0 written over the
 * columns n_i..N-1, then the SV over N positions for all rows. The scores
 * in the summation order `qk`: one chain (the default group of 8), or four
 * with sdpa_qk_group = 0 (emit_qk_block with chains = 4, prefill.rs:780,
 * 104-157: the tree of emit_qk "verbatim"). */
static void prefill_block_qk(qk_dot_fn qk, const uint16_t *q, const uint16_t *k, const uint16_t *v, float *scores,
                             uint16_t *out, uint64_t past, float scale, int head_dim, int rows, size_t q_row,
                             size_t out_row, int sink_on, float sink)
{
    const size_t d = (size_t)head_dim;
    const uint64_t N = past + (uint64_t)rows;
    const uint64_t rs = roundup16(N);                 /* PF_ROWB / 4 */
    for (int i = 0; i < rows; i++)
        for (uint64_t j = 0; j < N; j++)
            scores[i * rs + j] = qk(q + i * q_row, k + j * d, head_dim) * scale;
    for (int i = 0; i < rows; i++) {
        uint64_t ni = past + (uint64_t)i + 1;
        for (uint64_t j = ni; j < roundup16(ni); j++) scores[i * rs + j] = -INFINITY;
    }
    for (int i = 0; i < rows; i++)
        softmax_blocks(scores + i * rs, roundup16(past + (uint64_t)i + 1) / 16, sink_on, sink);
    for (int i = 0; i < rows; i++)
        for (int t = 0; t < rows - 1 - i; t++) scores[i * rs + past + (uint64_t)(i + 1 + t)] = 0.0f;
    for (int i = 0; i < rows; i++) {
        float acc[512];
        for (size_t c = 0; c < d; c++) acc[c] = 0.0f;
        for (uint64_t j = 0; j < N; j++) {
            const float p = scores[i * rs + j];
            const uint16_t *vr = v + j * d;
            for (size_t c = 0; c < d; c++) acc[c] = fmaf(oracle_bf16_to_f32(vr[c]), p, acc[c]);
        }
        for (size_t c = 0; c < d; c++) out[i * out_row + c] = oracle_cvtneps2bf16(acc[c]);
    }
}

void oracle_sdpa_prefill_block(const uint16_t *q, const uint16_t *k,
                               const uint16_t *v, float *scores, uint16_t *out,
                               uint64_t past, float scale, int head_dim,
                               int rows, size_t q_row, size_t out_row)
{
    prefill_block_qk(oracle_qk_dot, q, k, v, scores, out, past, scale, head_dim, rows, q_row, out_row, 0, 0.0f);
}

/* The block with the softmax sink: emit_softmax is re-emitted per row
 * (decode.rs:207-210), so each row's softmax is the head's. */
void oracle_sdpa_prefill_block_sink(const uint16_t *q, const uint16_t *k,
                                    const uint16_t *v, float *scores, uint16_t *out,
                                    uint64_t past, float scale, int head_dim,
                                    int rows, size_t q_row, size_t out_row, float sink)
{
    prefill_block_qk(oracle_qk_dot, q, k, v, scores, out, past, scale, head_dim, rows, q_row, out_row, 1, sink);
}

void oracle_sdpa_prefill_block_qk0(const uint16_t *q, const uint16_t *k,
                                   const uint16_t *v, float *scores, uint16_t *out,
                                   uint64_t past, float scale, int head_dim,
                                   int rows, size_t q_row, size_t out_row)
{
    prefill_block_qk(oracle_fused_qk_dot, q, k, v, scores, out, past, scale, head_dim, rows, q_row, out_row, 0,
                     0.0f);
}

/* tile_selector's geometry checks (attention.rs:61-98) plus the shape
 * checks of SdpaShape (ir.rs:130-148). */
int oracle_check_geometry(const oracle_attention_spec *s, const oracle_attention_call *c)
{
    if (s->heads == 0 || s->gqa == 0 || s->heads % s->gqa != 0) return -1;
    if (s->head_dim == 0 || s->head_dim % 32 != 0 || s->head_dim > 512) return -1;
    if (s->q_head < s->head_dim || s->heads * s->q_head > s->q_row) return -1;
    if (s->heads * s->head_dim > s->out_row) return -1;
    if (c->sink != 0.0f) return -1;
    if (c->kv_stride < (c->past + c->rows) * s->head_dim) return -1;
    return 0;
}

/* The selector (attention.rs:122-208) over every task of every pass of 256
 * rows: h = task / chunks (non-grouped order), kvh = h / gqa. */
int oracle_attention_scalar(const oracle_attention_spec *s, const oracle_attention_call *c)
{
    if (oracle_check_geometry(s, c) != 0) return -1;
    const uint64_t d = s->head_dim, rows_all = c->rows;
    float *scratch = (float *)malloc(sizeof(float) * 8 * roundup16(c->past + rows_all + 16));
    if (!scratch) return -1;
    for (uint64_t p0 = 0; p0 < rows_all; p0 += 256) {
        const uint64_t rows = rows_all - p0 < 256 ? rows_all - p0 : 256;
        const uint64_t past = c->past + p0;
        const uint64_t chunks = (rows + 7) / 8;
        for (uint64_t task = 0; task < chunks * s->heads; task++) {
            const uint64_t h = task / chunks, ch = task % chunks, kvh = h / s->gqa;
            const uint64_t r0 = ch * 8, r1 = r0 + 8 < rows ? r0 + 8 : rows;
            const uint16_t *kk = c->keys + kvh * c->kv_stride, *vv = c->values + kvh * c->kv_stride;
            if (r1 - r0 == 8) {
                const uint64_t ar = p0 + r0;
                oracle_sdpa_prefill_block(c->q + ar * s->q_row + h * s->q_head, kk, vv, scratch,
                                          c->output + ar * s->out_row + h * d, past + r0, c->scale,
                                          (int)d, 8, s->q_row, s->out_row);
            } else {
                for (uint64_t r = r0; r < r1; r++) {
                    const uint64_t ar = p0 + r;
                    oracle_sdpa_head(c->q + ar * s->q_row + h * s->q_head, kk, vv, scratch,
                                     c->output + ar * s->out_row + h * d, past + r + 1, c->scale, (int)d);
                }
            }
        }
    }
    free(scratch);
    return 0;
}
