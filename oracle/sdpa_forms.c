/*
 * sdpa_forms.c — TEST INFRASTRUCTURE ONLY (the oracle; see sdpa_oracle.h).
 *
 * Exact scalar emulations of the two other decode head kernels the reference
 * emits for x86, next to the default Chained AVX-512 one of sdpa_scalar.c:
 *
 *   - the Fused form (knob sdpa_form = fused, src/jit/knobs.rs:66-68; form
 *     src/jit/ir.rs:109-114): an online softmax over blocks of 16 positions,
 *     emit_fused, src/jit/target/x86/emit_sdpa/x86/decode.rs:501-669;
 *   - the AVX2 arm, what the engine emits on a host without AVX-512 BF16
 *     (src/jit/sdpa.rs:452-471): the Chained form with eight lanes,
 *     src/jit/target/x86/emit_sdpa_avx2.rs:231-470.
 *
 * And the attention node under each (the selector of
 * src/jit/target/x86/execution/attention.rs:56-224 with the kernels that
 * src/jit/sdpa.rs hands it). Built with -ffp-contract=off: only the written
 * fmaf calls fuse, as only the emitted FMA instructions do.
 */
#include "sdpa_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline float from_bits(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static inline uint32_t to_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }
/* vmaxps dst, src1, src2 lane: src1 when src1 > src2, else src2 (Intel SDM). */
static inline float vmax(float a, float b) { return a > b ? a : b; }

/* ---- Fused form -------------------------------------------------------------- */

/* The score of one position in emit_fused (decode.rs:551-580), before the
 * scale: n32 = head_dim/32 chunks of 32 bf16, chunk c into accumulator
 * c % n_acc (n_acc = min(4, n32)) by vdpbf16ps, the accumulators added as
 * (w0 + w1) + (w2 + w3) (sequentially below four), then the hsum tree. */
float oracle_fused_qk_dot(const uint16_t *q, const uint16_t *k, int head_dim)
{
    const int n32 = head_dim / 32, n_acc = n32 < 4 ? n32 : 4;
    float w[4][16];
    memset(w, 0, sizeof(w));
    for (int c = 0; c < n32; c++)
        for (int L = 0; L < 16; L++) {
            const uint16_t *qp = q + 32 * c + 2 * L, *kp = k + 32 * c + 2 * L;
            const uint32_t a = ((uint32_t)kp[1] << 16) | kp[0];
            const uint32_t b = ((uint32_t)qp[1] << 16) | qp[0];
            w[c % n_acc][L] = oracle_dpbf16_lane(w[c % n_acc][L], a, b);
        }
    float lanes[16];
    for (int L = 0; L < 16; L++) {
        if (n_acc == 4) {
            const float a01 = w[0][L] + w[1][L], a23 = w[2][L] + w[3][L];
            lanes[L] = a01 + a23;
        } else {
            float s = w[0][L];
            for (int a = 1; a < n_acc; a++) s = s + w[a][L];
            lanes[L] = s;
        }
    }
    return oracle_hsum16(lanes);
}

/* hmax (base.rs:271-282), as the Chained form uses it. */
static float hmax16(const float l[16])
{
    float s[8], t[4];
    for (int i = 0; i < 8; i++) s[i] = vmax(l[i], l[i + 8]);
    for (int i = 0; i < 4; i++) t[i] = vmax(s[i], s[i + 4]);
    const float u0 = vmax(t[0], t[2]), u1 = vmax(t[1], t[3]);
    return vmax(u0, u1);
}

/* emit_fused (decode.rs:501-669) on one query head against `n` rows: per block
 * of 16 positions, the 16 scores (-inf past n), the new maximum
 * hmax(max(scores, m)), corr = P(m_old - m_new) lane by lane, p = P(s - m_new),
 * sum = sum * corr + p lane by lane, acc = acc * corr, then acc += V_j * p_j
 * (FMA) for the block's positions in order. After the last block: 1 / hsum(sum)
 * (vdivss), acc times it (vmulps), vcvtneps2bf16. n = 0 writes zeros.
 * acc_out (optional): the head_dim f32 accumulators before the conversion. */
int oracle_fused_head(const uint16_t *q, const uint16_t *k, const uint16_t *v, uint16_t *out, uint64_t n,
                      float scale, int head_dim, float *acc_out)
{
    if (head_dim <= 0 || head_dim % 32 != 0 || head_dim > 256) return -1;   /* ir.rs:146-148, FUSED_MAX_ACC */
    const size_t d = (size_t)head_dim;
    float acc[256];
    for (size_t c = 0; c < d; c++) acc[c] = 0.0f;
    float maxv = -INFINITY, sumv[16];
    for (int L = 0; L < 16; L++) sumv[L] = 0.0f;
    if (n != 0) {
        for (uint64_t b0 = 0; b0 < n; b0 += 16) {
            const uint64_t cnt = n - b0 < 16 ? n - b0 : 16;
            float s[16];
            for (int L = 0; L < 16; L++) s[L] = -INFINITY;
            for (uint64_t j = 0; j < cnt; j++) s[j] = oracle_fused_qk_dot(q, k + (b0 + j) * d, head_dim) * scale;
            float blk[16];
            for (int L = 0; L < 16; L++) blk[L] = vmax(s[L], maxv);     /* vmaxps blk, w0, maxv */
            const float mnew = hmax16(blk);
            const float corr = oracle_exp_poly(maxv - mnew);            /* vsubps w1, maxv, blk */
            maxv = mnew;
            float p[16];
            for (int L = 0; L < 16; L++) p[L] = oracle_exp_poly(s[L] - maxv);
            for (int L = 0; L < 16; L++) {
                sumv[L] = sumv[L] * corr;
                sumv[L] = sumv[L] + p[L];
            }
            for (size_t c = 0; c < d; c++) acc[c] = acc[c] * corr;
            for (uint64_t j = 0; j < cnt; j++) {
                const uint16_t *vr = v + (b0 + j) * d;
                for (size_t c = 0; c < d; c++) acc[c] = fmaf(oracle_bf16_to_f32(vr[c]), p[j], acc[c]);
            }
        }
        const float inv = 1.0f / oracle_hsum16(sumv);
        for (size_t c = 0; c < d; c++) acc[c] = acc[c] * inv;
    }
    if (acc_out)
        for (size_t c = 0; c < d; c++) acc_out[c] = acc[c];
    for (size_t c = 0; c < d; c++) out[c] = oracle_cvtneps2bf16(acc[c]);
    return 0;
}

/* ---- AVX2 arm ------------------------------------------------------------------ */

/* dp_bf16 (emit_sdpa_avx2.rs:195-205) on one f32 lane: the even element of
 * the pair (shifted up) first, then the odd one (masked), each an FMA with
 * one rounding; no DAZ or FTZ (the default MXCSR). */
static inline float avx2_dp_lane(float acc, uint16_t k0, uint16_t k1, uint16_t q0, uint16_t q1)
{
    acc = fmaf(oracle_bf16_to_f32(k0), oracle_bf16_to_f32(q0), acc);
    acc = fmaf(oracle_bf16_to_f32(k1), oracle_bf16_to_f32(q1), acc);
    return acc;
}

/* hsum of a ymm (emit_sdpa_avx2.rs:158-164): high half onto the low half,
 * then two vhaddps: (x0 + x1) + (x2 + x3). */
static float avx2_hsum8(const float l[8])
{
    float x[4];
    for (int i = 0; i < 4; i++) x[i] = l[i] + l[i + 4];
    const float h0 = x[0] + x[1], h1 = x[2] + x[3];
    return h0 + h1;
}

/* hmax of a ymm (emit_sdpa_avx2.rs:167-178): high half onto the low half,
 * then vshufps (1,0,3,2) + vmaxps and (2,3,0,1) + vmaxps, dst first. */
static float avx2_hmax8(const float l[8])
{
    float x[4];
    for (int i = 0; i < 4; i++) x[i] = vmax(l[i], l[i + 4]);
    const float y0 = vmax(x[0], x[1]), y2 = vmax(x[2], x[3]);
    return vmax(y0, y2);
}

/* cvt_bf16 (emit_sdpa_avx2.rs:208-217): ((b >> 16) & 1) + 0x7FFF + b, then
 * >> 16, in 32-bit integer lanes (no special case for NaN or denormals). */
uint16_t oracle_avx2_cvt_bf16(float x)
{
    const uint32_t b = to_bits(x);
    return (uint16_t)((((b >> 16) & 1u) + 0x7FFFu + b) >> 16);
}

/* The QK score of one position in the AVX2 arm (emit_sdpa_avx2.rs:262-305),
 * before the scale: head_dim/16 blocks of 16 bf16 (8 lanes), block b into
 * chain b % n_acc (n_acc = min(4, blocks)), the chains added as
 * (0 + 1) + (2 + 3) (sequentially below four), then hsum8. */
float oracle_avx2_qk_dot(const uint16_t *q, const uint16_t *k, int head_dim)
{
    const int nb16 = head_dim / 16, n_acc = nb16 < 4 ? (nb16 > 0 ? nb16 : 1) : 4;
    float a[4][8];
    memset(a, 0, sizeof(a));
    for (int b = 0; b < nb16; b++)
        for (int L = 0; L < 8; L++) {
            const int e = 16 * b + 2 * L;
            a[b % n_acc][L] = avx2_dp_lane(a[b % n_acc][L], k[e], k[e + 1], q[e], q[e + 1]);
        }
    float lanes[8];
    for (int L = 0; L < 8; L++) {
        if (n_acc == 4) {
            const float s01 = a[0][L] + a[1][L], s23 = a[2][L] + a[3][L];
            lanes[L] = s01 + s23;
        } else {
            float s = a[0][L];
            for (int c = 1; c < n_acc; c++) s = s + a[c][L];
            lanes[L] = s;
        }
    }
    return avx2_hsum8(lanes);
}

/* The AVX2 head (emit_sdpa_avx2.rs:231-470): scores with -inf padding to a
 * multiple of 8; softmax over ceil(n/8) blocks of 8 (lane-wise max, hmax8;
 * exponentials with lane sums in block order, hsum8; vdivps by the sum); SV
 * with FMA in position order; the integer RNE conversion. With the sink
 * (emit_sdpa_avx2.rs:362-400): vmaxss(hmax, sink), the exponential of
 * sink - max added after the hsum, 1/sum by vdivss and vmulps.
 * scores: at least roundup8(n) f32. */
static int avx2_head(const uint16_t *q, const uint16_t *k, const uint16_t *v, float *scores, uint16_t *out,
                     uint64_t n, float scale, int head_dim, int sink_on, float sink)
{
    if (head_dim <= 0 || head_dim % 16 != 0 || head_dim > 512) return -1;      /* check_avx2 */
    const size_t d = (size_t)head_dim;
    for (uint64_t j = 0; j < n; j++) scores[j] = oracle_avx2_qk_dot(q, k + j * d, head_dim) * scale;
    const uint64_t nb = (n + 7) / 8;
    for (uint64_t j = n; j < 8 * nb; j++) scores[j] = -INFINITY;
    float acc[512];
    for (size_t c = 0; c < d; c++) acc[c] = 0.0f;
    if (n != 0) {
        float maxv[8];
        for (int L = 0; L < 8; L++) maxv[L] = -INFINITY;
        for (uint64_t b = 0; b < nb; b++)
            for (int L = 0; L < 8; L++) maxv[L] = vmax(maxv[L], scores[8 * b + L]);
        const float hm = avx2_hmax8(maxv);
        const float m = sink_on ? vmax(hm, sink) : hm;
        float sumv[8] = {0};
        for (uint64_t b = 0; b < nb; b++)
            for (int L = 0; L < 8; L++) {
                const float w = oracle_exp_poly(scores[8 * b + L] - m);
                sumv[L] = sumv[L] + w;
                scores[8 * b + L] = w;
            }
        float sum = avx2_hsum8(sumv);
        if (sink_on) {
            sum = sum + oracle_exp_poly(sink - m);
            const float inv = 1.0f / sum;
            for (uint64_t i = 0; i < 8 * nb; i++) scores[i] = scores[i] * inv;
        } else {
            for (uint64_t i = 0; i < 8 * nb; i++) scores[i] = scores[i] / sum;
        }
        for (uint64_t j = 0; j < n; j++) {
            const float p = scores[j];
            const uint16_t *vr = v + j * d;
            for (size_t c = 0; c < d; c++) acc[c] = fmaf(oracle_bf16_to_f32(vr[c]), p, acc[c]);
        }
    }
    for (size_t c = 0; c < d; c++) out[c] = oracle_avx2_cvt_bf16(acc[c]);
    return 0;
}

int oracle_avx2_head(const uint16_t *q, const uint16_t *k, const uint16_t *v, float *scores, uint16_t *out,
                     uint64_t n, float scale, int head_dim)
{
    return avx2_head(q, k, v, scores, out, n, scale, head_dim, 0, 0.0f);
}

int oracle_avx2_head_sink(const uint16_t *q, const uint16_t *k, const uint16_t *v, float *scores, uint16_t *out,
                          uint64_t n, float scale, int head_dim, float sink)
{
    return avx2_head(q, k, v, scores, out, n, scale, head_dim, 1, sink);
}

/* ---- the attention node under a form ------------------------------------------ */

typedef struct form_job {
    const oracle_attention_spec *s;
    const oracle_attention_call *c;
    int form;
    uint64_t t0, t1;     /* task range: (q head, pass, chunk) flattened as below */
    int rc;
} form_job;

/* One task of the node: row group (pass p0, chunk of up to 8 rows) of q head h.
 * Chained: a full chunk runs the 8-row prefill block, other rows the Chained
 * head. Fused: the same block kernel (the prefill policy has no form,
 * src/jit/sdpa.rs:111-176), other rows the Fused head, or the Chained head
 * above head_dim 256 where the Fused form declines and the engine falls back
 * (src/jit/sdpa.rs:491-510). AVX2: no block kernel (prefill_kernel returns
 * None without AVX-512 BF16, src/jit/sdpa.rs:118-120), so every row runs the
 * AVX2 head (the selector's chunk of one row, attention.rs:99). */
static int run_rows(const oracle_attention_spec *s, const oracle_attention_call *c, int form, uint64_t h,
                    uint64_t r0, uint64_t r1, uint64_t pass_past, uint64_t pass_row0, float *scratch)
{
    const uint64_t d = s->head_dim, kvh = h / s->gqa;
    const uint16_t *kk = c->keys + kvh * c->kv_stride, *vv = c->values + kvh * c->kv_stride;
    if (form != 2 && form != 5 && r1 - r0 == 8) {
        const uint64_t ar = pass_row0 + r0;
        if (form == 4)
            oracle_sdpa_prefill_block_sink(c->q + ar * s->q_row + h * s->q_head, kk, vv, scratch,
                                           c->output + ar * s->out_row + h * d, pass_past + r0, c->scale, (int)d, 8,
                                           s->q_row, s->out_row, c->sink);
        else if (form == 3)
            oracle_sdpa_prefill_block_qk0(c->q + ar * s->q_row + h * s->q_head, kk, vv, scratch,
                                          c->output + ar * s->out_row + h * d, pass_past + r0, c->scale, (int)d, 8,
                                          s->q_row, s->out_row);
        else
            oracle_sdpa_prefill_block(c->q + ar * s->q_row + h * s->q_head, kk, vv, scratch,
                                      c->output + ar * s->out_row + h * d, pass_past + r0, c->scale, (int)d, 8,
                                      s->q_row, s->out_row);
        return 0;
    }
    for (uint64_t r = r0; r < r1; r++) {
        const uint64_t ar = pass_row0 + r, n = pass_past + r + 1;
        const uint16_t *qp = c->q + ar * s->q_row + h * s->q_head;
        uint16_t *op = c->output + ar * s->out_row + h * d;
        if (form == 1 && d <= 256) {
            if (oracle_fused_head(qp, kk, vv, op, n, c->scale, (int)d, NULL) != 0) return -1;
        } else if (form == 2) {
            if (oracle_avx2_head(qp, kk, vv, scratch, op, n, c->scale, (int)d) != 0) return -1;
        } else if (form == 5) {
            if (oracle_avx2_head_sink(qp, kk, vv, scratch, op, n, c->scale, (int)d, c->sink) != 0) return -1;
        } else if (form == 4) {
            oracle_sdpa_head_sink(qp, kk, vv, scratch, op, n, c->scale, (int)d, c->sink);
        } else if (form == 3) {
            oracle_sdpa_head_qk0(qp, kk, vv, scratch, op, n, c->scale, (int)d);
        } else {
            oracle_sdpa_head(qp, kk, vv, scratch, op, n, c->scale, (int)d);
        }
    }
    return 0;
}

static void *form_worker(void *arg)
{
    form_job *j = (form_job *)arg;
    const oracle_attention_spec *s = j->s;
    const oracle_attention_call *c = j->c;
    const uint64_t chunk = j->form == 2 || j->form == 5 ? 1 : 8;
    const uint64_t groups = (c->rows + chunk - 1) / chunk;
    float *scratch = (float *)malloc(sizeof(float) * 8 * (((c->past + c->rows + 16) + 15) & ~(uint64_t)15));
    if (!scratch) {
        j->rc = -1;
        return NULL;
    }
    j->rc = 0;
    for (uint64_t t = j->t0; t < j->t1 && j->rc == 0; t++) {
        const uint64_t h = t / groups, gi = t % groups;
        /* row group gi of the call: rows [gi*chunk, ...) inside passes of 256 */
        const uint64_t row = gi * chunk, p0 = row / 256 * 256;
        const uint64_t rows_pass = c->rows - p0 < 256 ? c->rows - p0 : 256;
        const uint64_t r0 = row - p0, r1 = r0 + chunk < rows_pass ? r0 + chunk : rows_pass;
        j->rc = run_rows(s, c, j->form, h, r0, r1, c->past + p0, p0, scratch);
    }
    free(scratch);
    return NULL;
}

/* The attention node with the given decode form (0 Chained, 1 Fused, 2 AVX2,
 * 3 Chained with sdpa_qk_group = 0, 4 Chained with the softmax sink c->sink,
 * 5 AVX2 with the sink; the Fused form declines a sink, src/jit/emit_sdpa.rs:
 * 468-470, and the engine then runs the Chained one)
 * on `threads` threads (0 or 1: the calling thread), tasks = (q head, row
 * group) in contiguous ranges. Rows are processed in passes of 256, so a row
 * group never straddles a pass. Returns 0, or -1 on an invalid geometry. */
int oracle_attention_form(const oracle_attention_spec *s, const oracle_attention_call *c, int form, int threads)
{
    if (form < 0 || form > 5) return -1;
    oracle_attention_call cg = *c;
    if (form >= 4) cg.sink = 0.0f;                 /* the sink forms take any value */
    if (oracle_check_geometry(s, &cg) != 0) return -1;
    if (c->rows == 0) return 0;
    const uint64_t chunk = form == 2 || form == 5 ? 1 : 8;
    const uint64_t tasks = s->heads * ((c->rows + chunk - 1) / chunk);
    int nt = threads < 1 ? 1 : threads;
    if ((uint64_t)nt > tasks) nt = (int)tasks;
    form_job jobs[256];
    pthread_t tids[256];
    if (nt > 256) nt = 256;
    for (int i = 0; i < nt; i++) {
        jobs[i].s = s;
        jobs[i].c = c;
        jobs[i].form = form;
        jobs[i].t0 = tasks * (uint64_t)i / (uint64_t)nt;
        jobs[i].t1 = tasks * (uint64_t)(i + 1) / (uint64_t)nt;
        jobs[i].rc = 0;
    }
    for (int i = 1; i < nt; i++) pthread_create(&tids[i], NULL, form_worker, &jobs[i]);
    form_worker(&jobs[0]);
    int rc = jobs[0].rc;
    for (int i = 1; i < nt; i++) {
        pthread_join(tids[i], NULL);
        if (jobs[i].rc != 0) rc = jobs[i].rc;
    }
    return rc;
}

/* oracle_exp_poly over an array (for the tests' numeric-scheme models). */
void oracle_exp_poly_n(const float *x, float *y, uint64_t n)
{
    for (uint64_t i = 0; i < n; i++) y[i] = oracle_exp_poly(x[i]);
}
