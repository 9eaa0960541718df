/*
 * elem_scalar.c — TEST INFRASTRUCTURE ONLY (the oracle; see sdpa_oracle.h).
 *
 * Exact scalar emulation of the AVX-512 element kernels that herbert-jit-bf16
 * emits around its attention node (src/jit/target/x86/emit_elem.rs): the head
 * RMS norm (Gemma convention), the rotate_half RoPE and the sigmoid output
 * gate. Built with -ffp-contract=off: only the FMAs of the emitted code fuse.
 */
#include "sdpa_oracle.h"

#include <math.h>
#include <stdint.h>
#include <string.h>

static inline float f32(uint16_t b) { return oracle_bf16_to_f32(b); }

/* emit_elem.rs:239-335. Pass 1: sum of squares, one vdpbf16ps(x, x) per block
 * of 32 into chain c % min(4, blocks); chains added in order into chain 0;
 * hsum; then scalar: * fl(1/dim), + eps, vsqrtss, 1.0 / that (vdivss).
 * Pass 2: y = cvtneps2bf16((x * inv) * w'), w' = w or w + 1.0 in f32. */
float oracle_rms_sumsq(const uint16_t *x, int dim)
{
    const int nb = dim / 32, nacc = nb < 4 ? nb : 4;
    float acc[4][16];
    memset(acc, 0, sizeof acc);
    for (int c = 0; c < nb; c++)
        for (int L = 0; L < 16; L++) {
            uint32_t pair;
            memcpy(&pair, x + 32 * c + 2 * L, 4);          /* low half: element 2L, high: 2L+1 */
            acc[c % nacc][L] = oracle_dpbf16_lane(acc[c % nacc][L], pair, pair);
        }
    for (int a = 1; a < nacc; a++)
        for (int L = 0; L < 16; L++) acc[0][L] = acc[0][L] + acc[a][L];
    return oracle_hsum16(acc[0]);
}

void oracle_rmsnorm(const uint16_t *x, const uint16_t *w, uint16_t *y, int dim, float eps, int plus_one)
{
    float s = oracle_rms_sumsq(x, dim);
    s = s * (1.0f / (float)dim);
    s = s + eps;
    s = sqrtf(s);
    const float inv = 1.0f / s;
    for (int i = 0; i < dim; i++) {
        float ww = f32(w[i]);
        if (plus_one) ww = ww + 1.0f;
        float v = f32(x[i]) * inv;
        v = v * ww;
        y[i] = oracle_cvtneps2bf16(v);
    }
}

/* emit_elem.rs:479-520: for i < dim/2, a = x[i], b = x[i + dim/2]:
 * a' = fma(-b, s, a * c) (vmulps then vfnmadd231ps), b' = fma(b, c, a * s)
 * (vmulps then vfmadd231ps), each rounded to bf16 with vcvtneps2bf16. */
void oracle_rope(uint16_t *x, const uint16_t *cos_row, const uint16_t *sin_row, int dim)
{
    const int half = dim / 2;
    for (int i = 0; i < half; i++) {
        const float a = f32(x[i]), b = f32(x[i + half]);
        const float c = f32(cos_row[i]), s = f32(sin_row[i]);
        const float ra = fmaf(-b, s, a * c);
        const float rb = fmaf(b, c, a * s);
        x[i] = oracle_cvtneps2bf16(ra);
        x[i + half] = oracle_cvtneps2bf16(rb);
    }
}

/* transforms.rs:32-81: per head, norm (in place, y = x) then rope; the rope
 * kernel is compiled at the rotary width, so it reaches only the first
 * `rotary` dimensions of the head (scheduler.rs, "a RoPE kernel per distinct
 * rotary_ndims"). */
void oracle_head_norm_rope(uint16_t *row, const uint16_t *w, const uint16_t *cos_row,
                           const uint16_t *sin_row, int heads, int stride, int dim, int rotary,
                           float eps, int plus_one)
{
    for (int h = 0; h < heads; h++) {
        uint16_t *x = row + (size_t)h * stride;
        oracle_rmsnorm(x, w, x, dim, eps, plus_one);
        oracle_rope(x, cos_row, sin_row, rotary);
    }
}

/* emit_elem.rs:350-440 (SigmoidMul arm): e = 0 - b (vxorps, vsubps);
 * e = vminps(e, 88): the second operand when either is NaN; exp_inline;
 * e = e + 1; y = cvtneps2bf16(a / e). */
void oracle_sigmoid_mul(const uint16_t *a, const uint16_t *b, uint16_t *y, int n)
{
    for (int i = 0; i < n; i++) {
        float e = 0.0f - f32(b[i]);
        e = e < 88.0f ? e : 88.0f;
        e = oracle_exp_poly(e);
        e = e + 1.0f;
        y[i] = oracle_cvtneps2bf16(f32(a[i]) / e);
    }
}
