/*
 * sdpa_oracle.h — TEST INFRASTRUCTURE ONLY.
 *
 * The oracle is what the HIP attention kernels are compared with: a CPU
 * restatement of the attention (SDPA) step that xigh/herbert-jit-bf16 emits at
 * run time as x86 AVX-512 BF16 machine code. Only tests/, the smoke check and
 * the CPU-baseline leg of bench.py may load it; the product library
 * (libhsdpa.so) never links or calls it.
 *
 * Two restatements of the same instruction sequence live behind this header:
 *   - sdpa_scalar.c : an exact scalar emulation (bit-for-bit the emitted code,
 *                     lane by lane), written from the reference emitters and
 *                     the public Intel SDM semantics of each instruction;
 *   - sdpa_avx512.c : the same sequence in AVX-512 BF16 intrinsics, threaded
 *                     like the reference's worker pool; it is the CPU baseline
 *                     and a second, independent check of the scalar one.
 *
 * Reference files restated (paths relative to the reference root):
 *   src/jit/target/x86/emit_sdpa/x86/{base,decode,prefill,assembly}.rs,
 *   src/jit/exp_constants.rs, src/jit/emit_sdpa.rs, src/jit/sdpa.rs,
 *   src/jit/target/x86/execution/attention.rs, src/jit/execution/abi.rs,
 *   src/core/tensor.rs.
 */
#ifndef SDPA_ORACLE_H
#define SDPA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- single-instruction semantics (scalar emulation) -------------------- */

/* bf16 -> f32, exact widening (src/core/tensor.rs:8-11). */
float oracle_bf16_to_f32(uint16_t b);
/* f32 -> bf16, integer round-to-nearest-even without NaN handling, as the
 * host helper of the engine writes it (src/core/tensor.rs:14-24,
 * src/jit/model.rs:904-908). */
uint16_t oracle_f32_to_bf16_rne(float x);
/* f32 -> bf16 as the kernels' epilogue instruction vcvtneps2bf16 does it
 * (src/jit/target/x86/emit_sdpa/x86/decode.rs:424): denormals to signed
 * zero, NaN quieted, otherwise RNE. */
uint16_t oracle_cvtneps2bf16(float x);
/* One f32 lane of vdpbf16ps: acc += a.odd*b.odd, then acc += a.even*b.even,
 * each an exact product added with one RNE rounding, DAZ on inputs and FTZ
 * on outputs (Intel SDM, VDPBF16PS). `a`, `b` hold the bf16 pair as
 * (odd << 16) | even. */
float oracle_dpbf16_lane(float acc, uint32_t a, uint32_t b);
/* The emitted exponential: src/jit/target/x86/emit_sdpa/x86/base.rs:189-212
 * with the constants of src/jit/exp_constants.rs:14-23. */
float oracle_exp_poly(float x);

/* ---- kernels (scalar emulation) ---------------------------------------- */

/* Decode head, Chained form with the default QK group (8), one query head
 * against `n` cached rows (src/jit/target/x86/emit_sdpa/x86/assembly.rs:116-174).
 * scores: at least roundup16(n) f32 of scratch. out: head_dim bf16. n >= 1. */
void oracle_sdpa_head(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                      float *scores, uint16_t *out, uint64_t n, float scale,
                      int head_dim);

/* Prefill block of `rows` consecutive queries of one head
 * (src/jit/target/x86/emit_sdpa/x86/prefill.rs:733-912). Row i sees
 * past+i+1 keys. q rows at stride q_row (u16), out rows at stride out_row.
 * scores: rows * roundup16(past+rows) f32 of scratch. */
void oracle_sdpa_prefill_block(const uint16_t *q, const uint16_t *k,
                               const uint16_t *v, float *scores, uint16_t *out,
                               uint64_t past, float scale, int head_dim,
                               int rows, size_t q_row, size_t out_row);

/* The same head and block with the knob sdpa_qk_group = 0
 * (src/jit/sdpa.rs:178-202): the row kernel's four accumulation chains
 * (decode.rs:59-128 with chains = 4, prefill.rs:104-157 with chains = 4),
 * whose score equals oracle_fused_qk_dot's; softmax and SV unchanged. */
void oracle_sdpa_head_qk0(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                          float *scores, uint16_t *out, uint64_t n, float scale,
                          int head_dim);
void oracle_sdpa_prefill_block_qk0(const uint16_t *q, const uint16_t *k,
                                   const uint16_t *v, float *scores, uint16_t *out,
                                   uint64_t past, float scale, int head_dim,
                                   int rows, size_t q_row, size_t out_row);

/* The head and the block with the softmax sink on (SdpaShape::sink,
 * src/jit/ir.rs:55-60): emit_softmax with sink_on (decode.rs:239-290). */
void oracle_sdpa_head_sink(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                           float *scores, uint16_t *out, uint64_t n, float scale,
                           int head_dim, float sink);
void oracle_sdpa_prefill_block_sink(const uint16_t *q, const uint16_t *k,
                                    const uint16_t *v, float *scores, uint16_t *out,
                                    uint64_t past, float scale, int head_dim,
                                    int rows, size_t q_row, size_t out_row, float sink);

/* The score of one (query, key) pair as the grouped QK computes it, before
 * the scale (single chain + the hsum tree, prefill.rs:302-331). */
float oracle_qk_dot(const uint16_t *q, const uint16_t *k, int head_dim);

/* ---- the attention node ------------------------------------------------- */

/* Per-layer geometry (src/jit/execution/abi.rs:136-151), strides in bf16
 * elements. */
typedef struct oracle_attention_spec {
    uint64_t heads;    /* query heads */
    uint64_t gqa;      /* query heads per KV head */
    uint64_t head_dim;
    uint64_t q_row;    /* elements between query rows */
    uint64_t q_head;   /* elements between query heads */
    uint64_t out_row;  /* elements between output rows */
} oracle_attention_spec;

/* Per-call addresses (src/jit/execution/abi.rs:156-180). */
typedef struct oracle_attention_call {
    const uint16_t *q;
    const uint16_t *keys;    /* [kv_heads][kv_stride], position p at p*head_dim */
    const uint16_t *values;
    uint16_t *output;
    uint64_t rows;
    uint64_t past;
    uint64_t kv_stride;      /* elements per KV head */
    float scale;
    float sink;              /* the sink value: 0 except under the sink forms of
                                oracle_attention_form (4 and 5) */
} oracle_attention_call;

/* The whole attention node, scalar emulation, single thread: task ->
 * (q head, chunk of 8 rows); a full chunk runs the prefill block, a partial
 * one the decode head per row with n = past + r + 1
 * (src/jit/target/x86/execution/attention.rs:105-224). Rows are processed
 * in passes of 256 like the engine (src/jit/schedule.rs:282-299). Returns 0,
 * or -1 on an invalid geometry. */
int oracle_attention_scalar(const oracle_attention_spec *spec,
                            const oracle_attention_call *call);

/* Geometry checks shared by both restatements: 0 when valid. */
int oracle_check_geometry(const oracle_attention_spec *spec,
                          const oracle_attention_call *call);

/* ---- the other decode forms (sdpa_forms.c) -------------------------------- */

/* The score of one position in the Fused form, before the scale: four
 * vdpbf16ps chains over the 32-element chunks, (w0 + w1) + (w2 + w3), hsum
 * (src/jit/target/x86/emit_sdpa/x86/decode.rs:551-580). */
float oracle_fused_qk_dot(const uint16_t *q, const uint16_t *k, int head_dim);
/* The Fused decode head (emit_fused, decode.rs:501-669): online softmax over
 * blocks of 16 positions. n = 0 writes zeros. acc_out (may be null) receives
 * the head_dim f32 accumulators before the bf16 conversion. Returns -1 above
 * head_dim 256 (the form declines, src/jit/ir.rs:146-148). */
int oracle_fused_head(const uint16_t *q, const uint16_t *k, const uint16_t *v, uint16_t *out, uint64_t n,
                      float scale, int head_dim, float *acc_out);
/* The AVX2 arm's QK score before the scale (even element then odd, four
 * chains over 16-element blocks, an 8-lane tree; emit_sdpa_avx2.rs:262-305). */
float oracle_avx2_qk_dot(const uint16_t *q, const uint16_t *k, int head_dim);
/* The AVX2 decode head (src/jit/target/x86/emit_sdpa_avx2.rs:231-470).
 * scores: at least roundup8(n) f32. Returns -1 when head_dim is not a
 * multiple of 16 (check_avx2). */
int oracle_avx2_head(const uint16_t *q, const uint16_t *k, const uint16_t *v, float *scores, uint16_t *out,
                     uint64_t n, float scale, int head_dim);
/* The same with the softmax sink on (emit_sdpa_avx2.rs:362-400). */
int oracle_avx2_head_sink(const uint16_t *q, const uint16_t *k, const uint16_t *v, float *scores, uint16_t *out,
                          uint64_t n, float scale, int head_dim, float sink);
/* oracle_exp_poly element by element over n floats. */
void oracle_exp_poly_n(const float *x, float *y, uint64_t n);
/* The AVX2 arm's integer round to nearest even (emit_sdpa_avx2.rs:208-217). */
uint16_t oracle_avx2_cvt_bf16(float x);
/* The attention node under a decode form: 0 Chained (as
 * oracle_attention_scalar), 1 Fused (full 8-row chunks still take the block
 * kernel; other rows the Fused head, or the Chained one above head_dim 256),
 * 2 AVX2 (every row the AVX2 head), 3 Chained with sdpa_qk_group = 0 (block
 * and head with the four-chain QK), 4 Chained with the softmax sink call->sink
 * (block and head), 5 AVX2 with the sink. The Fused form declines a sink
 * (src/jit/emit_sdpa.rs:468-470) and the engine runs the Chained one: form 4.
 * `threads` workers over (q head, row group) tasks. Returns 0 or -1. */
int oracle_attention_form(const oracle_attention_spec *spec, const oracle_attention_call *call, int form,
                          int threads);

/* ---- AVX-512 BF16 restatement (the CPU baseline) ------------------------ */

/* 1 if this host can run the AVX-512 BF16 path. */
int oracle_avx512_available(void);
/* The attention node on `threads` pinned workers (0 = one per physical
 * core), decode as Hq tasks and prefill as ceil(rows/8)*Hq block tasks per
 * pass of 256 rows, contiguous task ranges per worker. Returns 0, -1 on an
 * invalid geometry, -2 when AVX-512 BF16 is absent. */
int oracle_attention_avx512(const oracle_attention_spec *spec,
                            const oracle_attention_call *call, int threads);
/* Physical cores the pool would use by default. */
int oracle_physical_cores(void);
/* Compare oracle_dpbf16_lane with the hardware instruction on `lanes`
 * seeded random lanes (normal, denormal, zero and signed operands). Returns
 * the number of mismatching lanes, or -1 without AVX-512 BF16. */
long oracle_dpbf16_selfcheck(uint64_t seed, long lanes);
/* Compare oracle_cvtneps2bf16 and oracle_exp_poly with their intrinsic
 * sequences on `count` seeded inputs plus edge cases. Returns mismatches or
 * -1 without AVX-512 BF16. */
long oracle_cvt_exp_selfcheck(uint64_t seed, long count);

/* ---- The element kernels around the attention (elem_scalar.c) ------------
 * Restatements of the AVX-512 element kernels of
 * src/jit/target/x86/emit_elem.rs that the attention chain uses. */

/* The hsum tree of base.rs:258-267 / emit_elem.rs:175-183 on 16 lanes. */
float oracle_hsum16(const float *lanes);
/* The sum of squares of ElemOp::RmsNorm (emit_elem.rs:251-271): vdpbf16ps
 * chains, chain sums in order, hsum. */
float oracle_rms_sumsq(const uint16_t *x, int dim);
/* ElemOp::RmsNorm / RmsNormGemma (emit_elem.rs:239-335) on one vector of
 * `dim` bf16 (a multiple of 32): y may alias x. */
void oracle_rmsnorm(const uint16_t *x, const uint16_t *w, uint16_t *y, int dim, float eps, int plus_one);
/* ElemOp::Rope (emit_elem.rs:479-520), rotate_half, in place on `dim` bf16
 * with dim/2 cos and sin entries. */
void oracle_rope(uint16_t *x, const uint16_t *cos_row, const uint16_t *sin_row, int dim);
/* The head-norm-rope node on one row (transforms.rs:32-81 with the binding of
 * lowering.rs:549-577): for each of `heads` heads `stride` apart, the norm in
 * place, then the rope over its first `rotary` dimensions. */
void oracle_head_norm_rope(uint16_t *row, const uint16_t *w, const uint16_t *cos_row,
                           const uint16_t *sin_row, int heads, int stride, int dim, int rotary,
                           float eps, int plus_one);
/* ElemOp::SigmoidMul (emit_elem.rs:350-440): y = a / (1 + exp(min(0 - b, 88)))
 * on `n` bf16 (y may alias a). */
void oracle_sigmoid_mul(const uint16_t *a, const uint16_t *b, uint16_t *y, int n);

#ifdef __cplusplus
}
#endif
#endif
