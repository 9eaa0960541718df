/*
 * sdpa_avx512.c — TEST INFRASTRUCTURE ONLY (the oracle; see sdpa_oracle.h).
 *
 * The SDPA instruction sequence that herbert-jit-bf16 emits for AVX-512 BF16,
 * restated with compiler intrinsics, and scheduled like the engine's worker
 * pool. It is the CPU baseline reported beside the GPU numbers, and its
 * output must equal the scalar emulation (sdpa_scalar.c) bit for bit.
 *
 *   decode head   : assembly.rs:116-174 (QK group 8: prefill.rs:496-542,
 *                   qk_reduce prefill.rs:302-331, store_scores 348-359;
 *                   remainder emit_qk decode.rs:59-128 with one chain;
 *                   softmax decode.rs:212-293; SV decode.rs:348-428)
 *   prefill block : prefill.rs:733-912 (emit_qk_group 379-477 with
 *                   qk_pair 1, emit_qk_block 104-157, emit_sv_block 642-700)
 *   node          : attention.rs:105-224; task split entry.rs:411-428
 *   pool          : one worker per physical core, L3 groups interleaved
 *                   (src/pool/topology.rs:11-21,62-70)
 */
#define _GNU_SOURCE
#include "sdpa_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define AVX __attribute__((target("avx512f,avx512bw,avx512vl,avx512dq,avx512bf16,fma")))

static inline uint64_t roundup16(uint64_t n) { return (n + 15u) & ~(uint64_t)15u; }

/* ---- building blocks ------------------------------------------------------ */

AVX static inline __m512 dp(__m512 acc, __m512i a, __m512i b)
{
    return _mm512_dpbf16_ps(acc, (__m512bh)a, (__m512bh)b);
}

/* hsum (base.rs:258-267) */
AVX static inline float hsum(__m512 v)
{
    __m256 s = _mm256_add_ps(_mm512_castps512_ps256(v), _mm512_extractf32x8_ps(v, 1));
    __m128 t = _mm_add_ps(_mm256_castps256_ps128(s), _mm256_extractf128_ps(s, 1));
    t = _mm_hadd_ps(t, t);
    t = _mm_hadd_ps(t, t);
    return _mm_cvtss_f32(t);
}

/* hmax (base.rs:271-282) */
AVX static inline float hmax(__m512 v)
{
    __m256 s = _mm256_max_ps(_mm512_castps512_ps256(v), _mm512_extractf32x8_ps(v, 1));
    __m128 t = _mm_max_ps(_mm256_castps256_ps128(s), _mm256_extractf128_ps(s, 1));
    t = _mm_max_ps(t, _mm_shuffle_ps(t, t, 0x4E));
    t = _mm_max_ps(t, _mm_shuffle_ps(t, t, 0xB1));
    return _mm_cvtss_f32(t);
}

/* exp_inline (base.rs:189-212), constants exp_constants.rs:14-23 */
AVX static inline __m512 exp16(__m512 io)
{
    io = _mm512_max_ps(io, _mm512_set1_ps(-87.33654f));
    __m512 t1 = _mm512_mul_ps(io, _mm512_set1_ps(1.442695f));
    __m512 t2 = _mm512_roundscale_ps(t1, 0);
    t1 = _mm512_sub_ps(t1, t2);
    __m512 t3 = _mm512_set1_ps(0.00967248f);
    t3 = _mm512_fmadd_ps(t1, t3, _mm512_set1_ps(0.05550411f));
    t3 = _mm512_fmadd_ps(t1, t3, _mm512_set1_ps(0.2402265f));
    t3 = _mm512_fmadd_ps(t1, t3, _mm512_set1_ps(0.6931472f));
    t3 = _mm512_fmadd_ps(t1, t3, _mm512_set1_ps(1.0f));
    __m512i k = _mm512_cvtps_epi32(t2);
    k = _mm512_add_epi32(_mm512_slli_epi32(k, 23), _mm512_set1_epi32(0x3F800000));
    return _mm512_mul_ps(t3, _mm512_castsi512_ps(k));
}

/* qk_reduce at g = 8 (prefill.rs:302-331): four pairing levels, the last
 * one pairing the register with itself; 8 scores land duplicated in lanes
 * {0,1,4,5,8,9,12,13}. */
AVX static inline __m512 pair(__m512 a, __m512 b, int level)
{
    __m512 lo, hi;
    switch (level) {
    case 0: hi = _mm512_shuffle_f32x4(a, b, 0xEE); lo = _mm512_shuffle_f32x4(a, b, 0x44); break;
    case 1: hi = _mm512_shuffle_f32x4(a, b, 0xDD); lo = _mm512_shuffle_f32x4(a, b, 0x88); break;
    default: hi = _mm512_shuffle_ps(a, b, 0xDD); lo = _mm512_shuffle_ps(a, b, 0x88); break;
    }
    return _mm512_add_ps(lo, hi);
}

AVX static inline __m512 reduce8(const __m512 acc[8])
{
    __m512 r0 = pair(acc[0], acc[1], 0), r1 = pair(acc[2], acc[3], 0);
    __m512 r2 = pair(acc[4], acc[5], 0), r3 = pair(acc[6], acc[7], 0);
    __m512 s0 = pair(r0, r1, 1), s1 = pair(r2, r3, 1);
    __m512 u = pair(s0, s1, 2);
    return pair(u, u, 3);
}

/* qk_position (prefill.rs:268-278) at g = 8 */
static inline int qk_position8(int m) { return m < 4 ? 2 * m : 2 * (m - 4) + 1; }

/* One score with one chain and the hsum tree (emit_qk, one chain). */
AVX static inline float qk_one(const uint16_t *q, const uint16_t *k, int n32)
{
    __m512 acc = _mm512_setzero_ps();
    for (int c = 0; c < n32; c++)
        acc = dp(acc, _mm512_loadu_si512(k + 32 * c), _mm512_loadu_si512(q + 32 * c));
    return hsum(acc);
}

/* emit_softmax (decode.rs:212-293), no sink */
AVX static void softmax_avx(float *sc, uint64_t nb)
{
    __m512 maxv = _mm512_set1_ps(-INFINITY);
    for (uint64_t b = 0; b < nb; b++) maxv = _mm512_max_ps(maxv, _mm512_loadu_ps(sc + 16 * b));
    const __m512 m = _mm512_set1_ps(hmax(maxv));
    __m512 sumv = _mm512_setzero_ps();
    for (uint64_t b = 0; b < nb; b++) {
        __m512 w = exp16(_mm512_sub_ps(_mm512_loadu_ps(sc + 16 * b), m));
        sumv = _mm512_add_ps(sumv, w);
        _mm512_storeu_ps(sc + 16 * b, w);
    }
    const __m512 s = _mm512_set1_ps(hsum(sumv));
    for (uint64_t b = 0; b < nb; b++) _mm512_storeu_ps(sc + 16 * b, _mm512_div_ps(_mm512_loadu_ps(sc + 16 * b), s));
}

AVX static inline __m512 widen(const uint16_t *p)
{
    return _mm512_castsi512_ps(_mm512_slli_epi32(_mm512_cvtepu16_epi32(_mm256_loadu_si256((const __m256i *)p)), 16));
}

/* ---- the decode head ------------------------------------------------------ */

AVX static void head_avx(const uint16_t *q, const uint16_t *k, const uint16_t *v, float *sc,
                         uint16_t *out, uint64_t n, float scale, int d)
{
    const int n32 = d / 32, nv = d / 16;
    __m512i qv[16];
    for (int c = 0; c < n32; c++) qv[c] = _mm512_loadu_si512(q + 32 * c);
    const __m512 scv = _mm512_set1_ps(scale);
    const uint64_t groups = n >> 3;
    for (uint64_t g = 0; g < groups; g++) {
        const uint16_t *kg = k + (size_t)(8 * g) * d;
        __m512 acc[8];
        for (int m = 0; m < 8; m++) {
            const uint16_t *kr = kg + (size_t)qk_position8(m) * d;
            __m512 a = _mm512_setzero_ps();
            for (int c = 0; c < n32; c++) a = dp(a, qv[c], _mm512_loadu_si512(kr + 32 * c));
            acc[m] = a;
        }
        __m512 s = _mm512_mul_ps(reduce8(acc), scv);
        _mm512_mask_compressstoreu_ps(sc + 8 * g, 0x3333, s);
    }
    for (uint64_t j = groups * 8; j < n; j++) {
        __m128 t = _mm_mul_ss(_mm_set_ss(qk_one(q, k + (size_t)j * d, n32)), _mm_set_ss(scale));
        sc[j] = _mm_cvtss_f32(t);
    }
    for (uint64_t j = n; j < roundup16(n); j++) sc[j] = -INFINITY;
    softmax_avx(sc, roundup16(n) / 16);
    __m512 acc[32];
    for (int c = 0; c < nv; c++) acc[c] = _mm512_setzero_ps();
    for (uint64_t j = 0; j < n; j++) {
        const __m512 p = _mm512_set1_ps(sc[j]);
        const uint16_t *vr = v + (size_t)j * d;
        for (int c = 0; c < nv; c++) acc[c] = _mm512_fmadd_ps(widen(vr + 16 * c), p, acc[c]);
    }
    for (int c = 0; c < nv; c++) _mm256_storeu_si256((__m256i *)(out + 16 * c), (__m256i)_mm512_cvtneps_pbh(acc[c]));
}

/* ---- the prefill block (rows = 8) ----------------------------------------- */

AVX static void block_avx(const uint16_t *q, const uint16_t *k, const uint16_t *v, float *sc,
                          uint16_t *out, uint64_t past, float scale, int d, size_t q_row,
                          size_t out_row)
{
    enum { R = 8 };
    const int n32 = d / 32, nv = d / 16;
    const uint64_t N = past + R, rs = roundup16(N);
    const __m512 scv = _mm512_set1_ps(scale);
    const uint64_t groups = N >> 3;
    for (uint64_t g = 0; g < groups; g++) {
        const uint16_t *kg = k + (size_t)(8 * g) * d;
        for (int i = 0; i < R; i++) {
            const uint16_t *qi = q + i * q_row;
            __m512 acc[8];
            for (int m = 0; m < 8; m++) acc[m] = _mm512_setzero_ps();
            for (int m = 0; m < 8; m++) {
                const uint16_t *kr = kg + (size_t)qk_position8(m) * d;
                for (int c = 0; c < n32; c++)
                    acc[m] = dp(acc[m], _mm512_loadu_si512(qi + 32 * c), _mm512_loadu_si512(kr + 32 * c));
            }
            __m512 s = _mm512_mul_ps(reduce8(acc), scv);
            _mm512_mask_compressstoreu_ps(sc + i * rs + 8 * g, 0x3333, s);
        }
    }
    for (uint64_t j = groups * 8; j < N; j++)
        for (int i = 0; i < R; i++) {
            __m128 t = _mm_mul_ss(_mm_set_ss(qk_one(q + i * q_row, k + (size_t)j * d, n32)), _mm_set_ss(scale));
            sc[i * rs + j] = _mm_cvtss_f32(t);
        }
    for (int i = 0; i < R; i++) {
        const uint64_t ni = past + i + 1;
        for (uint64_t j = ni; j < roundup16(ni); j++) sc[i * rs + j] = -INFINITY;
        softmax_avx(sc + i * rs, roundup16(ni) / 16);
    }
    for (int i = 0; i < R; i++)
        for (int t = 0; t < R - 1 - i; t++) sc[i * rs + past + i + 1 + t] = 0.0f;
    /* SV: dimension groups of 32 outside, positions inside (nb = 2) */
    for (int g = 0; g < nv / 2; g++) {
        __m512 acc[R][2];
        for (int i = 0; i < R; i++) acc[i][0] = acc[i][1] = _mm512_setzero_ps();
        for (uint64_t j = 0; j < N; j++) {
            const uint16_t *vr = v + (size_t)j * d + 32 * g;
            const __m512 v0 = widen(vr), v1 = widen(vr + 16);
            for (int i = 0; i < R; i++) {
                const __m512 p = _mm512_set1_ps(sc[i * rs + j]);
                acc[i][0] = _mm512_fmadd_ps(v0, p, acc[i][0]);
                acc[i][1] = _mm512_fmadd_ps(v1, p, acc[i][1]);
            }
        }
        for (int i = 0; i < R; i++) {
            uint16_t *o = out + i * out_row + 32 * g;
            _mm256_storeu_si256((__m256i *)o, (__m256i)_mm512_cvtneps_pbh(acc[i][0]));
            _mm256_storeu_si256((__m256i *)(o + 16), (__m256i)_mm512_cvtneps_pbh(acc[i][1]));
        }
    }
}

/* ---- the pinned pool -------------------------------------------------------- */

static int read_int_file(const char *path, int *out)
{
    FILE *f = fopen(path, "r");
    if (!f) return -1;
    int ok = fscanf(f, "%d", out) == 1 ? 0 : -1;
    fclose(f);
    return ok;
}

/* First logical CPU of every physical core, L3 groups interleaved. */
static int core_ids(int *ids, int cap)
{
    int cpus[1024], l3[1024], n = 0;
    for (int c = 0; c < 1024 && n < cap; c++) {
        char p[256];
        snprintf(p, sizeof p, "/sys/devices/system/cpu/cpu%d/topology/thread_siblings_list", c);
        FILE *f = fopen(p, "r");
        if (!f) continue;
        int first = -1;
        if (fscanf(f, "%d", &first) != 1) first = -1;
        fclose(f);
        if (first != c) continue;
        snprintf(p, sizeof p, "/sys/devices/system/cpu/cpu%d/cache/index3/id", c);
        int id = 0;
        if (read_int_file(p, &id) != 0) id = 0;
        cpus[n] = c;
        l3[n] = id;
        n++;
    }
    if (n == 0) return 0;
    cpu_set_t allowed;
    if (sched_getaffinity(0, sizeof allowed, &allowed) == 0) {
        int m = 0;
        for (int i = 0; i < n; i++)
            if (CPU_ISSET(cpus[i], &allowed)) { cpus[m] = cpus[i]; l3[m] = l3[i]; m++; }
        n = m;
    }
    /* round-robin over L3 groups, in order of first appearance */
    int used[1024] = {0}, out = 0;
    while (out < n) {
        int seen[1024], ns = 0;
        for (int i = 0; i < n; i++) {
            if (used[i]) continue;
            int dup = 0;
            for (int s = 0; s < ns; s++) dup |= seen[s] == l3[i];
            if (dup) continue;
            seen[ns++] = l3[i];
            used[i] = 1;
            ids[out++] = cpus[i];
        }
    }
    return n;
}

int oracle_physical_cores(void)
{
    int ids[1024];
    int n = core_ids(ids, 1024);
    return n > 0 ? n : 1;
}

typedef struct job {
    const oracle_attention_spec *s;
    const oracle_attention_call *c;
    uint64_t p0, rows, past, chunks, tasks;
    int participants;
} job;

typedef struct pool {
    int n;
    pthread_t th[1024];
    int cpu[1024];
    pthread_mutex_t mu;
    pthread_cond_t go, done;
    uint64_t gen;
    int remaining;
    int quit;
    job j;
    float *scratch[1024];
    size_t scratch_len;
} pool;

static pool *g_pool;

AVX static void run_tasks(const job *j, int me, float *scratch)
{
    const oracle_attention_spec *s = j->s;
    const oracle_attention_call *c = j->c;
    /* entry.rs:411-428: contiguous ranges of ceil(tasks / participants) */
    const uint64_t per = (j->tasks + j->participants - 1) / j->participants;
    const uint64_t t0 = per * me, t1 = t0 + per < j->tasks ? t0 + per : j->tasks;
    const uint64_t d = s->head_dim;
    for (uint64_t task = t0; task < t1; task++) {
        const uint64_t h = task / j->chunks, ch = task % j->chunks, kvh = h / s->gqa;
        const uint64_t r0 = ch * 8, r1 = r0 + 8 < j->rows ? r0 + 8 : j->rows;
        const uint16_t *kk = c->keys + kvh * c->kv_stride, *vv = c->values + kvh * c->kv_stride;
        if (r1 - r0 == 8) {
            const uint64_t ar = j->p0 + r0;
            block_avx(c->q + ar * s->q_row + h * s->q_head, kk, vv, scratch,
                      c->output + ar * s->out_row + h * d, j->past + r0, c->scale, (int)d, s->q_row,
                      s->out_row);
        } else {
            for (uint64_t r = r0; r < r1; r++) {
                const uint64_t ar = j->p0 + r;
                head_avx(c->q + ar * s->q_row + h * s->q_head, kk, vv, scratch,
                         c->output + ar * s->out_row + h * d, j->past + r + 1, c->scale, (int)d);
            }
        }
    }
}

typedef struct warg { pool *p; int me; } warg;

static void *worker(void *arg)
{
    warg *w = (warg *)arg;
    pool *p = w->p;
    const int me = w->me;
    free(w);
    cpu_set_t set;
    CPU_ZERO(&set);
    CPU_SET(p->cpu[me], &set);
    pthread_setaffinity_np(pthread_self(), sizeof set, &set);
    uint64_t seen = 0;
    for (;;) {
        pthread_mutex_lock(&p->mu);
        while (p->gen == seen && !p->quit) pthread_cond_wait(&p->go, &p->mu);
        if (p->quit) { pthread_mutex_unlock(&p->mu); return NULL; }
        seen = p->gen;
        job j = p->j;
        pthread_mutex_unlock(&p->mu);
        if (me < j.participants) run_tasks(&j, me, p->scratch[me]);
        pthread_mutex_lock(&p->mu);
        if (--p->remaining == 0) pthread_cond_signal(&p->done);
        pthread_mutex_unlock(&p->mu);
    }
}

static void pool_destroy(pool *p)
{
    pthread_mutex_lock(&p->mu);
    p->quit = 1;
    pthread_cond_broadcast(&p->go);
    pthread_mutex_unlock(&p->mu);
    for (int i = 0; i < p->n; i++) pthread_join(p->th[i], NULL);
    for (int i = 0; i < p->n; i++) free(p->scratch[i]);
    free(p);
}

static pool *pool_get(int n)
{
    if (g_pool && g_pool->n == n) return g_pool;
    if (g_pool) { pool_destroy(g_pool); g_pool = NULL; }
    pool *p = (pool *)calloc(1, sizeof(pool));
    if (!p) return NULL;
    int ids[1024];
    int nc = core_ids(ids, 1024);
    for (int i = 0; i < n; i++) p->cpu[i] = nc > 0 ? ids[i % nc] : 0;
    p->n = n;
    pthread_mutex_init(&p->mu, NULL);
    pthread_cond_init(&p->go, NULL);
    pthread_cond_init(&p->done, NULL);
    for (int i = 0; i < n; i++) {
        warg *w = (warg *)malloc(sizeof(warg));
        w->p = p;
        w->me = i;
        pthread_create(&p->th[i], NULL, worker, w);
    }
    g_pool = p;
    return p;
}

static int pool_scratch(pool *p, size_t len)
{
    if (p->scratch_len >= len) return 0;
    for (int i = 0; i < p->n; i++) {
        free(p->scratch[i]);
        p->scratch[i] = (float *)aligned_alloc(64, ((len * sizeof(float)) + 63) & ~(size_t)63);
        if (!p->scratch[i]) return -1;
    }
    p->scratch_len = len;
    return 0;
}

int oracle_avx512_available(void)
{
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("avx512dq") &&
           __builtin_cpu_supports("avx512bf16");
}

int oracle_attention_avx512(const oracle_attention_spec *s, const oracle_attention_call *c, int threads)
{
    if (!oracle_avx512_available()) return -2;
    if (oracle_check_geometry(s, c) != 0) return -1;
    if (c->rows == 0) return 0;
    if (threads <= 0) threads = oracle_physical_cores();
    if (threads > 1024) threads = 1024;
    pool *p = pool_get(threads);
    if (!p) return -1;
    if (pool_scratch(p, 8 * roundup16(c->past + c->rows + 16)) != 0) return -1;
    for (uint64_t p0 = 0; p0 < c->rows; p0 += 256) {
        job j;
        j.s = s;
        j.c = c;
        j.p0 = p0;
        j.rows = c->rows - p0 < 256 ? c->rows - p0 : 256;
        j.past = c->past + p0;
        j.chunks = (j.rows + 7) / 8;
        j.tasks = j.chunks * s->heads;
        j.participants = threads;
        pthread_mutex_lock(&p->mu);
        p->j = j;
        p->remaining = p->n;
        p->gen++;
        pthread_cond_broadcast(&p->go);
        while (p->remaining > 0) pthread_cond_wait(&p->done, &p->mu);
        pthread_mutex_unlock(&p->mu);
    }
    return 0;
}

/* ---- self-checks of the scalar emulation against the hardware ------------- */

static inline uint64_t splitmix(uint64_t *s)
{
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* bf16 bit patterns biased toward the cases that tell the rules apart:
 * ordinary normals, denormals, zeros of both signs, tiny exponents. */
static uint16_t pick_bf16(uint64_t *s)
{
    uint64_t r = splitmix(s);
    uint16_t sign = (uint16_t)((r >> 63) << 15);
    switch (r & 7) {
    case 0: return sign | (uint16_t)((r >> 8) & 0x7F);                 /* denormal or zero */
    case 1: return sign | (uint16_t)(0x0080 + ((r >> 8) & 0x3FF));     /* near the bottom */
    default: return sign | (uint16_t)(0x3C00 + ((r >> 8) & 0x07FF));  /* around 1 */
    }
}

AVX static long dp_check(uint64_t seed, long lanes)
{
    uint64_t st = seed;
    long bad = 0;
    for (long done = 0; done < lanes; done += 16) {
        uint32_t a[16], b[16];
        float acc[16], hw[16];
        for (int L = 0; L < 16; L++) {
            a[L] = ((uint32_t)pick_bf16(&st) << 16) | pick_bf16(&st);
            b[L] = ((uint32_t)pick_bf16(&st) << 16) | pick_bf16(&st);
            uint64_t r = splitmix(&st);
            uint32_t ab = (uint32_t)r;
            if ((r >> 32) % 8 == 0) ab &= 0x807FFFFFu;   /* denormal accumulator */
            else ab = (ab & 0x80FFFFFFu) | 0x3C000000u;
            memcpy(&acc[L], &ab, 4);
        }
        __m512 r = dp(_mm512_loadu_ps(acc), _mm512_loadu_si512(a), _mm512_loadu_si512(b));
        _mm512_storeu_ps(hw, r);
        for (int L = 0; L < 16; L++) {
            float e = oracle_dpbf16_lane(acc[L], a[L], b[L]);
            uint32_t x, y;
            memcpy(&x, &e, 4);
            memcpy(&y, &hw[L], 4);
            bad += x != y;
        }
    }
    return bad;
}

long oracle_dpbf16_selfcheck(uint64_t seed, long lanes)
{
    if (!oracle_avx512_available()) return -1;
    return dp_check(seed, lanes);
}

AVX static long cvt_exp_check(uint64_t seed, long count)
{
    uint64_t st = seed;
    long bad = 0;
    static const uint32_t edges[] = {0x00000000u, 0x80000000u, 0x00000001u, 0x807FFFFFu, 0x7F800000u,
                                     0xFF800000u, 0x7FC00001u, 0xFF812345u, 0x3F808000u, 0x3F818000u,
                                     0x3F80FFFFu, 0x7F7FFFFFu, 0x00800000u, 0xC2AEAC50u, 0xC2AF0000u};
    const long ne = (long)(sizeof edges / sizeof edges[0]);
    for (long i = 0; i < count + ne; i += 16) {
        float x[16], y[16];
        for (int L = 0; L < 16; L++) {
            long idx = i + L;
            uint32_t bits;
            if (idx < ne) bits = edges[idx];
            else {
                uint64_t r = splitmix(&st);
                bits = (uint32_t)r;
                if ((r >> 40) & 1) { /* exp domain: scores minus max, in [-100, 0] */
                    float f = -(float)((r >> 41) % 100000000ull) * 1e-6f;
                    memcpy(&bits, &f, 4);
                }
            }
            memcpy(&x[L], &bits, 4);
        }
        uint16_t hw16[16];
        _mm256_storeu_si256((__m256i *)hw16, (__m256i)_mm512_cvtneps_pbh(_mm512_loadu_ps(x)));
        _mm512_storeu_ps(y, exp16(_mm512_loadu_ps(x)));
        for (int L = 0; L < 16; L++) {
            bad += oracle_cvtneps2bf16(x[L]) != hw16[L];
            uint32_t xb;
            memcpy(&xb, &x[L], 4);
            if ((xb & 0x7F800000u) == 0x7F800000u && (xb & 0x7FFFFFu)) continue; /* NaN in */
            float e = oracle_exp_poly(x[L]);
            uint32_t p, q;
            memcpy(&p, &e, 4);
            memcpy(&q, &y[L], 4);
            if (e != e && y[L] != y[L]) continue; /* both NaN */
            bad += p != q;
        }
    }
    return bad;
}

long oracle_cvt_exp_selfcheck(uint64_t seed, long count)
{
    if (!oracle_avx512_available()) return -1;
    return cvt_exp_check(seed, count);
}
