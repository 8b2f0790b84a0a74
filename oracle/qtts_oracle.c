/*
 * qtts_oracle.c — CPU restatement of the QORA-TTS per-frame decode path.
 *
 * TEST INFRASTRUCTURE.  This file is the oracle the HIP path is checked
 * against and the CPU baseline bench.py times.  It is never linked into the
 * product library.  Build: oracle/Makefile (-O2 -mavx2 -ffp-contract=off,
 * no fast-math), so every f32 operation below rounds exactly once, in the
 * order the cited Rust code performs it.
 *
 * Citations are to the reference crate's src/ files (file:line).
 */
#define _GNU_SOURCE
#include "qtts_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

#define GROUP 32            /* Q4_GROUP_SIZE, gemv.rs:18 */
#define PACKED_PER_GROUP 16

/* ===================================================================== */
/* conversions and RNG                                                    */
/* ===================================================================== */

/* half::f16::to_f32 — exact for every f16 (IEEE binary16 -> binary32). */
float oq_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {                      /* subnormal: normalise */
            int e = -1;
            do { man <<= 1; e++; } while ((man & 0x400u) == 0);
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* half::f16::from_f32 — round to nearest, ties to even; overflow -> inf,
 * NaN stays NaN (quiet). */
uint16_t oq_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFF) {
        return (uint16_t)(sign | 0x7C00u | (man ? (0x200u | (man >> 13)) : 0));
    }
    int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;          /* rounds to zero */
        man |= 0x800000u;                             /* implicit bit   */
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half_m = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half_m & 1u))) half_m++;
        return (uint16_t)(sign | half_m);
    }
    uint32_t half_m = man >> 13;
    uint32_t rem = man & 0x1FFFu;
    uint32_t out = sign | ((uint32_t)e << 10) | half_m;
    if (rem > 0x1000u || (rem == 0x1000u && (half_m & 1u))) out++;  /* may carry into exp: correct */
    return (uint16_t)out;
}

/* xorshift64 with shifts 13/7/17 (gemv.rs:693-698, generate_new.rs:18-20). */
uint64_t oq_xorshift(uint64_t *s)
{
    *s ^= *s << 13;
    *s ^= *s >> 7;
    *s ^= *s << 17;
    return *s;
}

/* simple_rand (generate_new.rs:17-22): (state as f32) / (u64::MAX as f32).
 * Both conversions round to nearest-even; u64::MAX becomes 2^64. */
float oq_simple_rand(uint64_t *s)
{
    oq_xorshift(s);
    float num = (float)*s;
    float den = (float)UINT64_MAX;
    return num / den;
}

/* ===================================================================== */
/* Q4 GEMV kernels                                                        */
/* ===================================================================== */

/* gemv_q4_scalar (gemv.rs:249-287). */
void oq_gemv_q4_scalar(const float *x, const uint8_t *packed,
                       const uint16_t *scales, int64_t n, int64_t k0,
                       int64_t k1, float *out)
{
    const int64_t groups = n / GROUP;
    const int64_t row_bytes = groups * PACKED_PER_GROUP;
    memset(out, 0, (size_t)n * sizeof(float));
    for (int64_t ki = k0; ki < k1; ki++) {
        const float xv = x[ki];
        if (xv == 0.0f) continue;
        const int64_t sb = ki * groups;
        const int64_t pb = ki * row_bytes;
        for (int64_t g = 0; g < groups; g++) {
            const float s = oq_f16_to_f32(scales[sb + g]) * xv;
            if (s == 0.0f) continue;
            float lut[16];
            for (int i = 0; i < 16; i++) lut[i] = (i == 8) ? 0.0f : s * (float)(i - 8);
            const uint8_t *p = packed + pb + g * PACKED_PER_GROUP;
            float *o = out + g * GROUP;
            for (int j = 0; j < PACKED_PER_GROUP; j++) {
                const uint8_t b = p[j];
                o[2 * j] += lut[b & 0x0F];
                o[2 * j + 1] += lut[b >> 4];
            }
        }
    }
}

/* gemv_q4_avx2 (simd.rs:76-153): (cvt(nib) - 8) * s per lane, k-major
 * accumulation, interleaved back to column order. */
__attribute__((target("avx2")))
static void gemv_q4_avx2_impl(const float *x, const uint8_t *packed,
                              const uint16_t *scales, int64_t n, int64_t k0,
                              int64_t k1, float *out)
{
    const int64_t groups = n / GROUP;
    const int64_t row_bytes = groups * PACKED_PER_GROUP;
    memset(out, 0, (size_t)n * sizeof(float));
    const __m256i mask = _mm256_set1_epi32(0x0F);
    const __m256 eight = _mm256_set1_ps(8.0f);
    for (int64_t ki = k0; ki < k1; ki++) {
        const float xv = x[ki];
        if (xv == 0.0f) continue;
        const int64_t sb = ki * groups;
        const int64_t pb = ki * row_bytes;
        for (int64_t g = 0; g < groups; g++) {
            const float s = oq_f16_to_f32(scales[sb + g]) * xv;
            if (s == 0.0f) continue;
            const __m256 sv = _mm256_set1_ps(s);
            const __m128i bytes =
                _mm_loadu_si128((const __m128i *)(packed + pb + g * PACKED_PER_GROUP));
            for (int h = 0; h < 2; h++) {
                const __m128i half = h == 0 ? bytes : _mm_srli_si128(bytes, 8);
                const __m256i v8 = _mm256_cvtepu8_epi32(half);
                const __m256i lo = _mm256_and_si256(v8, mask);
                const __m256i hi = _mm256_srli_epi32(v8, 4);
                const __m256 lov = _mm256_mul_ps(_mm256_sub_ps(_mm256_cvtepi32_ps(lo), eight), sv);
                const __m256 hiv = _mm256_mul_ps(_mm256_sub_ps(_mm256_cvtepi32_ps(hi), eight), sv);
                const __m256 a = _mm256_unpacklo_ps(lov, hiv);
                const __m256 b = _mm256_unpackhi_ps(lov, hiv);
                const __m256 first = _mm256_permute2f128_ps(a, b, 0x20);
                const __m256 second = _mm256_permute2f128_ps(a, b, 0x31);
                float *o = out + g * GROUP + h * 16;
                _mm256_storeu_ps(o, _mm256_add_ps(_mm256_loadu_ps(o), first));
                _mm256_storeu_ps(o + 8, _mm256_add_ps(_mm256_loadu_ps(o + 8), second));
            }
        }
    }
}

static int host_has_avx2(void)
{
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2");
}

int oq_gemv_q4_avx2(const float *x, const uint8_t *packed,
                    const uint16_t *scales, int64_t n, int64_t k0, int64_t k1,
                    float *out)
{
    if (!host_has_avx2()) return 0;
    gemv_q4_avx2_impl(x, packed, scales, n, k0, k1, out);
    return 1;
}

/* gemv_q4_avx512 (simd.rs:203-269): per group the 16-entry table
 * lut = (q - 8) * s as one 16-lane product, the low and high nibbles of the
 * 16 packed bytes looked up in it, then interleaved back to column order
 * (lanes 0,16,1,17,... and 8,24,9,25,...) and added to the outputs. */
__attribute__((target("avx512f")))
static void gemv_q4_avx512_impl(const float *x, const uint8_t *packed,
                                const uint16_t *scales, int64_t n, int64_t k0,
                                int64_t k1, float *out)
{
    const int64_t groups = n / GROUP;
    const int64_t row_bytes = groups * PACKED_PER_GROUP;
    memset(out, 0, (size_t)n * sizeof(float));
    float fac[16];
    int32_t il_first[16], il_second[16];
    for (int i = 0; i < 16; i++) {
        fac[i] = (float)(i - 8);
        il_first[i] = (i & 1) ? 16 + i / 2 : i / 2;        /* lo[i/2] or hi[i/2]       */
        il_second[i] = (i & 1) ? 24 + i / 2 : 8 + i / 2;   /* lo[8+i/2] or hi[8+i/2]   */
    }
    const __m512 factors = _mm512_loadu_ps(fac);
    const __m512i ilo = _mm512_loadu_si512((const void *)il_first);
    const __m512i ihi = _mm512_loadu_si512((const void *)il_second);
    const __m512i mask = _mm512_set1_epi32(0x0F);
    for (int64_t ki = k0; ki < k1; ki++) {
        const float xv = x[ki];
        if (xv == 0.0f) continue;
        const int64_t sb = ki * groups;
        const int64_t pb = ki * row_bytes;
        for (int64_t g = 0; g < groups; g++) {
            const float s = oq_f16_to_f32(scales[sb + g]) * xv;
            if (s == 0.0f) continue;
            const __m512 lut = _mm512_mul_ps(factors, _mm512_set1_ps(s));
            const __m128i bytes =
                _mm_loadu_si128((const __m128i *)(packed + pb + g * PACKED_PER_GROUP));
            const __m512i b32 = _mm512_cvtepu8_epi32(bytes);
            const __m512 lov = _mm512_permutexvar_ps(_mm512_and_epi32(b32, mask), lut);
            const __m512 hiv = _mm512_permutexvar_ps(_mm512_srli_epi32(b32, 4), lut);
            const __m512 first = _mm512_permutex2var_ps(lov, ilo, hiv);
            const __m512 second = _mm512_permutex2var_ps(lov, ihi, hiv);
            float *o = out + g * GROUP;
            _mm512_storeu_ps(o, _mm512_add_ps(_mm512_loadu_ps(o), first));
            _mm512_storeu_ps(o + 16, _mm512_add_ps(_mm512_loadu_ps(o + 16), second));
        }
    }
}

static int host_has_avx512(void)
{
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f");
}

int oq_gemv_q4_avx512(const float *x, const uint8_t *packed,
                      const uint16_t *scales, int64_t n, int64_t k0, int64_t k1,
                      float *out)
{
    if (!host_has_avx512()) return 0;
    gemv_q4_avx512_impl(x, packed, scales, n, k0, k1, out);
    return 1;
}

/* ISA of the inner kernel: -1 as gemv_q4_inner picks it (gemv.rs:230-243:
 * AVX-512 when the host has it, else AVX2, else scalar), or forced to
 * OQ_ISA_SCALAR / OQ_ISA_AVX2 / OQ_ISA_AVX512 (when the host has it).  All
 * three are bit-identical to the scalar kernel. */
static int g_isa = -1;

int oq_set_isa(int isa)
{
    if (isa == OQ_ISA_AVX512 && !host_has_avx512()) return -1;
    if (isa == OQ_ISA_AVX2 && !host_has_avx2()) return -1;
    g_isa = isa;
    return oq_get_isa();
}

int oq_get_isa(void)
{
    if (g_isa >= 0) return g_isa;
    return host_has_avx512() ? OQ_ISA_AVX512 : host_has_avx2() ? OQ_ISA_AVX2 : OQ_ISA_SCALAR;
}

/* The inner kernel the chunked GEMV calls. */
static void gemv_inner(const float *x, const uint8_t *packed,
                       const uint16_t *scales, int64_t n, int64_t k0,
                       int64_t k1, float *out)
{
    switch (oq_get_isa()) {
    case OQ_ISA_AVX512: gemv_q4_avx512_impl(x, packed, scales, n, k0, k1, out); break;
    case OQ_ISA_AVX2: gemv_q4_avx2_impl(x, packed, scales, n, k0, k1, out); break;
    default: oq_gemv_q4_scalar(x, packed, scales, n, k0, k1, out); break;
    }
}

/* ---- persistent chunk pool (gpool.rs:17-66 restated with pthreads) ---- */

static int g_workers = 16;     /* gpool.rs:29-34 default min(avail,16) */
static int g_threads = 0;

typedef struct {
    const float *x;
    const qtts_q4_host *w;
    int64_t chunk_k, num_chunks;
    float *parts;
    atomic_long next;
    atomic_long done;
} gemv_job;

static pthread_mutex_t pool_mu = PTHREAD_MUTEX_INITIALIZER;
static pthread_cond_t pool_cv = PTHREAD_COND_INITIALIZER;
static pthread_cond_t pool_done_cv = PTHREAD_COND_INITIALIZER;
static gemv_job *pool_job = NULL;
static long pool_gen = 0;
static int pool_started = 0;
static int pool_nthreads = 0;
static int pool_active = 0;     /* workers holding a pointer to pool_job */

static void run_chunks(gemv_job *j)
{
    for (;;) {
        long c = atomic_fetch_add(&j->next, 1);
        if (c >= j->num_chunks) break;
        int64_t k0 = c * j->chunk_k;
        int64_t k1 = (c + 1) * j->chunk_k;
        if (k1 > j->w->k) k1 = j->w->k;
        if (k0 > k1) k0 = k1;
        gemv_inner(j->x, j->w->packed, j->w->scales, j->w->n, k0, k1,
                   j->parts + c * j->w->n);
        atomic_fetch_add(&j->done, 1);
    }
}

static void *pool_main(void *arg)
{
    (void)arg;
    long seen = 0;
    for (;;) {
        pthread_mutex_lock(&pool_mu);
        while (pool_gen == seen) pthread_cond_wait(&pool_cv, &pool_mu);
        seen = pool_gen;
        gemv_job *j = pool_job;
        if (j) pool_active++;
        pthread_mutex_unlock(&pool_mu);
        if (j) {
            run_chunks(j);
            pthread_mutex_lock(&pool_mu);
            pool_active--;
            pthread_cond_broadcast(&pool_done_cv);
            pthread_mutex_unlock(&pool_mu);
        }
    }
    return NULL;
}

static void pool_ensure(int threads)
{
    pthread_mutex_lock(&pool_mu);
    while (pool_nthreads < threads - 1) {   /* the caller is one worker */
        pthread_t t;
        pthread_create(&t, NULL, pool_main, NULL);
        pthread_detach(t);
        pool_nthreads++;
    }
    pool_started = 1;
    pthread_mutex_unlock(&pool_mu);
}

void oq_set_workers(int workers, int threads)
{
    g_workers = workers < 1 ? 1 : workers;
    g_threads = threads;
    if (threads > 1) pool_ensure(threads);
}

int oq_get_workers(void) { return g_workers; }

/* gemv_q4 (gemv.rs:290-346). */
void oq_gemv_q4(const float *x, const qtts_q4_host *w, float *out)
{
    const int64_t k = w->k, n = w->n;
    int64_t nt = (k * n) / 500000;
    if (nt < 1) nt = 1;
    if (nt > g_workers) nt = g_workers;
    if (k * n < 500000) nt = 1;
    if (nt <= 1) {
        gemv_inner(x, w->packed, w->scales, n, 0, k, out);
        return;
    }
    int64_t num_chunks = nt * 4;
    if (num_chunks > k) num_chunks = k;
    if (num_chunks < nt) num_chunks = nt;
    const int64_t chunk_k = (k + num_chunks - 1) / num_chunks;
    float *parts = (float *)malloc((size_t)num_chunks * n * sizeof(float));
    gemv_job j;
    j.x = x; j.w = w; j.chunk_k = chunk_k; j.num_chunks = num_chunks;
    j.parts = parts;
    atomic_init(&j.next, 0);
    atomic_init(&j.done, 0);
    if (g_threads > 1 && pool_started) {
        pthread_mutex_lock(&pool_mu);
        pool_job = &j;
        pool_gen++;
        pthread_cond_broadcast(&pool_cv);
        pthread_mutex_unlock(&pool_mu);
        run_chunks(&j);
        pthread_mutex_lock(&pool_mu);
        /* the job lives on this stack: wait until no worker still holds it */
        while (atomic_load(&j.done) < num_chunks || pool_active > 0)
            pthread_cond_wait(&pool_done_cv, &pool_mu);
        pool_job = NULL;
        pthread_mutex_unlock(&pool_mu);
    } else {
        run_chunks(&j);
    }
    /* partials summed in chunk order into a zeroed vector (gemv.rs:340-345) */
    memset(out, 0, (size_t)n * sizeof(float));
    for (int64_t c = 0; c < num_chunks; c++) {
        const float *p = parts + c * n;
        for (int64_t i = 0; i < n; i++) out[i] += p[i];
    }
    free(parts);
}

/* gemm_q4 (gemv.rs:349-412): every row is a full-k gemv_q4_inner. */
void oq_gemm_q4(const float *X, int64_t rows, const qtts_q4_host *w, float *Y)
{
    for (int64_t t = 0; t < rows; t++)
        gemv_inner(X + t * w->k, w->packed, w->scales, w->n, 0, w->k,
                   Y + t * w->n);
}

/* embed_lookup_q4 (gemv.rs:415-437), talker.rs:119-142. */
void oq_embed_lookup_q4(const qtts_q4_host *w, int64_t row, int64_t width,
                        float *out)
{
    const int64_t groups = width / GROUP;
    const int64_t sb = row * groups;
    const int64_t pb = row * groups * PACKED_PER_GROUP;
    memset(out, 0, (size_t)width * sizeof(float));
    for (int64_t g = 0; g < groups; g++) {
        const float sc = oq_f16_to_f32(w->scales[sb + g]);
        const uint8_t *p = w->packed + pb + g * PACKED_PER_GROUP;
        for (int j = 0; j < PACKED_PER_GROUP; j++) {
            const int q0 = (int)(p[j] & 0x0F) - 8;
            const int q1 = (int)((p[j] >> 4) & 0x0F) - 8;
            out[g * GROUP + 2 * j] = sc * (float)q0;
            out[g * GROUP + 2 * j + 1] = sc * (float)q1;
        }
    }
}

/* quantize_f32_to_q4 (gemv.rs:92-130). */
void oq_quantize_q4(const float *data, int64_t k, int64_t n, uint8_t *packed,
                    uint16_t *scales)
{
    const int64_t groups = n / GROUP;
    for (int64_t ki = 0; ki < k; ki++) {
        for (int64_t g = 0; g < groups; g++) {
            const int64_t gi = ki * groups + g;
            const int64_t c0 = g * GROUP;
            float absmax = 0.0f;
            for (int j = 0; j < GROUP; j++) {
                float v = fabsf(data[ki * n + c0 + j]);
                if (v > absmax) absmax = v;
            }
            const float scale = absmax / 7.0f;
            scales[gi] = oq_f32_to_f16(scale);
            const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
            for (int j = 0; j < GROUP; j += 2) {
                float r0 = roundf(data[ki * n + c0 + j] * inv);      /* half away from zero, as Rust */
                float r1 = roundf(data[ki * n + c0 + j + 1] * inv);
                r0 = r0 < -8.0f ? -8.0f : (r0 > 7.0f ? 7.0f : r0);
                r1 = r1 < -8.0f ? -8.0f : (r1 > 7.0f ? 7.0f : r1);
                const uint8_t q0 = (uint8_t)(r0 + 8.0f);
                const uint8_t q1 = (uint8_t)(r1 + 8.0f);
                packed[gi * PACKED_PER_GROUP + j / 2] = (uint8_t)(q0 | (q1 << 4));
            }
        }
    }
}

/* ===================================================================== */
/* elementwise                                                            */
/* ===================================================================== */

/* rms_norm_f16 (gemv.rs:445-454). */
void oq_rms_norm_f16(const float *x, const uint16_t *gamma, int64_t n,
                     float *out)
{
    float ss = 0.0f;
    for (int64_t i = 0; i < n; i++) ss += x[i] * x[i];
    const float inv = 1.0f / sqrtf(ss / (float)n + 1e-6f);
    for (int64_t i = 0; i < n; i++) out[i] = x[i] * inv * oq_f16_to_f32(gamma[i]);
}

/* softmax_raw (gemv.rs:471-482). */
void oq_softmax_raw(float *s, int64_t n)
{
    float mx = -INFINITY;
    for (int64_t i = 0; i < n; i++) mx = fmaxf(mx, s[i]);
    float sum = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        s[i] = expf(s[i] - mx);
        sum += s[i];
    }
    const float inv = 1.0f / sum;
    for (int64_t i = 0; i < n; i++) s[i] *= inv;
}

/* silu (gemv.rs:486-488). */
float oq_silu(float x) { return x / (1.0f + expf(-x)); }

/* apply_qk_norm (talker.rs:89-99, code_predictor.rs:84-93). */
void oq_qk_norm(float *d, int64_t heads, int64_t hd, const uint16_t *gamma)
{
    for (int64_t h = 0; h < heads; h++) {
        float *v = d + h * hd;
        float ss = 0.0f;
        for (int64_t i = 0; i < hd; i++) ss += v[i] * v[i];
        const float inv = 1.0f / sqrtf(ss / (float)hd + 1e-6f);
        for (int64_t i = 0; i < hd; i++) v[i] = v[i] * inv * oq_f16_to_f32(gamma[i]);
    }
}

/* build_mrope_tables (rope.rs:11-41).  With sections [24,20,20] the dim
 * index runs 0..63 continuously, so the table equals the predictor's
 * standard table (loader.rs:393-408): f64 angle, cast to f32. */
void oq_rope_table(int64_t head_dim, int64_t max_pos, double theta,
                   float *cos_t, float *sin_t)
{
    const int64_t half = head_dim / 2;
    for (int64_t i = 0; i < half; i++) {
        const double freq = 1.0 / pow(theta, (double)(2 * i) / (double)head_dim);
        for (int64_t pos = 0; pos < max_pos; pos++) {
            const double ang = (double)pos * freq;
            cos_t[pos * half + i] = (float)cos(ang);
            sin_t[pos * half + i] = (float)sin(ang);
        }
    }
}

/* apply_mrope_interleaved with equal section positions (rope.rs:51-93) and
 * apply_rope_split (code_predictor.rs:97-121): rotate-half pairs (i, i+64). */
void oq_rope_apply(float *d, int64_t heads, int64_t hd, int64_t pos,
                   const float *cos_t, const float *sin_t, int64_t rows)
{
    const int64_t half = hd / 2;
    if (pos + 1 > rows) return;          /* code_predictor.rs:107 */
    const float *c = cos_t + pos * half;
    const float *s = sin_t + pos * half;
    for (int64_t h = 0; h < heads; h++) {
        float *b = d + h * hd;
        for (int64_t i = 0; i < half; i++) {
            const float x1 = b[i], x2 = b[half + i];
            b[i] = x1 * c[i] - x2 * s[i];
            b[half + i] = x2 * c[i] + x1 * s[i];
        }
    }
}

/* ===================================================================== */
/* KV cache                                                               */
/* ===================================================================== */

oq_kv *oq_kv_new(int32_t n_layers, int32_t n_kv, int32_t hd, int64_t cap)
{
    oq_kv *kv = (oq_kv *)calloc(1, sizeof(oq_kv));
    kv->n_layers = n_layers; kv->n_kv = n_kv; kv->hd = hd; kv->cap = cap;
    kv->len = (int64_t *)calloc((size_t)n_layers, sizeof(int64_t));
    kv->K = (float **)calloc((size_t)n_layers, sizeof(float *));
    kv->V = (float **)calloc((size_t)n_layers, sizeof(float *));
    for (int l = 0; l < n_layers; l++) {
        kv->K[l] = (float *)calloc((size_t)cap * n_kv * hd, sizeof(float));
        kv->V[l] = (float *)calloc((size_t)cap * n_kv * hd, sizeof(float));
    }
    return kv;
}

void oq_kv_free(oq_kv *kv)
{
    if (!kv) return;
    for (int l = 0; l < kv->n_layers; l++) { free(kv->K[l]); free(kv->V[l]); }
    free(kv->K); free(kv->V); free(kv->len); free(kv);
}

void oq_kv_reset(oq_kv *kv) { for (int l = 0; l < kv->n_layers; l++) kv->len[l] = 0; }
float *oq_kv_k(oq_kv *kv, int32_t l) { return kv->K[l]; }
float *oq_kv_v(oq_kv *kv, int32_t l) { return kv->V[l]; }
int64_t oq_kv_len(oq_kv *kv, int32_t l) { return kv->len[l]; }
void oq_kv_set_len(oq_kv *kv, int64_t len) { for (int l = 0; l < kv->n_layers; l++) kv->len[l] = len; }

/* ===================================================================== */
/* one decoder layer, decode (talker.rs:274-350, code_predictor.rs:450-510) */
/* ===================================================================== */

typedef struct {
    int64_t hidden, n_heads, n_kv, hd, inter;
    const float *cos_t, *sin_t;
    int64_t rope_rows;
} layer_dims;

/* GQA decode attention over kv_len cached positions (talker.rs:304-331). */
static void decode_attention(const layer_dims *d, const float *q,
                             const float *K, const float *V, int64_t kv_len,
                             float *out)
{
    const int64_t groups = d->n_heads / d->n_kv;
    const float scale = 1.0f / sqrtf((float)d->hd);
    const int64_t stride = d->n_kv * d->hd;
    float *scores = (float *)malloc((size_t)(kv_len > 0 ? kv_len : 1) * sizeof(float));
    memset(out, 0, (size_t)(d->n_heads * d->hd) * sizeof(float));
    for (int64_t h = 0; h < d->n_heads; h++) {
        const int64_t kvh = h / groups;
        const float *qv = q + h * d->hd;
        for (int64_t s = 0; s < kv_len; s++) {
            const float *kr = K + s * stride + kvh * d->hd;
            float dot = 0.0f;
            for (int64_t i = 0; i < d->hd; i++) dot += qv[i] * kr[i];
            scores[s] = dot * scale;
        }
        oq_softmax_raw(scores, kv_len);
        float *o = out + h * d->hd;
        for (int64_t s = 0; s < kv_len; s++) {
            const float *vr = V + s * stride + kvh * d->hd;
            const float p = scores[s];
            for (int64_t i = 0; i < d->hd; i++) o[i] += p * vr[i];
        }
    }
    free(scores);
}

static void layer_decode(const layer_dims *d, const qtts_layer_host *lw,
                         float *x, oq_kv *kv, int32_t layer, int64_t rope_pos)
{
    const int64_t H = d->hidden, qd = d->n_heads * d->hd, kd = d->n_kv * d->hd;
    float *xn = (float *)malloc(H * sizeof(float));
    float *q = (float *)malloc(qd * sizeof(float));
    float *k = (float *)malloc(kd * sizeof(float));
    float *v = (float *)malloc(kd * sizeof(float));
    float *att = (float *)malloc(qd * sizeof(float));
    float *o = (float *)malloc(H * sizeof(float));
    float *g = (float *)malloc(d->inter * sizeof(float));
    float *u = (float *)malloc(d->inter * sizeof(float));
    float *mo = (float *)malloc(H * sizeof(float));

    oq_rms_norm_f16(x, lw->input_norm, H, xn);
    oq_gemv_q4(xn, &lw->q_proj, q);
    oq_gemv_q4(xn, &lw->k_proj, k);
    oq_gemv_q4(xn, &lw->v_proj, v);
    oq_qk_norm(q, d->n_heads, d->hd, lw->q_norm);
    oq_qk_norm(k, d->n_kv, d->hd, lw->k_norm);
    oq_rope_apply(q, d->n_heads, d->hd, rope_pos, d->cos_t, d->sin_t, d->rope_rows);
    oq_rope_apply(k, d->n_kv, d->hd, rope_pos, d->cos_t, d->sin_t, d->rope_rows);

    /* KV append: K after QK-norm + RoPE, V raw (talker.rs:299-302) */
    const int64_t off = kv->len[layer];
    memcpy(kv->K[layer] + off * kd, k, kd * sizeof(float));
    memcpy(kv->V[layer] + off * kd, v, kd * sizeof(float));
    kv->len[layer] = off + 1;

    decode_attention(d, q, kv->K[layer], kv->V[layer], off + 1, att);
    oq_gemv_q4(att, &lw->o_proj, o);
    for (int64_t j = 0; j < H; j++) x[j] += o[j];

    oq_rms_norm_f16(x, lw->post_attn_norm, H, xn);
    oq_gemv_q4(xn, &lw->gate_proj, g);
    oq_gemv_q4(xn, &lw->up_proj, u);
    for (int64_t j = 0; j < d->inter; j++) g[j] = oq_silu(g[j]) * u[j];
    oq_gemv_q4(g, &lw->down_proj, mo);
    for (int64_t j = 0; j < H; j++) x[j] += mo[j];

    free(xn); free(q); free(k); free(v); free(att); free(o); free(g); free(u); free(mo);
}

/* One layer over `seq` rows at positions pos0.. (talker.rs:389-477,
 * code_predictor.rs:354-432): full-k gemm rows, causal attention. */
static void layer_prefill(const layer_dims *d, const qtts_layer_host *lw,
                          float *x, int64_t seq, oq_kv *kv, int32_t layer,
                          int64_t pos0)
{
    const int64_t H = d->hidden, qd = d->n_heads * d->hd, kd = d->n_kv * d->hd;
    const int64_t I = d->inter;
    float *xn = (float *)calloc((size_t)seq * H, sizeof(float));
    float *q = (float *)malloc((size_t)seq * qd * sizeof(float));
    float *k = (float *)malloc((size_t)seq * kd * sizeof(float));
    float *v = (float *)malloc((size_t)seq * kd * sizeof(float));
    float *att = (float *)calloc((size_t)seq * qd, sizeof(float));
    float *o = (float *)malloc((size_t)seq * H * sizeof(float));
    float *g = (float *)malloc((size_t)seq * I * sizeof(float));
    float *u = (float *)malloc((size_t)seq * I * sizeof(float));

    for (int64_t t = 0; t < seq; t++) oq_rms_norm_f16(x + t * H, lw->input_norm, H, xn + t * H);
    oq_gemm_q4(xn, seq, &lw->q_proj, q);
    oq_gemm_q4(xn, seq, &lw->k_proj, k);
    oq_gemm_q4(xn, seq, &lw->v_proj, v);
    for (int64_t t = 0; t < seq; t++) {
        oq_qk_norm(q + t * qd, d->n_heads, d->hd, lw->q_norm);
        oq_qk_norm(k + t * kd, d->n_kv, d->hd, lw->k_norm);
    }
    for (int64_t t = 0; t < seq; t++) {
        oq_rope_apply(q + t * qd, d->n_heads, d->hd, pos0 + t, d->cos_t, d->sin_t, d->rope_rows);
        oq_rope_apply(k + t * kd, d->n_kv, d->hd, pos0 + t, d->cos_t, d->sin_t, d->rope_rows);
    }
    const int64_t start = kv->len[layer];
    memcpy(kv->K[layer] + start * kd, k, (size_t)seq * kd * sizeof(float));
    memcpy(kv->V[layer] + start * kd, v, (size_t)seq * kd * sizeof(float));
    kv->len[layer] = start + seq;

    const int64_t groups = d->n_heads / d->n_kv;
    const float scale = 1.0f / sqrtf((float)d->hd);
    float *scores = (float *)malloc((size_t)(start + seq) * sizeof(float));
    for (int64_t h = 0; h < d->n_heads; h++) {
        const int64_t kvh = h / groups;
        for (int64_t t1 = 0; t1 < seq; t1++) {
            const int64_t alen = start + t1 + 1;
            const float *qv = q + t1 * qd + h * d->hd;
            for (int64_t s = 0; s < alen; s++) {
                const float *kr = kv->K[layer] + s * kd + kvh * d->hd;
                float dot = 0.0f;
                for (int64_t i = 0; i < d->hd; i++) dot += qv[i] * kr[i];
                scores[s] = dot * scale;
            }
            oq_softmax_raw(scores, alen);
            float *ov = att + t1 * qd + h * d->hd;
            for (int64_t s = 0; s < alen; s++) {
                const float *vr = kv->V[layer] + s * kd + kvh * d->hd;
                for (int64_t i = 0; i < d->hd; i++) ov[i] += scores[s] * vr[i];
            }
        }
    }
    free(scores);
    oq_gemm_q4(att, seq, &lw->o_proj, o);
    for (int64_t j = 0; j < seq * H; j++) x[j] += o[j];
    for (int64_t t = 0; t < seq; t++) oq_rms_norm_f16(x + t * H, lw->post_attn_norm, H, xn + t * H);
    oq_gemm_q4(xn, seq, &lw->gate_proj, g);
    oq_gemm_q4(xn, seq, &lw->up_proj, u);
    for (int64_t j = 0; j < seq * I; j++) g[j] = oq_silu(g[j]) * u[j];
    oq_gemm_q4(g, seq, &lw->down_proj, o);
    for (int64_t j = 0; j < seq * H; j++) x[j] += o[j];

    free(xn); free(q); free(k); free(v); free(att); free(o); free(g); free(u);
}

/* ===================================================================== */
/* talker                                                                 */
/* ===================================================================== */

static layer_dims talker_dims(const qtts_talker_host *t)
{
    layer_dims d;
    d.hidden = t->hidden; d.n_heads = t->n_heads; d.n_kv = t->n_kv_heads;
    d.hd = t->head_dim; d.inter = t->inter;
    d.cos_t = t->rope_cos; d.sin_t = t->rope_sin; d.rope_rows = t->rope_max_pos;
    return d;
}

/* forward_with_embedding (talker.rs:263-360). */
int oq_talker_step(const qtts_talker_host *t, const float *emb, oq_kv *kv,
                   int64_t position, float *out)
{
    const int64_t H = t->hidden;
    if (kv->len[0] + 1 > kv->cap) return QTTS_ERR_CAPACITY;
    layer_dims d = talker_dims(t);
    float *x = (float *)malloc(H * sizeof(float));
    memcpy(x, emb, H * sizeof(float));
    for (int32_t l = 0; l < t->n_layers; l++)
        layer_decode(&d, &t->layers[l], x, kv, l, position);
    oq_rms_norm_f16(x, t->final_norm, H, out);
    oq_gemv_q4(out, &t->codec_head, out + H);
    free(x);
    return QTTS_OK;
}

/* prefill_talker_raw_from (talker.rs:379-482). */
int oq_talker_prefill(const qtts_talker_host *t, const float *X, int64_t seq,
                      oq_kv *kv, int64_t start_pos, float *hidden_out)
{
    const int64_t H = t->hidden;
    if (seq < 1) return QTTS_ERR_INVALID;
    if (kv->len[0] != start_pos) return QTTS_ERR_STATE;   /* talker.rs:422 */
    if (start_pos + seq > kv->cap) return QTTS_ERR_CAPACITY;
    layer_dims d = talker_dims(t);
    float *x = (float *)malloc((size_t)seq * H * sizeof(float));
    memcpy(x, X, (size_t)seq * H * sizeof(float));
    for (int32_t l = 0; l < t->n_layers; l++)
        layer_prefill(&d, &t->layers[l], x, seq, kv, l, start_pos);
    oq_rms_norm_f16(x + (seq - 1) * H, t->final_norm, H, hidden_out);
    free(x);
    return QTTS_OK;
}

/* apply_codec_head (talker.rs:647-649). */
void oq_codec_head(const qtts_talker_host *t, const float *hidden, float *logits)
{
    oq_gemv_q4(hidden, &t->codec_head, logits);
}

/* embed_text_token (talker.rs:105-116). */
void oq_embed_text_token(const qtts_talker_host *t, uint32_t id, float *out)
{
    const int64_t th = t->text_hidden;
    const int64_t n1 = t->text_fc1.n;
    float *raw = (float *)malloc(th * sizeof(float));
    float *h = (float *)malloc(n1 * sizeof(float));
    oq_embed_lookup_q4(&t->text_embedding, id, th, raw);
    oq_gemv_q4(raw, &t->text_fc1, h);
    for (int64_t j = 0; j < n1; j++) h[j] += t->text_fc1_bias[j];
    for (int64_t j = 0; j < n1; j++) h[j] = oq_silu(h[j]);
    oq_gemv_q4(h, &t->text_fc2, out);
    for (int64_t j = 0; j < t->text_fc2.n; j++) out[j] += t->text_fc2_bias[j];
    free(raw); free(h);
}

/* embed_codec_token (talker.rs:152-154). */
void oq_embed_codec_token(const qtts_talker_host *t, uint32_t id, float *out)
{
    oq_embed_lookup_q4(&t->codec_embedding, id, t->hidden, out);
}

/* ===================================================================== */
/* code predictor                                                         */
/* ===================================================================== */

static layer_dims pred_dims(const qtts_predictor_host *p)
{
    layer_dims d;
    d.hidden = p->hidden; d.n_heads = p->n_heads; d.n_kv = p->n_kv_heads;
    d.hd = p->head_dim; d.inter = p->inter;
    d.cos_t = p->rope_cos; d.sin_t = p->rope_sin; d.rope_rows = p->rope_max_pos;
    return d;
}

/* project_input (code_predictor.rs:51-61). */
static void project_input(const qtts_predictor_host *p, const float *in, float *out)
{
    if (p->has_input_proj) {
        oq_gemv_q4(in, &p->input_proj, out);
        if (p->input_proj_bias)
            for (int64_t j = 0; j < p->input_proj.n; j++) out[j] += p->input_proj_bias[j];
    } else {
        memcpy(out, in, (size_t)p->hidden * sizeof(float));
    }
}

/* sample_argmax (code_predictor.rs:335-341): max_by keeps the LAST of equal
 * maxima.  NaN would panic in Rust; returns UINT32_MAX here. */
uint32_t oq_argmax_last(const float *v, int64_t n)
{
    if (n <= 0) return 0;
    int64_t best = 0;
    if (isnan(v[0])) return UINT32_MAX;
    for (int64_t i = 1; i < n; i++) {
        if (isnan(v[i])) return UINT32_MAX;
        if (!(v[best] > v[i])) best = i;
    }
    return (uint32_t)best;
}

/* generate_acoustic_codes (code_predictor.rs:218-273) with prefill
 * (code_predictor.rs:345-438) and decode steps (code_predictor.rs:441-513). */
int oq_predictor_chain(const qtts_predictor_host *p, const float *th,
                       const float *sem, oq_kv *kv, uint32_t *codes_out,
                       const uint32_t *forced)
{
    const int64_t h = p->hidden;
    const int64_t ed = p->codec_embeddings[0].n;
    layer_dims d = pred_dims(p);
    oq_kv_reset(kv);                                   /* :227-231 */
    float *x = (float *)malloc(2 * h * sizeof(float));
    float *hid = (float *)malloc(h * sizeof(float));
    float *logits = (float *)malloc((size_t)p->vocab * sizeof(float));
    float *emb = (float *)malloc(ed * sizeof(float));
    project_input(p, th, x);                           /* :235-236 */
    project_input(p, sem, x + h);
    for (int32_t l = 0; l < p->n_layers; l++)          /* :244, prefill at positions 0,1 */
        layer_prefill(&d, &p->layers[l], x, 2, kv, l, 0);
    oq_rms_norm_f16(x + h, p->final_norm, h, hid);
    oq_gemv_q4(hid, &p->lm_heads[0], logits);          /* :247-248 */
    uint32_t code = oq_argmax_last(logits, p->lm_heads[0].n);
    int rc = QTTS_OK;
    if (code == UINT32_MAX) { rc = QTTS_ERR_NAN; code = 0; }
    codes_out[0] = code;
    int64_t offset = 2;
    for (int32_t g = 1; g < p->n_groups; g++) {        /* :253-270 */
        const uint32_t prev = forced ? forced[g - 1] : codes_out[g - 1];
        oq_embed_lookup_q4(&p->codec_embeddings[g - 1], prev, ed, emb);
        project_input(p, emb, x);
        for (int32_t l = 0; l < p->n_layers; l++)
            layer_decode(&d, &p->layers[l], x, kv, l, kv->len[l]);
        oq_rms_norm_f16(x, p->final_norm, h, hid);
        oq_gemv_q4(hid, &p->lm_heads[g], logits);
        code = oq_argmax_last(logits, p->lm_heads[g].n);
        if (code == UINT32_MAX) { rc = QTTS_ERR_NAN; code = 0; }
        codes_out[g] = code;
        offset++;
    }
    (void)offset;
    free(x); free(hid); free(logits); free(emb);
    return rc;
}

/* predict_codes (code_predictor.rs:126-216), the legacy loop's predictor
 * (generate.rs:210-213): project the talker hidden, run the layers over a
 * cache that persists across calls (the position of the new row is the
 * cache length, RoPE at that offset), final norm, then every lm head:
 * logits [n_groups][vocab]. */
int oq_predict_codes(const qtts_predictor_host *p, const float *th, oq_kv *kv, float *logits)
{
    const int64_t h = p->hidden;
    layer_dims d = pred_dims(p);
    if (kv->len[0] >= kv->cap) return QTTS_ERR_CAPACITY;
    float *x = (float *)malloc(h * sizeof(float));
    float *hid = (float *)malloc(h * sizeof(float));
    project_input(p, th, x);                           /* :135 */
    for (int32_t l = 0; l < p->n_layers; l++)          /* :137-199 */
        layer_decode(&d, &p->layers[l], x, kv, l, kv->len[l]);
    oq_rms_norm_f16(x, p->final_norm, h, hid);         /* :202 */
    for (int32_t g = 0; g < p->n_groups; g++)          /* :205-208 */
        oq_gemv_q4(hid, &p->lm_heads[g], logits + (size_t)g * p->vocab);
    free(x); free(hid);
    return QTTS_OK;
}

/* get_acoustic_embeddings_sum (code_predictor.rs:287-300). */
void oq_acoustic_embed_sum(const qtts_predictor_host *p, const uint32_t *codes,
                           int32_t n, float *out)
{
    const int64_t ed = p->codec_embeddings[0].n;
    float *e = (float *)malloc(ed * sizeof(float));
    memset(out, 0, ed * sizeof(float));
    for (int32_t g = 0; g < n; g++) {
        oq_embed_lookup_q4(&p->codec_embeddings[g], codes[g], ed, e);
        for (int64_t j = 0; j < ed; j++) out[j] += e[j];
    }
    free(e);
}

/* ===================================================================== */
/* sampler (generate_new.rs:771-862)                                      */
/* ===================================================================== */

typedef struct { int64_t i; float p; } ranked;

/* Stable merge sort, descending by p (slice::sort_by with
 * b.partial_cmp(a)): equal values keep index order. */
static void sort_desc_stable(ranked *a, int64_t n, ranked *tmp)
{
    if (n < 2) return;
    const int64_t m = n / 2;
    sort_desc_stable(a, m, tmp);
    sort_desc_stable(a + m, n - m, tmp);
    int64_t i = 0, j = m, o = 0;
    while (i < m && j < n) {
        if (a[j].p > a[i].p) tmp[o++] = a[j++];
        else tmp[o++] = a[i++];
    }
    while (i < m) tmp[o++] = a[i++];
    while (j < n) tmp[o++] = a[j++];
    memcpy(a, tmp, (size_t)n * sizeof(ranked));
}

static int any_nan(const float *s, int64_t n)
{
    for (int64_t i = 0; i < n; i++) if (isnan(s[i])) return 1;
    return 0;
}

int oq_sample_token(const float *logits, int64_t n,
                    const qtts_sample_params *p, const uint32_t *prev,
                    int64_t n_prev, uint64_t *rng, float temperature,
                    uint32_t *out)
{
    float *s = (float *)malloc((size_t)n * sizeof(float));
    memcpy(s, logits, (size_t)n * sizeof(float));
    if (p->repetition_penalty != 1.0f) {                          /* :775-785 */
        for (int64_t i = 0; i < n_prev; i++) {
            const uint32_t t = prev[i];
            if ((int64_t)t < n) {
                if (s[t] > 0.0f) s[t] /= p->repetition_penalty;
                else s[t] *= p->repetition_penalty;
            }
        }
    }
    if (temperature != 1.0f && temperature > 0.0f)                /* :788-792 */
        for (int64_t i = 0; i < n; i++) s[i] /= temperature;
    float mx = -INFINITY;                                          /* :795-802 */
    for (int64_t i = 0; i < n; i++) mx = fmaxf(mx, s[i]);
    for (int64_t i = 0; i < n; i++) s[i] = expf(s[i] - mx);
    float sum = 0.0f;
    for (int64_t i = 0; i < n; i++) sum += s[i];
    for (int64_t i = 0; i < n; i++) s[i] /= sum;

    ranked *r = NULL, *tmp = NULL;
    if ((p->top_k > 0 && p->top_k < n) || (p->top_p > 0.0f && p->top_p < 1.0f)) {
        r = (ranked *)malloc((size_t)n * sizeof(ranked));
        tmp = (ranked *)malloc((size_t)n * sizeof(ranked));
    }
    if (p->top_k > 0 && p->top_k < n) {                            /* :805-820 */
        if (any_nan(s, n)) { free(s); free(r); free(tmp); return QTTS_ERR_NAN; }
        for (int64_t i = 0; i < n; i++) { r[i].i = i; r[i].p = s[i]; }
        sort_desc_stable(r, n, tmp);
        for (int64_t i = p->top_k; i < n; i++) s[r[i].i] = 0.0f;
        float s2 = 0.0f;
        for (int64_t i = 0; i < n; i++) s2 += s[i];
        if (s2 > 0.0f) for (int64_t i = 0; i < n; i++) s[i] /= s2;
    }
    if (p->top_p > 0.0f && p->top_p < 1.0f) {                      /* :824-849 */
        if (any_nan(s, n)) { free(s); free(r); free(tmp); return QTTS_ERR_NAN; }
        for (int64_t i = 0; i < n; i++) { r[i].i = i; r[i].p = s[i]; }
        sort_desc_stable(r, n, tmp);
        float cum = 0.0f;
        int64_t cutoff = n;
        for (int64_t k = 0; k < n; k++) {
            cum += r[k].p;
            if (cum >= p->top_p) { cutoff = k + 1; break; }
        }
        if (cutoff < 1) cutoff = 1;
        for (int64_t i = cutoff; i < n; i++) s[r[i].i] = 0.0f;
        float s2 = 0.0f;
        for (int64_t i = 0; i < n; i++) s2 += s[i];
        if (s2 > 0.0f) for (int64_t i = 0; i < n; i++) s[i] /= s2;
    }
    free(r); free(tmp);
    const float rr = oq_simple_rand(rng);                          /* :852-861 */
    float cs = 0.0f;
    uint32_t res = 0;
    for (int64_t i = 0; i < n; i++) {
        cs += s[i];
        if (rr < cs) { res = (uint32_t)i; break; }
    }
    free(s);
    *out = res;
    return QTTS_OK;
}

/* The legacy loop's sampler (generate.rs:185-217): apply_repetition_penalty
 * (generate.rs:87-98) over every previous token when penalty > 1, then
 * sample_top_k (generate.rs:50-84): temperature <= 0 -> the last maximum
 * (max_by); else the top_k logits in descending order, probabilities
 * exp((l - max) / T) normalised by their sequential sum, and the first
 * index whose running sum passes simple_rand.  The reference orders equal
 * logits with an unstable sort; here ties keep index order.  top_k 0 (a
 * panic in the reference) is QTTS_ERR_INVALID, a NaN QTTS_ERR_NAN. */
int oq_sample_top_k(const float *logits, int64_t n, float temperature, int64_t top_k,
                    const uint32_t *prev, int64_t n_prev, float penalty, uint64_t *rng,
                    uint32_t *out)
{
    if (n < 1) return QTTS_ERR_INVALID;
    float *s = (float *)malloc((size_t)n * sizeof(float));
    memcpy(s, logits, (size_t)n * sizeof(float));
    if (penalty > 1.0f) {
        for (int64_t i = 0; i < n_prev; i++) {
            const uint32_t t = prev[i];
            if ((int64_t)t < n) {
                if (s[t] > 0.0f) s[t] /= penalty;
                else s[t] *= penalty;
            }
        }
    }
    if (any_nan(s, n)) { free(s); return QTTS_ERR_NAN; }
    if (temperature <= 0.0f) {
        *out = oq_argmax_last(s, n);
        free(s);
        return QTTS_OK;
    }
    const int64_t k = top_k < n ? top_k : n;
    if (k < 1) { free(s); return QTTS_ERR_INVALID; }
    ranked *r = (ranked *)malloc((size_t)n * sizeof(ranked));
    ranked *tmp = (ranked *)malloc((size_t)n * sizeof(ranked));
    for (int64_t i = 0; i < n; i++) { r[i].i = i; r[i].p = s[i]; }
    sort_desc_stable(r, n, tmp);
    float *pr = (float *)malloc((size_t)k * sizeof(float));
    const float mx = r[0].p;
    for (int64_t i = 0; i < k; i++) pr[i] = expf((r[i].p - mx) / temperature);
    float sum = 0.0f;
    for (int64_t i = 0; i < k; i++) sum += pr[i];
    for (int64_t i = 0; i < k; i++) pr[i] /= sum;
    const float rr = oq_simple_rand(rng);
    float cs = 0.0f;
    uint32_t res = (uint32_t)r[k - 1].i;
    for (int64_t i = 0; i < k; i++) {
        cs += pr[i];
        if (rr < cs) { res = (uint32_t)r[i].i; break; }
    }
    free(s); free(r); free(tmp); free(pr);
    *out = res;
    return QTTS_OK;
}

/* ===================================================================== */
/* frame loop body (generate_new.rs:606-675)                              */
/* ===================================================================== */

int oq_frame(const qtts_talker_host *t, const qtts_predictor_host *p,
             oq_kv *tkv, oq_kv *pkv, oq_gen *st, const qtts_sample_params *sp,
             const float *text_add, uint32_t *codes_out, int32_t *eos,
             const uint32_t *forced)
{
    const int64_t H = t->hidden;
    const float temp = st->frame_idx < sp->onset_frames ? sp->onset_temperature
                                                        : sp->temperature;  /* :82-88 */
    uint32_t c0;
    int rc = oq_sample_token(st->logits, t->vocab, sp, st->prev, 16, &st->rng,
                             temp, &c0);                                    /* :609 */
    if (rc) return rc;
    *eos = 0;
    codes_out[0] = c0;
    if (sp->eos_enabled && c0 == sp->codec_eos_id && !forced) {             /* :611-614 */
        *eos = 1;
        return QTTS_OK;
    }
    const uint32_t c0_used = forced ? forced[0] : c0;
    st->prev[0] = c0_used;                                                  /* :617 */
    float *sem = (float *)malloc(H * sizeof(float));
    oq_embed_codec_token(t, c0_used, sem);                                  /* :620 */
    uint32_t ac[15];
    rc = oq_predictor_chain(p, st->hidden, sem, pkv, ac, forced ? forced + 1 : NULL);
    if (rc) { free(sem); return rc; }
    const uint32_t *used = forced ? forced + 1 : ac;
    for (int g = 0; g < p->n_groups; g++) {                                 /* :633-636 */
        codes_out[g + 1] = ac[g];
        st->prev[g + 1] = used[g];
    }
    float *sum = (float *)malloc(H * sizeof(float));
    oq_acoustic_embed_sum(p, used, p->n_groups, sum);                      /* :640 */
    for (int64_t j = 0; j < H; j++) sem[j] += sum[j];                       /* :641-643 */
    for (int64_t j = 0; j < H; j++) sem[j] += text_add[j];                  /* :652-654 */
    float *res = (float *)malloc((size_t)(H + t->vocab) * sizeof(float));
    rc = oq_talker_step(t, sem, tkv, st->position, res);                    /* :658 */
    if (rc == QTTS_OK) {
        memcpy(st->hidden, res, H * sizeof(float));                         /* :663-665 */
        memcpy(st->logits, res + H, (size_t)t->vocab * sizeof(float));
        st->position += 1;
        st->frame_idx += 1;
    }
    free(sem); free(sum); free(res);
    return rc;
}

/* ===================================================================== */
/* prompt construction (generate_new.rs:82-476)                           */
/* ===================================================================== */

/* special ids (generate_new.rs:25-36) */
enum {
    OQ_IM_START = 151644, OQ_ASSISTANT = 77091, OQ_NEWLINE = 198,
    OQ_TTS_PAD = 151671, OQ_TTS_BOS = 151672, OQ_TTS_EOS = 151673,
    OQ_CODEC_THINK = 2154, OQ_CODEC_THINK_BOS = 2156, OQ_CODEC_THINK_EOS = 2157,
    OQ_CODEC_PAD = 2148, OQ_CODEC_BOS = 2149
};

/* frame_temperature (generate_new.rs:82-88). */
float oq_frame_temperature(const qtts_sample_params *sp, int64_t frame_idx)
{
    return frame_idx < sp->onset_frames ? sp->onset_temperature : sp->temperature;
}

/* out = a + b, element by element (add_embed, generate_new.rs:130-132). */
static void add_rows(const float *a, const float *b, int64_t n, float *out)
{
    for (int64_t j = 0; j < n; j++) out[j] = a[j] + b[j];
}

/* build_prefill_head (generate_new.rs:222-237): build_role_prefix (:91-97),
 * then build_codec_prefix_voice (:200-223) with a voice embedding or
 * build_codec_prefix_builtin (:226-238, overlay build_tts_pad_bos :100-108)
 * without.  out: [9][hidden]. */
void oq_build_prefill_head(const qtts_talker_host *t, uint32_t speaker_id, uint32_t language_id,
                           const float *voice, int64_t voice_len, float *out)
{
    const int64_t H = t->hidden;
    float *pad = (float *)malloc(H * sizeof(float));
    float *bos = (float *)malloc(H * sizeof(float));
    float *ce = (float *)malloc(H * sizeof(float));
    oq_embed_text_token(t, OQ_IM_START, out);
    oq_embed_text_token(t, OQ_ASSISTANT, out + H);
    oq_embed_text_token(t, OQ_NEWLINE, out + 2 * H);
    oq_embed_text_token(t, OQ_TTS_PAD, pad);
    oq_embed_text_token(t, OQ_TTS_BOS, bos);
    if (voice) {
        const uint32_t codec[4] = {OQ_CODEC_THINK, OQ_CODEC_THINK_BOS, language_id, OQ_CODEC_THINK_EOS};
        for (int i = 0; i < 4; i++) {
            oq_embed_codec_token(t, codec[i], ce);
            add_rows(ce, pad, H, out + (3 + i) * H);
        }
        float *p4 = out + 7 * H;
        memset(p4, 0, H * sizeof(float));
        const int64_t m = voice_len < H ? voice_len : H;
        for (int64_t j = 0; j < m; j++) p4[j] = voice[j] + pad[j];
        oq_embed_codec_token(t, OQ_CODEC_PAD, ce);
        add_rows(ce, bos, H, out + 8 * H);
    } else {
        const uint32_t codec[6] = {OQ_CODEC_THINK, OQ_CODEC_THINK_BOS, language_id, OQ_CODEC_THINK_EOS,
                                   speaker_id, OQ_CODEC_PAD};
        for (int i = 0; i < 6; i++) {
            oq_embed_codec_token(t, codec[i], ce);
            add_rows(ce, i < 5 ? pad : bos, H, out + (3 + i) * H);
        }
    }
    free(pad); free(bos); free(ce);
}

/* icl_block_layout (generate_new.rs:120-128). */
void oq_icl_layout(int64_t n_ref, int64_t n_text, int64_t n_frames, int64_t *icl_len, int64_t *rem_len)
{
    const int64_t text_len = n_ref + n_text + 1, codec_len = n_frames + 1;
    *icl_len = codec_len;
    *rem_len = text_len > codec_len ? text_len - codec_len : 0;
}

/* codec_full row f of the ICL block: CODEC_BOS for f = 0, else the talker
 * codec row of ref_codes[0][f-1] += the predictor rows of codes 1..15
 * (generate_new.rs:159-172).  codes: [16][n_frames]. */
static void codec_full_row(const qtts_talker_host *t, const qtts_predictor_host *p, const uint32_t *codes,
                           int64_t n_frames, int64_t f, float *row, float *tmp)
{
    const int64_t H = t->hidden;
    if (f == 0) {
        oq_embed_codec_token(t, OQ_CODEC_BOS, row);
        return;
    }
    oq_embed_codec_token(t, codes[f - 1], row);
    for (int g = 1; g < 16; g++) {
        oq_embed_lookup_q4(&p->codec_embeddings[g - 1], codes[(size_t)g * n_frames + f - 1], H, tmp);
        for (int64_t j = 0; j < H; j++) row[j] += tmp[j];
    }
}

/* build_icl_block (generate_new.rs:140-195): icl [icl_len][H], remainder
 * [rem_len][H] (NULL when rem_len is 0). */
void oq_build_icl_block(const qtts_talker_host *t, const qtts_predictor_host *p, const uint32_t *ref_tokens,
                        int64_t n_ref, const uint32_t *text_tokens, int64_t n_text, const uint32_t *codes,
                        int64_t n_frames, float *icl, float *rem)
{
    const int64_t H = t->hidden, text_len = n_ref + n_text + 1, codec_len = n_frames + 1;
    float *pad = (float *)malloc(H * sizeof(float));
    float *txt = (float *)malloc(H * sizeof(float));
    float *cod = (float *)malloc(H * sizeof(float));
    float *tmp = (float *)malloc(H * sizeof(float));
    oq_embed_text_token(t, OQ_TTS_PAD, pad);
    for (int64_t i = 0; i < (text_len > codec_len ? text_len : codec_len); i++) {
        /* text_full[i]: ref ++ text ++ [tts_eos] */
        const int have_text = i < text_len;
        if (have_text) {
            const uint32_t tok = i < n_ref ? ref_tokens[i] : i < n_ref + n_text ? text_tokens[i - n_ref] : OQ_TTS_EOS;
            oq_embed_text_token(t, tok, txt);
        }
        if (i < codec_len) {
            codec_full_row(t, p, codes, n_frames, i, cod, tmp);
            add_rows(have_text ? txt : pad, cod, H, icl + i * H);
        } else {
            memcpy(rem + (i - codec_len) * H, txt, H * sizeof(float));
        }
    }
    free(pad); free(txt); free(cod); free(tmp);
}

/* build_icl_prefix (generate_new.rs:244-280): the first n_ref pairs of the
 * ICL block, text row + codec_full row (CODEC_PAD past the frames). */
void oq_build_icl_prefix(const qtts_talker_host *t, const qtts_predictor_host *p, const uint32_t *ref_tokens,
                         int64_t n_ref, const uint32_t *codes, int64_t n_frames, float *out)
{
    const int64_t H = t->hidden;
    float *txt = (float *)malloc(H * sizeof(float));
    float *cod = (float *)malloc(H * sizeof(float));
    float *tmp = (float *)malloc(H * sizeof(float));
    for (int64_t i = 0; i < n_ref; i++) {
        oq_embed_text_token(t, ref_tokens[i], txt);
        if (i == 0 || i - 1 < n_frames)
            codec_full_row(t, p, codes, n_frames, i, cod, tmp);
        else
            oq_embed_codec_token(t, OQ_CODEC_PAD, cod);
        add_rows(txt, cod, H, out + i * H);
    }
    free(txt); free(cod); free(tmp);
}

/* build_trailing_text (generate_new.rs:756-767): text rows of tokens
 * 1..n-1, then TTS_EOS.  out: [max(n - 1, 0) + 1][H]. */
void oq_build_trailing_text(const qtts_talker_host *t, const uint32_t *tokens, int64_t n, float *out)
{
    const int64_t H = t->hidden;
    int64_t r = 0;
    for (int64_t i = 1; i < n; i++) oq_embed_text_token(t, tokens[i], out + (r++) * H);
    oq_embed_text_token(t, OQ_TTS_EOS, out + r * H);
}

/* prefill_custom_voice (generate_new.rs:361-476): the prompt rows, written
 * out step by step as that function writes them (role prefix; with a voice
 * embedding four codec+TTS_PAD rows, voice+TTS_PAD, PAD+TTS_BOS, then the
 * ICL rows or BOS+first text; without, the built-in speaker's six rows
 * under the [TTS_PAD x5, TTS_BOS] overlay, then BOS+first text), prefilled
 * into kv from position 0, then the codec head.  Returns the position the
 * frame loop starts from (generate_new.rs:560-565), or a negative status. */
int64_t oq_prefill_custom_voice(const qtts_talker_host *t, const uint32_t *text_tokens, int64_t n_text,
                                uint32_t speaker_id, uint32_t language_id, const float *voice, int64_t voice_len,
                                const float *icl_rows, int64_t n_icl, oq_kv *kv, float *hidden_out,
                                float *logits_out, float *rows_out)
{
    const int64_t H = t->hidden;
    const int has_first = !icl_rows && n_text > 0;
    const int64_t n = 9 + (icl_rows ? n_icl : has_first);
    float *x = (float *)malloc((size_t)n * H * sizeof(float));
    float *pad = (float *)malloc(H * sizeof(float));
    float *bos = (float *)malloc(H * sizeof(float));
    float *e = (float *)malloc(H * sizeof(float));
    oq_embed_text_token(t, OQ_IM_START, x);
    oq_embed_text_token(t, OQ_ASSISTANT, x + H);
    oq_embed_text_token(t, OQ_NEWLINE, x + 2 * H);
    int64_t r = 3;
    if (voice) {
        const uint32_t prefix_codec[4] = {OQ_CODEC_THINK, OQ_CODEC_THINK_BOS, language_id, OQ_CODEC_THINK_EOS};
        oq_embed_text_token(t, OQ_TTS_PAD, pad);
        oq_embed_text_token(t, OQ_TTS_BOS, bos);
        for (int i = 0; i < 4; i++) {
            oq_embed_codec_token(t, prefix_codec[i], e);
            for (int64_t j = 0; j < H; j++) x[r * H + j] = e[j] + pad[j];
            r++;
        }
        for (int64_t j = 0; j < H; j++) x[r * H + j] = 0.0f;
        for (int64_t j = 0; j < (voice_len < H ? voice_len : H); j++) x[r * H + j] = voice[j] + pad[j];
        r++;
        oq_embed_codec_token(t, OQ_CODEC_PAD, e);
        for (int64_t j = 0; j < H; j++) x[r * H + j] = e[j] + bos[j];
        r++;
        if (icl_rows) {
            memcpy(x + r * H, icl_rows, (size_t)n_icl * H * sizeof(float));
            r += n_icl;
        }
    } else {
        const uint32_t codec[6] = {OQ_CODEC_THINK, OQ_CODEC_THINK_BOS, language_id, OQ_CODEC_THINK_EOS,
                                   speaker_id, OQ_CODEC_PAD};
        oq_embed_text_token(t, OQ_TTS_PAD, pad);
        oq_embed_text_token(t, OQ_TTS_BOS, bos);
        for (int i = 0; i < 6; i++) {
            oq_embed_codec_token(t, codec[i], x + r * H);
            const float *ov = i < 5 ? pad : bos;
            for (int64_t j = 0; j < H; j++) x[r * H + j] += ov[j];
            r++;
        }
    }
    if (has_first) {
        float *first = (float *)malloc(H * sizeof(float));
        oq_embed_codec_token(t, OQ_CODEC_BOS, e);
        oq_embed_text_token(t, text_tokens[0], first);
        for (int64_t j = 0; j < H; j++) x[r * H + j] = e[j] + first[j];
        r++;
        free(first);
    }
    int rc = QTTS_OK;
    if (r != n) rc = QTTS_ERR_INVALID;   /* ICL rows without a voice embedding: not a reference layout */
    if (rc == QTTS_OK) {
        oq_kv_reset(kv);
        rc = oq_talker_prefill(t, x, n, kv, 0, hidden_out);
    }
    if (rc == QTTS_OK) oq_codec_head(t, hidden_out, logits_out);
    if (rc == QTTS_OK && rows_out) memcpy(rows_out, x, (size_t)n * H * sizeof(float));
    free(x); free(pad); free(bos); free(e);
    if (rc != QTTS_OK) return rc;
    return icl_rows ? 9 + n_icl : (n_text > 0 ? 10 : 9);
}
