/*
 * cpu_ref.c — CPU restatement of the codon-infer ESM-2 bidirectional forward
 * (FP32 / Q8_0 / Q4_0), and of its autoregressive one-token forward with a
 * KV cache, sampler and generation loop.  TEST INFRASTRUCTURE: the oracle for the HIP path and
 * the timed CPU baseline.  The product never links or calls this file.
 *
 * Numerics follow the reference routine by routine (file:line cited at each
 * function).  Build with -ffp-contract=off and without -ffast-math: Rust never
 * contracts a*b+c, and glibc's expf/sqrtf/powf/cosf/sinf are the same calls
 * Rust's f32 methods make on Linux, so the scalar parts reproduce the
 * reference's arithmetic operation for operation.  The GEMM micro-kernel is
 * the AVX2+FMA path of dot_row_batch_m4; the attention dot/axpy are the
 * 256-bit AVX paths, or at head_dim 64 on a host with AVX-512F the 512-bit
 * ones, as the reference dispatches at run time.
 */
#define _GNU_SOURCE
#include "cpu_ref.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Q8_0 / Q4_0 blocks                                                        */
/* ------------------------------------------------------------------------ */

static inline float rd_f32(const uint8_t *p) { float f; memcpy(&f, p, 4); return f; }
static inline void wr_f32(uint8_t *p, float f) { memcpy(p, &f, 4); }

/* Rust `f as i32` saturates and maps NaN to 0. */
static inline int64_t sat_i32(float f) {
    if (f != f) return 0;
    if (f >= 2147483647.0f) return 2147483647LL;
    if (f <= -2147483648.0f) return -2147483648LL;
    return (int64_t)f;
}

/* BlockQ8_0::quantize, lib.rs:648-660.  d = absmax/127, id = 1/d (0 if d==0),
 * q = clamp(round_half_away(x*id), -127, 127). */
static void q8_block(const float *src, uint8_t *blk) {
    float max_val = 0.0f;
    for (int i = 0; i < 32; i++) {
        float a = fabsf(src[i]);
        if (a > max_val) max_val = a;
    }
    float d = max_val / 127.0f;
    float id = (d == 0.0f) ? 0.0f : 1.0f / d;
    wr_f32(blk, d);
    for (int i = 0; i < 32; i++) {
        float r = roundf(src[i] * id);
        int8_t q;
        if (r != r) q = 0; /* (NaN).clamp() as i8 == 0 */
        else {
            if (r < -127.0f) r = -127.0f;
            if (r > 127.0f) r = 127.0f;
            q = (int8_t)r;
        }
        blk[4 + i] = (uint8_t)q;
    }
}

/* quantize_slice_to_q8, lib.rs:670-673 */
void cr_quantize_q8(const float *src, int64_t n, uint8_t *dst) {
    for (int64_t b = 0; b < n / 32; b++) q8_block(src + b * 32, dst + b * CR_Q8_BLOCK_BYTES);
}

/* BlockQ8_0::dequantize_to, lib.rs:663-667: q as f32 * d */
void cr_dequantize_q8(const uint8_t *blocks, int64_t nblocks, float *dst) {
    for (int64_t b = 0; b < nblocks; b++) {
        const uint8_t *blk = blocks + b * CR_Q8_BLOCK_BYTES;
        float d = rd_f32(blk);
        for (int i = 0; i < 32; i++) dst[b * 32 + i] = (float)(int8_t)blk[4 + i] * d;
    }
}

/* BlockQ4_0::quantize, lib.rs:1054-1071.  max = the first element of largest
 * |x| (signed); d = max / -8; q = clamp(round(x*id) + 8, 0, 15); byte j holds
 * element j in the low nibble and element j+16 in the high nibble. */
static void q4_block(const float *src, uint8_t *blk) {
    float max = 0.0f;
    for (int i = 0; i < 32; i++)
        if (fabsf(src[i]) > fabsf(max)) max = src[i];
    float d = (max == 0.0f) ? 0.0f : max / -8.0f;
    float id = (d == 0.0f) ? 0.0f : 1.0f / d;
    wr_f32(blk, d);
    for (int j = 0; j < 16; j++) {
        int64_t lo = sat_i32(roundf(src[j] * id)) + 8;
        int64_t hi = sat_i32(roundf(src[j + 16] * id)) + 8;
        lo = lo < 0 ? 0 : (lo > 15 ? 15 : lo);
        hi = hi < 0 ? 0 : (hi > 15 ? 15 : hi);
        blk[4 + j] = (uint8_t)((lo & 0x0F) | ((hi & 0x0F) << 4));
    }
}

/* quantize_slice_to_q4, lib.rs:1085-1088 */
void cr_quantize_q4(const float *src, int64_t n, uint8_t *dst) {
    for (int64_t b = 0; b < n / 32; b++) q4_block(src + b * 32, dst + b * CR_Q4_BLOCK_BYTES);
}

/* BlockQ4_0::dequantize_to, lib.rs:1074-1082: ((nibble) - 8) as f32 * d */
void cr_dequantize_q4(const uint8_t *blocks, int64_t nblocks, float *dst) {
    for (int64_t b = 0; b < nblocks; b++) {
        const uint8_t *blk = blocks + b * CR_Q4_BLOCK_BYTES;
        float d = rd_f32(blk);
        for (int j = 0; j < 16; j++) {
            dst[b * 32 + j] = (float)((int)(blk[4 + j] & 0x0F) - 8) * d;
            dst[b * 32 + j + 16] = (float)((int)((blk[4 + j] >> 4) & 0x0F) - 8) * d;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Tokenizer::encode, lib.rs:6511-6521                                        */
/* ------------------------------------------------------------------------ */

static int32_t aa_id(unsigned c) {
    switch (c) {
    case 'L': return 4;  case 'A': return 5;  case 'G': return 6;  case 'V': return 7;
    case 'S': return 8;  case 'E': return 9;  case 'R': return 10; case 'T': return 11;
    case 'I': return 12; case 'D': return 13; case 'P': return 14; case 'K': return 15;
    case 'Q': return 16; case 'N': return 17; case 'F': return 18; case 'Y': return 19;
    case 'M': return 20; case 'H': return 21; case 'W': return 22; case 'C': return 23;
    case 'X': return 24; case 'B': return 25; case 'U': return 26; case 'Z': return 27;
    case 'O': return 28; case '.': return 29; case '-': return 30; case '*': return 32;
    default: return 3;
    }
}

/* `<mask_1>` and `<mask>` become `*` (id 32) first; every other character,
 * counted as one Unicode scalar, maps through the table (unknown -> 3). */
int32_t cr_tokenize(const char *text, int32_t *out, int32_t cap) {
    int32_t n = 0;
    const unsigned char *s = (const unsigned char *)text;
    if (cap < 1) return -1;
    out[n++] = 0;
    while (*s) {
        int32_t id;
        if (strncmp((const char *)s, "<mask_1>", 8) == 0) { id = 32; s += 8; }
        else if (strncmp((const char *)s, "<mask>", 6) == 0) { id = 32; s += 6; }
        else {
            unsigned c = *s;
            int len = 1;
            if (c >= 0xF0) len = 4; else if (c >= 0xE0) len = 3; else if (c >= 0xC0) len = 2;
            id = (len == 1) ? aa_id(c) : 3;
            for (int i = 0; i < len && *s; i++) s++;
        }
        if (n >= cap) return -1;
        out[n++] = id;
    }
    if (n >= cap) return -1;
    out[n++] = 2;
    return n;
}

/* ------------------------------------------------------------------------ */
/* Elementwise math                                                          */
/* ------------------------------------------------------------------------ */

/* layer_norm, lib.rs:2556-2562 (eps 1e-5, sequential sums) */
void cr_layer_norm(float *out, const float *x, const float *w, const float *b, int32_t dim) {
    float sum = 0.0f;
    for (int i = 0; i < dim; i++) sum += x[i];
    float mean = sum / (float)dim;
    float var = 0.0f;
    for (int i = 0; i < dim; i++) { float c = x[i] - mean; var += c * c; }
    var = var / (float)dim;
    float inv = 1.0f / sqrtf(var + 1e-5f);
    for (int i = 0; i < dim; i++) out[i] = w[i] * (x[i] - mean) * inv + b[i];
}

/* erf_f32, lib.rs:3485-3491: Abramowitz & Stegun 7.1.26 */
float cr_erf(float x) {
    float sign = (x < 0.0f) ? -1.0f : 1.0f;
    float ax = fabsf(x);
    float t = 1.0f / (1.0f + 0.3275911f * ax);
    float y = 1.0f - (((((1.061405429f * t - 1.453152027f) * t) + 1.421413741f) * t - 0.284496736f) * t
                      + 0.254829592f) * t * expf(-ax * ax);
    return sign * y;
}

/* gelu, lib.rs:3493-3498 */
void cr_gelu(float *out, const float *x, int64_t n) {
    const float inv_sqrt2 = 0.70710678118654752440f;
    for (int64_t i = 0; i < n; i++) out[i] = 0.5f * x[i] * (1.0f + cr_erf(x[i] * inv_sqrt2));
}

/* softmax, lib.rs:3500-3504 */
void cr_softmax(float *x, int32_t n) {
    float m = -INFINITY;
    for (int i = 0; i < n; i++) m = fmaxf(m, x[i]);
    float sum = 0.0f;
    for (int i = 0; i < n; i++) { x[i] = expf(x[i] - m); sum += x[i]; }
    float inv = 1.0f / sum;
    for (int i = 0; i < n; i++) x[i] *= inv;
}

/* BidirectionalRunState::new RoPE tables, lib.rs:2513-2522 */
void cr_rope_tables(int32_t max_len, int32_t head_dim, float *cos_t, float *sin_t) {
    int half = head_dim / 2;
    for (int pos = 0; pos < max_len; pos++)
        for (int j = 0; j < half; j++) {
            float freq = 1.0f / powf(10000.0f, (float)(j * 2) / (float)head_dim);
            float val = (float)pos * freq;
            cos_t[pos * half + j] = cosf(val);
            sin_t[pos * half + j] = sinf(val);
        }
}

/* apply_rope, lib.rs:3533-3552: split-half pairs (j, j+hd/2) */
void cr_apply_rope(float *q, float *k, const float *cos_t, const float *sin_t,
                   int32_t pos, int32_t dim, int32_t n_heads) {
    int hd = dim / n_heads, half = hd / 2;
    const float *c = cos_t + (int64_t)pos * half, *s = sin_t + (int64_t)pos * half;
    for (int h = 0; h < n_heads; h++)
        for (int j = 0; j < half; j++) {
            int i0 = h * hd + j, i1 = i0 + half;
            float q0 = q[i0], q1 = q[i1], k0 = k[i0], k1 = k[i1];
            q[i0] = q0 * c[j] - q1 * s[j];
            q[i1] = q1 * c[j] + q0 * s[j];
            k[i0] = k0 * c[j] - k1 * s[j];
            k[i1] = k1 * c[j] + k0 * s[j];
        }
}

/* log_softmax_canonical, lib.rs:4426-4441: over ids 4..=23 only */
void cr_log_softmax_canonical(const float *logits, float *out) {
    for (int i = 0; i < 33; i++) out[i] = -INFINITY;
    float m = -INFINITY;
    for (int i = 4; i <= 23; i++) if (logits[i] > m) m = logits[i];
    float s = 0.0f;
    for (int i = 4; i <= 23; i++) s += expf(logits[i] - m);
    float lse = m + logf(s);
    for (int i = 4; i <= 23; i++) out[i] = logits[i] - lse;
}

/* One DMS row from the logits at the scored position, pipeline.rs:152-172
 * (masked marginal; the wild-type marginal rows, 201-220, are the same
 * arithmetic): canonical log-softmax, Shannon entropy over ids 4..=23 in
 * ascending id order with p = exp(lp) counted when p > 1e-12, and
 * deltas[c] = lp[aa_c] - lp[wt] in CANONICAL_AAS order (benchmark.rs:702-707),
 * exactly 0 for the wild-type column. */
static const int32_t CR_CANONICAL_TOK[20] = {5, 23, 13, 9, 18, 6, 21, 12, 15, 4, 20, 17, 14, 16, 10, 8, 11, 7, 22, 19};

void cr_dms_score(const float *logits, int32_t wt_tok, float *deltas20, float *entropy) {
    float lp[33];
    cr_log_softmax_canonical(logits, lp);
    float h = 0.0f;
    for (int i = 4; i <= 23; i++) {
        float p = expf(lp[i]);
        if (p > 1e-12f) h -= p * lp[i];
    }
    *entropy = h;
    for (int c = 0; c < 20; c++)
        deltas20[c] = CR_CANONICAL_TOK[c] == wt_tok ? 0.0f : lp[CR_CANONICAL_TOK[c]] - lp[wt_tok];
}

/* accumulate_head_apc, lib.rs:5036-5076 */
void cr_accumulate_head_apc(const float *A, float *cl, int32_t S, int32_t n, float w) {
    if (n == 0 || w == 0.0f) return;
    float *rs = (float *)malloc(sizeof(float) * (size_t)n);
    float total = 0.0f;
    for (int i = 0; i < n; i++) {
        float r = 0.0f;
        for (int j = 0; j < n; j++)
            r += A[(int64_t)(i + 1) * S + (j + 1)] + A[(int64_t)(j + 1) * S + (i + 1)];
        rs[i] = r;
        total += r;
    }
    float inv_total = (fabsf(total) > 1e-12f) ? 1.0f / total : 0.0f;
    for (int i = 0; i < n; i++) {
        float ri = rs[i] * inv_total;
        for (int j = 0; j < n; j++) {
            float s = A[(int64_t)(i + 1) * S + (j + 1)] + A[(int64_t)(j + 1) * S + (i + 1)];
            float apc = s - ri * rs[j];
            cl[(int64_t)i * n + j] += w * apc;
        }
    }
    free(rs);
}

/* ------------------------------------------------------------------------ */
/* Persistent fork/join pool (ThreadPool::run_parallel, lib.rs:2676-2783):    */
/* the caller runs slice 0, workers run slices 1..n-1.                       */
/* ------------------------------------------------------------------------ */

typedef void (*cr_job_fn)(const void *ctx, int t, int n);

#define CR_MAX_WORKERS 256
static struct {
    pthread_mutex_t mu;
    pthread_cond_t job_cv, done_cv;
    pthread_mutex_t run_lock;
    int started, n_workers;
    unsigned long generation;
    cr_job_fn fn;
    const void *ctx;
    int n_threads, done;
} g_pool = {PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER, PTHREAD_COND_INITIALIZER,
            PTHREAD_MUTEX_INITIALIZER, 0, 0, 0, 0, 0, 0, 0};

static void *pool_worker(void *arg) {
    int idx = (int)(intptr_t)arg; /* slice index = idx + 1 */
    unsigned long seen = 0;
    for (;;) {
        pthread_mutex_lock(&g_pool.mu);
        while (g_pool.generation == seen) pthread_cond_wait(&g_pool.job_cv, &g_pool.mu);
        seen = g_pool.generation;
        cr_job_fn fn = g_pool.fn;
        const void *ctx = g_pool.ctx;
        int n = g_pool.n_threads;
        pthread_mutex_unlock(&g_pool.mu);
        if (idx + 1 < n) fn(ctx, idx + 1, n);
        pthread_mutex_lock(&g_pool.mu);
        if (idx + 1 < n) {
            g_pool.done++;
            pthread_cond_signal(&g_pool.done_cv);
        }
        pthread_mutex_unlock(&g_pool.mu);
    }
    return NULL;
}

static void run_parallel(int n, cr_job_fn fn, const void *ctx) {
    if (n <= 1) { fn(ctx, 0, 1); return; }
    if (n > CR_MAX_WORKERS) n = CR_MAX_WORKERS;
    pthread_mutex_lock(&g_pool.run_lock);
    pthread_mutex_lock(&g_pool.mu);
    while (g_pool.n_workers < n - 1) {
        pthread_t th;
        pthread_attr_t at;
        pthread_attr_init(&at);
        pthread_attr_setdetachstate(&at, PTHREAD_CREATE_DETACHED);
        pthread_create(&th, &at, pool_worker, (void *)(intptr_t)g_pool.n_workers);
        pthread_attr_destroy(&at);
        g_pool.n_workers++;
    }
    g_pool.fn = fn;
    g_pool.ctx = ctx;
    g_pool.n_threads = n;
    g_pool.done = 0;
    g_pool.generation++;
    pthread_cond_broadcast(&g_pool.job_cv);
    pthread_mutex_unlock(&g_pool.mu);
    fn(ctx, 0, n);
    pthread_mutex_lock(&g_pool.mu);
    while (g_pool.done < n - 1) pthread_cond_wait(&g_pool.done_cv, &g_pool.mu);
    pthread_mutex_unlock(&g_pool.mu);
    pthread_mutex_unlock(&g_pool.run_lock);
}

/* ------------------------------------------------------------------------ */
/* Tiled GEMM (matmul_tiled_{fp32,q8,q4}_parallel, lib.rs:4766-4961)          */
/* ------------------------------------------------------------------------ */

/* hsum256_ps_avx, lib.rs:2566-2573 */
static inline float hsum256(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v), hi = _mm256_extractf128_ps(v, 1);
    __m128 s = _mm_add_ps(lo, hi);
    __m128 h64 = _mm_movehl_ps(s, s);
    __m128 s64 = _mm_add_ps(s, h64);
    __m128 h32 = _mm_shuffle_ps(s64, s64, 0x55);
    return _mm_cvtss_f32(_mm_add_ss(s64, h32));
}

/* dot_row_batch_m4_avx2_fma, lib.rs:4443-4531: one weight row against the
 * token batch, 4 tokens at a time, two 8-wide FMA accumulators per token over
 * k-chunks of 16, then hsum(acc_a + acc_b), scalar tail, + bias. */
__attribute__((target("avx2,fma")))
static void dot_row_batch_m4(float *out, int out_stride, int out_col, const float *x,
                             const float *w_row, float bias, int in_dim, int seq_len) {
    int chunks16 = in_dim / 16, rem = chunks16 * 16;
    int p = 0;
    for (; p + 4 <= seq_len; p += 4) {
        const float *x0 = x + (int64_t)p * in_dim, *x1 = x0 + in_dim, *x2 = x1 + in_dim, *x3 = x2 + in_dim;
        __m256 a0 = _mm256_setzero_ps(), b0 = _mm256_setzero_ps();
        __m256 a1 = _mm256_setzero_ps(), b1 = _mm256_setzero_ps();
        __m256 a2 = _mm256_setzero_ps(), b2 = _mm256_setzero_ps();
        __m256 a3 = _mm256_setzero_ps(), b3 = _mm256_setzero_ps();
        for (int c = 0; c < chunks16; c++) {
            int k = c * 16;
            __m256 w0 = _mm256_loadu_ps(w_row + k), w1 = _mm256_loadu_ps(w_row + k + 8);
            a0 = _mm256_fmadd_ps(w0, _mm256_loadu_ps(x0 + k), a0);
            b0 = _mm256_fmadd_ps(w1, _mm256_loadu_ps(x0 + k + 8), b0);
            a1 = _mm256_fmadd_ps(w0, _mm256_loadu_ps(x1 + k), a1);
            b1 = _mm256_fmadd_ps(w1, _mm256_loadu_ps(x1 + k + 8), b1);
            a2 = _mm256_fmadd_ps(w0, _mm256_loadu_ps(x2 + k), a2);
            b2 = _mm256_fmadd_ps(w1, _mm256_loadu_ps(x2 + k + 8), b2);
            a3 = _mm256_fmadd_ps(w0, _mm256_loadu_ps(x3 + k), a3);
            b3 = _mm256_fmadd_ps(w1, _mm256_loadu_ps(x3 + k + 8), b3);
        }
        float v0 = hsum256(_mm256_add_ps(a0, b0)), v1 = hsum256(_mm256_add_ps(a1, b1));
        float v2 = hsum256(_mm256_add_ps(a2, b2)), v3 = hsum256(_mm256_add_ps(a3, b3));
        for (int k = rem; k < in_dim; k++) {
            float wk = w_row[k];
            v0 += wk * x0[k]; v1 += wk * x1[k]; v2 += wk * x2[k]; v3 += wk * x3[k];
        }
        out[(int64_t)p * out_stride + out_col] = v0 + bias;
        out[(int64_t)(p + 1) * out_stride + out_col] = v1 + bias;
        out[(int64_t)(p + 2) * out_stride + out_col] = v2 + bias;
        out[(int64_t)(p + 3) * out_stride + out_col] = v3 + bias;
    }
    for (; p < seq_len; p++) {
        const float *xp = x + (int64_t)p * in_dim;
        __m256 a = _mm256_setzero_ps(), b = _mm256_setzero_ps();
        for (int c = 0; c < chunks16; c++) {
            int k = c * 16;
            a = _mm256_fmadd_ps(_mm256_loadu_ps(w_row + k), _mm256_loadu_ps(xp + k), a);
            b = _mm256_fmadd_ps(_mm256_loadu_ps(w_row + k + 8), _mm256_loadu_ps(xp + k + 8), b);
        }
        float v = hsum256(_mm256_add_ps(a, b));
        for (int k = rem; k < in_dim; k++) v += w_row[k] * xp[k];
        out[(int64_t)p * out_stride + out_col] = v + bias;
    }
}

typedef struct {
    int32_t wdtype;
    float *out;
    const float *x;
    const void *w;
    const float *bias;
    int in_dim, out_dim, seq_len;
} gemm_job;

/* run_tiled_{fp32,q8,q4}_slice, lib.rs:4776-4801, 4839-4868, 4906-4935:
 * thread t owns output rows [t*chunk, (t+1)*chunk); quantized rows are
 * unpacked once to FP32 (q*d) before the micro-kernel. */
static void gemm_slice(const void *ctx, int t, int n) {
    const gemm_job *j = (const gemm_job *)ctx;
    int chunk = (j->out_dim + n - 1) / n;
    int start = t * chunk;
    if (start >= j->out_dim) return;
    int end = start + chunk < j->out_dim ? start + chunk : j->out_dim;
    int bpr = j->in_dim / 32;
    float *wbuf = NULL;
    if (j->wdtype != CR_FP32) wbuf = (float *)aligned_alloc(64, sizeof(float) * (size_t)((j->in_dim + 15) & ~15));
    for (int i = start; i < end; i++) {
        const float *wrow;
        if (j->wdtype == CR_FP32) {
            wrow = (const float *)j->w + (int64_t)i * j->in_dim;
        } else if (j->wdtype == CR_Q8_0) {
            cr_dequantize_q8((const uint8_t *)j->w + (int64_t)i * bpr * CR_Q8_BLOCK_BYTES, bpr, wbuf);
            wrow = wbuf;
        } else {
            cr_dequantize_q4((const uint8_t *)j->w + (int64_t)i * bpr * CR_Q4_BLOCK_BYTES, bpr, wbuf);
            wrow = wbuf;
        }
        dot_row_batch_m4(j->out, j->out_dim, i, j->x, wrow, j->bias[i], j->in_dim, j->seq_len);
    }
    free(wbuf);
}

void cr_matmul_tiled(int32_t wdtype, float *out, const float *x, const void *w, const float *bias,
                     int32_t in_dim, int32_t out_dim, int32_t seq_len, int32_t num_threads) {
    gemm_job j = {wdtype, out, x, w, bias, in_dim, out_dim, seq_len};
    if (num_threads <= 1 || out_dim < 16) gemm_slice(&j, 0, 1);
    else run_parallel(num_threads, gemm_slice, &j);
}

/* ------------------------------------------------------------------------ */
/* Attention micro-kernels: dot_product_head_avx / accumulate_value_head_avx  */
/* (lib.rs:3292-3394).  Products are not fused; reduction tree as written.   */
/* ------------------------------------------------------------------------ */

__attribute__((target("avx")))
static float dot_head(const float *q, const float *k, int hd) {
#define P8(i) _mm256_mul_ps(_mm256_loadu_ps(q + 8 * (i)), _mm256_loadu_ps(k + 8 * (i)))
    switch (hd) {
    case 16: return hsum256(_mm256_add_ps(P8(0), P8(1)));
    case 24: return hsum256(_mm256_add_ps(_mm256_add_ps(P8(0), P8(1)), P8(2)));
    case 32: return hsum256(_mm256_add_ps(_mm256_add_ps(P8(0), P8(1)), _mm256_add_ps(P8(2), P8(3))));
    case 64: {
        __m256 s01 = _mm256_add_ps(P8(0), P8(1)), s23 = _mm256_add_ps(P8(2), P8(3));
        __m256 s45 = _mm256_add_ps(P8(4), P8(5)), s67 = _mm256_add_ps(P8(6), P8(7));
        return hsum256(_mm256_add_ps(_mm256_add_ps(s01, s23), _mm256_add_ps(s45, s67)));
    }
    default: {
        float s = 0.0f;
        for (int i = 0; i < hd; i++) s += q[i] * k[i];
        return s;
    }
    }
#undef P8
}

static void axpy_head(float *out, const float *v, float p, int hd) {
    for (int i = 0; i < hd; i++) out[i] += p * v[i];
}

/* dot_product_head_avx512_d64 / accumulate_value_head_avx512_d64
 * (lib.rs:3398-3434): what the reference runs at head_dim 64 when the host
 * has AVX-512F (lib.rs:5113, 5457, 5816, 3452).  Dot: 16-wide products of
 * q[0..16) * k[0..16), then three fused multiply-adds of the next 16-wide
 * slices into the same accumulator, then _mm512_reduce_add_ps, whose order is
 * the halving tree (lanes i + i+8, then i + i+4, i + i+2, then 0 + 1).  Axpy:
 * one fused multiply-add per element, out = fma(p, v, out). */
__attribute__((target("avx512f")))
static float dot_head_d64_avx512(const float *q, const float *k) {
    __m512 acc = _mm512_mul_ps(_mm512_loadu_ps(q), _mm512_loadu_ps(k));
    acc = _mm512_fmadd_ps(_mm512_loadu_ps(q + 16), _mm512_loadu_ps(k + 16), acc);
    acc = _mm512_fmadd_ps(_mm512_loadu_ps(q + 32), _mm512_loadu_ps(k + 32), acc);
    acc = _mm512_fmadd_ps(_mm512_loadu_ps(q + 48), _mm512_loadu_ps(k + 48), acc);
    float a[16], b[8], c[4], e[2];
    _mm512_storeu_ps(a, acc);
    for (int i = 0; i < 8; i++) b[i] = a[i] + a[i + 8];
    for (int i = 0; i < 4; i++) c[i] = b[i] + b[i + 4];
    for (int i = 0; i < 2; i++) e[i] = c[i] + c[i + 2];
    return e[0] + e[1];
}

__attribute__((target("avx512f")))
static void axpy_head_d64_avx512(float *out, const float *v, float p) {
    const __m512 pv = _mm512_set1_ps(p);
    for (int i = 0; i < 64; i += 16)
        _mm512_storeu_ps(out + i, _mm512_fmadd_ps(pv, _mm512_loadu_ps(v + i), _mm512_loadu_ps(out + i)));
}

/* is_x86_feature_detected!("avx512f") at head_dim 64, as the reference
 * decides per forward; cr_set_attention_isa(1) forces the 256-bit path. */
static int g_force_avx = 0;
void cr_set_attention_isa(int32_t avx_only) { g_force_avx = avx_only != 0; }
int32_t cr_attention_uses_avx512(int32_t hd) {
    return hd == 64 && !g_force_avx && __builtin_cpu_supports("avx512f");
}

static inline float dot_head_dispatch(int avx512, const float *q, const float *k, int hd) {
    return avx512 ? dot_head_d64_avx512(q, k) : dot_head(q, k, hd);
}
static inline void axpy_head_dispatch(int avx512, float *out, const float *v, float p, int hd) {
    if (avx512) axpy_head_d64_avx512(out, v, p);
    else axpy_head(out, v, p, hd);
}

/* ------------------------------------------------------------------------ */
/* The bidirectional forward: forward_bidirectional_parallel_ext (FP32,       */
/* lib.rs:5097-5440), forward_bidirectional_q8 (5442-5788),                  */
/* forward_bidirectional_q4_ext (5800-6147).                                 */
/* ------------------------------------------------------------------------ */

static int64_t wblock_bytes(int32_t dtype) {
    return dtype == CR_Q8_0 ? CR_Q8_BLOCK_BYTES : (dtype == CR_Q4_0 ? CR_Q4_BLOCK_BYTES : 0);
}

/* byte offset of matrix l within a tensor-major stack of [out][in] matrices */
static const void *mat_at(const void *base, int32_t dtype, int64_t l, int64_t out_dim, int64_t in_dim) {
    int64_t elems = l * out_dim * in_dim;
    if (dtype == CR_FP32) return (const float *)base + elems;
    return (const uint8_t *)base + (elems / 32) * wblock_bytes(dtype);
}

int32_t cr_forward(const cr_config *cfg, const cr_weights *w, const int32_t *tokens,
                   int32_t S, int32_t nt, const cr_outputs *o) {
    const int d = cfg->dim, F = cfg->hidden_dim, L = cfg->n_layers, H = cfg->n_heads, V = cfg->vocab_size;
    if (S < 1 || d <= 0 || H <= 0 || d % H != 0 || d % 32 != 0 || F % 32 != 0) return -1;
    const int hd = d / H;
    const int32_t dt = w->dtype;
    for (int p = 0; p < S; p++)
        if (tokens[p] < 0 || tokens[p] >= V) return -2;
    const int n_res = S >= 2 ? S - 2 : 0;
    const int do_contacts = (o->contacts != NULL) && n_res > 0;
    if (do_contacts && n_res > 1024) return -4; /* row_sums: [f32; 1024], lib.rs:5046 */
    if (do_contacts && !o->contact_w) return -1;
    const float inv_scale = 1.0f / sqrtf((float)hd);
    const int avx512 = cr_attention_uses_avx512(hd);

    float *x = calloc((size_t)S * d, 4), *xb = calloc((size_t)S * d, 4);
    float *q = calloc((size_t)S * d, 4), *k = calloc((size_t)S * d, 4), *v = calloc((size_t)S * d, 4);
    float *oa = calloc((size_t)S * d, 4);
    int hbw = F > d ? F : d;
    float *hb = calloc((size_t)S * hbw, 4), *hb2 = calloc((size_t)S * hbw, 4);
    float *att = calloc((size_t)S, 4);
    float *head_att = do_contacts ? calloc((size_t)S * S, 4) : NULL;
    float *final_att = calloc((size_t)S * S, 4);
    float *rc = calloc((size_t)S * (hd / 2 > 0 ? hd / 2 : 1), 4), *rsn = calloc((size_t)S * (hd / 2 > 0 ? hd / 2 : 1), 4);
    float *cl = do_contacts ? calloc((size_t)n_res * n_res, 4) : NULL;
    cr_rope_tables(S, hd, rc, rsn);

    /* embedding + token-dropout rescale (lib.rs:5117-5131, 5461-5479, 5820-5833) */
    int mask_count = 0;
    for (int p = 0; p < S; p++) mask_count += tokens[p] == 32;
    float ratio = (float)mask_count / (float)S;
    float scale = (ratio >= 1.0f) ? 0.0f : (1.0f - 0.12f) / (1.0f - ratio);
    for (int p = 0; p < S; p++) {
        int t = tokens[p];
        float *xp = x + (int64_t)p * d;
        if (t == 32) { memset(xp, 0, sizeof(float) * d); continue; }
        if (dt == CR_Q8_0) {
            cr_dequantize_q8((const uint8_t *)w->token_embedding_table + (int64_t)t * (d / 32) * CR_Q8_BLOCK_BYTES, d / 32, xp);
            for (int i = 0; i < d; i++) xp[i] *= scale;
        } else {
            const float *e = (const float *)w->token_embedding_table + (int64_t)t * d;
            for (int i = 0; i < d; i++) xp[i] = e[i] * scale;
        }
    }

    for (int l = 0; l < L; l++) {
        const float *ln1w = w->ln_1_weight + (int64_t)l * d, *ln1b = w->ln_1_bias + (int64_t)l * d;
        for (int p = 0; p < S; p++) cr_layer_norm(xb + (int64_t)p * d, x + (int64_t)p * d, ln1w, ln1b, d);
        cr_matmul_tiled(dt, q, xb, mat_at(w->wq, dt, l, d, d), w->bq + (int64_t)l * d, d, d, S, nt);
        cr_matmul_tiled(dt, k, xb, mat_at(w->wk, dt, l, d, d), w->bk + (int64_t)l * d, d, d, S, nt);
        cr_matmul_tiled(dt, v, xb, mat_at(w->wv, dt, l, d, d), w->bv + (int64_t)l * d, d, d, S, nt);
        for (int p = 0; p < S; p++) cr_apply_rope(q + (int64_t)p * d, k + (int64_t)p * d, rc, rsn, p, d, H);

        const int last = (l == L - 1);
        if (last) memset(final_att, 0, sizeof(float) * (size_t)S * S);
        for (int h = 0; h < H; h++) {
            for (int p = 0; p < S; p++) {
                const float *qh = q + (int64_t)p * d + h * hd;
                for (int t = 0; t < S; t++)
                    att[t] = dot_head_dispatch(avx512, qh, k + (int64_t)t * d + h * hd, hd) * inv_scale;
                cr_softmax(att, S);
                if (do_contacts) memcpy(head_att + (int64_t)p * S, att, sizeof(float) * S);
                if (o->attn) memcpy(o->attn + (((int64_t)l * H + h) * S + p) * S, att, sizeof(float) * S);
                if (last) {
                    float hw = 1.0f / (float)H;
                    for (int t = 0; t < S; t++) final_att[(int64_t)p * S + t] += att[t] * hw;
                }
                float *out = oa + (int64_t)p * d + h * hd;
                memset(out, 0, sizeof(float) * hd);
                for (int t = 0; t < S; t++) axpy_head_dispatch(avx512, out, v + (int64_t)t * d + h * hd, att[t], hd);
            }
            if (do_contacts)
                cr_accumulate_head_apc(head_att, cl, S, n_res, o->contact_w[l * H + h]);
        }

        cr_matmul_tiled(dt, xb, oa, mat_at(w->wo, dt, l, d, d), w->bo + (int64_t)l * d, d, d, S, nt);
        for (int64_t i = 0; i < (int64_t)S * d; i++) x[i] += xb[i];
        const float *ln2w = w->ln_2_weight + (int64_t)l * d, *ln2b = w->ln_2_bias + (int64_t)l * d;
        for (int p = 0; p < S; p++) cr_layer_norm(xb + (int64_t)p * d, x + (int64_t)p * d, ln2w, ln2b, d);
        cr_matmul_tiled(dt, hb, xb, mat_at(w->fc1_weight, dt, l, F, d), w->fc1_bias + (int64_t)l * F, d, F, S, nt);
        cr_gelu(hb2, hb, (int64_t)S * F);
        cr_matmul_tiled(dt, xb, hb2, mat_at(w->fc2_weight, dt, l, d, F), w->fc2_bias + (int64_t)l * d, F, d, S, nt);
        for (int64_t i = 0; i < (int64_t)S * d; i++) x[i] += xb[i];
        if (o->layer_hidden) memcpy(o->layer_hidden + (int64_t)l * S * d, x, sizeof(float) * (size_t)S * d);
    }

    if (do_contacts) {
        for (int64_t i = 0; i < (int64_t)n_res * n_res; i++)
            o->contacts[i] = 1.0f / (1.0f + expf(-(cl[i] + o->contact_b)));
    }
    if (o->final_att) memcpy(o->final_att, final_att, sizeof(float) * (size_t)S * S);

    for (int p = 0; p < S; p++) cr_layer_norm(xb + (int64_t)p * d, x + (int64_t)p * d, w->ln_f_weight, w->ln_f_bias, d);
    memcpy(x, xb, sizeof(float) * (size_t)S * d);
    if (o->hidden) memcpy(o->hidden, x, sizeof(float) * (size_t)S * d);

    /* LM head, lib.rs:5379-5439: classifier = [ln_w, ln_b, dense_w, dense_b, dec_w, dec_b] */
    int64_t req = 3 * (int64_t)d + (int64_t)d * d + (int64_t)V * d + V;
    if (o->logits) {
        if (w->classifier_len >= req) {
            const float *cw = w->classifier_weights;
            const float *lnw = cw, *lnb = cw + d, *dw = cw + 2 * d, *db = cw + 2 * d + (int64_t)d * d;
            const float *decw = cw + 3 * d + (int64_t)d * d, *decb = decw + (int64_t)V * d;
            cr_matmul_tiled(CR_FP32, hb, x, dw, db, d, d, S, nt);
            cr_gelu(hb2, hb, (int64_t)S * d);
            for (int p = 0; p < S; p++) cr_layer_norm(xb + (int64_t)p * d, hb2 + (int64_t)p * d, lnw, lnb, d);
            cr_matmul_tiled(CR_FP32, o->logits, xb, decw, decb, d, V, S, nt);
        } else {
            /* tied-embedding fallback, lib.rs:5427-5439 (Q8: 5775-5787) */
            float *zb = calloc((size_t)V, 4);
            cr_matmul_tiled(dt == CR_Q8_0 ? CR_Q8_0 : CR_FP32, o->logits, x, w->token_embedding_table, zb, d, V, S, nt);
            free(zb);
        }
    }

    free(x); free(xb); free(q); free(k); free(v); free(oa); free(hb); free(hb2); free(att);
    free(head_att); free(final_att); free(rc); free(rsn); free(cl);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* The autoregressive path: forward_parallel (FP32, lib.rs:3558-3739),        */
/* forward_q8 (3741-3930), forward_q4 (4016-4201), one token at a position   */
/* against a KV cache, and generate_sequence* (6538-6827).                   */
/* ------------------------------------------------------------------------ */

/* matmul_avx2_fma, lib.rs:2577-2596: four 8-wide FMA accumulators over
 * 32-wide chunks, hsum((a0 + a1) + (a2 + a3)), + bias. */
__attribute__((target("avx2,fma")))
static void matvec_f32(float *out, const float *x, const float *w, const float *bias, int in_dim, int r0, int r1) {
    int chunks = in_dim / 32, rem = chunks * 32;
    for (int i = r0; i < r1; i++) {
        const float *wr = w + (int64_t)i * in_dim;
        __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps(), a2 = _mm256_setzero_ps(), a3 = _mm256_setzero_ps();
        for (int c = 0; c < chunks; c++) {
            int o = c * 32;
            a0 = _mm256_fmadd_ps(_mm256_loadu_ps(wr + o), _mm256_loadu_ps(x + o), a0);
            a1 = _mm256_fmadd_ps(_mm256_loadu_ps(wr + o + 8), _mm256_loadu_ps(x + o + 8), a1);
            a2 = _mm256_fmadd_ps(_mm256_loadu_ps(wr + o + 16), _mm256_loadu_ps(x + o + 16), a2);
            a3 = _mm256_fmadd_ps(_mm256_loadu_ps(wr + o + 24), _mm256_loadu_ps(x + o + 24), a3);
        }
        float v = hsum256(_mm256_add_ps(_mm256_add_ps(a0, a1), _mm256_add_ps(a2, a3)));
        for (int k = rem; k < in_dim; k++) v += wr[k] * x[k];
        out[i] = v + bias[i];
    }
}

/* matmul_q8_avx2_fma, lib.rs:2916-2948: per block an 8-wide FMA accumulator
 * of (q as f32) * x over 4 chunks, row_sum += hsum(acc) * d, + bias. */
__attribute__((target("avx2,fma")))
static void matvec_q8(float *out, const float *x, const uint8_t *w, const float *bias, int in_dim, int r0, int r1) {
    int bpr = in_dim / 32;
    for (int i = r0; i < r1; i++) {
        float row = 0.0f;
        for (int b = 0; b < bpr; b++) {
            const uint8_t *blk = w + ((int64_t)i * bpr + b) * CR_Q8_BLOCK_BYTES;
            const float *xb = x + b * 32;
            __m256 acc = _mm256_setzero_ps();
            for (int c = 0; c < 4; c++) {
                __m128i raw = _mm_loadl_epi64((const __m128i *)(blk + 4 + c * 8));
                __m256 vq = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(raw));
                acc = _mm256_fmadd_ps(vq, _mm256_loadu_ps(xb + c * 8), acc);
            }
            row += hsum256(acc) * rd_f32(blk);
        }
        out[i] = row + bias[i];
    }
}

/* matmul_q4_avx2_fma, lib.rs:3155-3210: low nibbles - 8 are elements 0..15,
 * high nibbles - 8 elements 16..31, four FMAs in element order. */
__attribute__((target("avx2,fma")))
static void matvec_q4(float *out, const float *x, const uint8_t *w, const float *bias, int in_dim, int r0, int r1) {
    int bpr = in_dim / 32;
    for (int i = r0; i < r1; i++) {
        float row = 0.0f;
        for (int b = 0; b < bpr; b++) {
            const uint8_t *blk = w + ((int64_t)i * bpr + b) * CR_Q4_BLOCK_BYTES;
            const float *xb = x + b * 32;
            int8_t lo[16], hi[16];
            for (int j = 0; j < 16; j++) {
                lo[j] = (int8_t)((blk[4 + j] & 0x0F) - 8);
                hi[j] = (int8_t)((blk[4 + j] >> 4) - 8);
            }
            __m128i vlo = _mm_loadu_si128((const __m128i *)lo), vhi = _mm_loadu_si128((const __m128i *)hi);
            __m256 acc = _mm256_setzero_ps();
            acc = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(vlo)), _mm256_loadu_ps(xb), acc);
            acc = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(vlo, 8))),
                                  _mm256_loadu_ps(xb + 8), acc);
            acc = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(vhi)), _mm256_loadu_ps(xb + 16), acc);
            acc = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(vhi, 8))),
                                  _mm256_loadu_ps(xb + 24), acc);
            row += hsum256(acc) * rd_f32(blk);
        }
        out[i] = row + bias[i];
    }
}

typedef struct {
    int32_t wdtype;
    float *out;
    const float *x;
    const void *w;
    const float *bias;
    int in_dim, out_dim;
} matvec_job;

/* run_{fp32,q8,q4}_slice, lib.rs:2845-2858, 3011-3025, 3249-3263 */
static void matvec_slice(const void *ctx, int t, int n) {
    const matvec_job *j = (const matvec_job *)ctx;
    int chunk = (j->out_dim + n - 1) / n, r0 = t * chunk;
    if (r0 >= j->out_dim) return;
    int r1 = r0 + chunk < j->out_dim ? r0 + chunk : j->out_dim;
    if (j->wdtype == CR_FP32) matvec_f32(j->out, j->x, (const float *)j->w, j->bias, j->in_dim, r0, r1);
    else if (j->wdtype == CR_Q8_0) matvec_q8(j->out, j->x, (const uint8_t *)j->w, j->bias, j->in_dim, r0, r1);
    else matvec_q4(j->out, j->x, (const uint8_t *)j->w, j->bias, j->in_dim, r0, r1);
}

/* matmul_parallel / matmul_q8_parallel / matmul_q4_parallel
 * (lib.rs:2860-2882, 3027-3051, 3265-3289) */
void cr_matmul_vec(int32_t wdtype, float *out, const float *x, const void *w, const float *bias,
                   int32_t in_dim, int32_t out_dim, int32_t num_threads) {
    matvec_job j = {wdtype, out, x, w, bias, in_dim, out_dim};
    if (num_threads <= 1 || out_dim < 32) matvec_slice(&j, 0, 1);
    else run_parallel(num_threads, matvec_slice, &j);
}

/* RunState::new, lib.rs:2464-2486: per-layer K/V caches [L][max_len][d],
 * RoPE tables for max_len positions, logits. */
cr_run_state *cr_run_state_new(const cr_config *cfg, int32_t max_len) {
    const int hd = cfg->dim / cfg->n_heads;
    cr_run_state *s = calloc(1, sizeof *s);
    s->max_len = max_len;
    s->key_cache = calloc((size_t)cfg->n_layers * max_len * cfg->dim, 4);
    s->value_cache = calloc((size_t)cfg->n_layers * max_len * cfg->dim, 4);
    s->rope_cos = calloc((size_t)max_len * (hd / 2), 4);
    s->rope_sin = calloc((size_t)max_len * (hd / 2), 4);
    s->logits = calloc((size_t)cfg->vocab_size, 4);
    cr_rope_tables(max_len, hd, s->rope_cos, s->rope_sin);
    return s;
}

void cr_run_state_free(cr_run_state *s) {
    if (!s) return;
    free(s->key_cache); free(s->value_cache); free(s->rope_cos); free(s->rope_sin); free(s->logits);
    free(s);
}

int32_t cr_forward_step(const cr_config *cfg, const cr_weights *w, int32_t token, int32_t pos, cr_run_state *s,
                        int32_t nt) {
    const int d = cfg->dim, F = cfg->hidden_dim, L = cfg->n_layers, H = cfg->n_heads, V = cfg->vocab_size;
    if (token < 0 || token >= V) return -2;
    if (pos < 0 || pos >= s->max_len) return -3;
    const int hd = d / H;
    const int32_t dt = w->dtype;
    const float inv_scale = 1.0f / sqrtf((float)hd);
    const float embed_scale = 1.0f - 0.12f;
    float *x = calloc(d, 4), *xb = calloc(d, 4), *xb2 = calloc(d, 4);
    float *q = calloc(d, 4), *k = calloc(d, 4), *v = calloc(d, 4), *att = calloc((size_t)pos + 1, 4);
    int hbw = F > d ? F : d;
    float *hb = calloc(hbw, 4), *hb2 = calloc(hbw, 4);

    /* embedding (lib.rs:3567-3575; Q8 3753-3765): <mask> is a zero row */
    if (token != 32) {
        if (dt == CR_Q8_0)
            cr_dequantize_q8((const uint8_t *)w->token_embedding_table + (int64_t)token * (d / 32) * CR_Q8_BLOCK_BYTES,
                             d / 32, x);
        else
            memcpy(x, (const float *)w->token_embedding_table + (int64_t)token * d, sizeof(float) * d);
        for (int i = 0; i < d; i++) x[i] *= embed_scale;
    }
    for (int l = 0; l < L; l++) {
        cr_layer_norm(xb, x, w->ln_1_weight + (int64_t)l * d, w->ln_1_bias + (int64_t)l * d, d);
        cr_matmul_vec(dt, q, xb, mat_at(w->wq, dt, l, d, d), w->bq + (int64_t)l * d, d, d, nt);
        cr_matmul_vec(dt, k, xb, mat_at(w->wk, dt, l, d, d), w->bk + (int64_t)l * d, d, d, nt);
        cr_matmul_vec(dt, v, xb, mat_at(w->wv, dt, l, d, d), w->bv + (int64_t)l * d, d, d, nt);
        cr_apply_rope(q, k, s->rope_cos, s->rope_sin, pos, d, H);
        float *kc = s->key_cache + (int64_t)l * s->max_len * d, *vc = s->value_cache + (int64_t)l * s->max_len * d;
        memcpy(kc + (int64_t)pos * d, k, sizeof(float) * d);
        memcpy(vc + (int64_t)pos * d, v, sizeof(float) * d);
        /* attention_head_avx1, lib.rs:3438-3483 (AVX-512 at head_dim 64 when
         * the host has it, else the 256-bit path) */
        const int avx512 = cr_attention_uses_avx512(hd);
        for (int h = 0; h < H; h++) {
            const float *qh = q + h * hd;
            for (int t = 0; t <= pos; t++)
                att[t] = dot_head_dispatch(avx512, qh, kc + (int64_t)t * d + h * hd, hd) * inv_scale;
            cr_softmax(att, pos + 1);
            float *o = xb2 + h * hd;
            memset(o, 0, sizeof(float) * hd);
            for (int t = 0; t <= pos; t++) axpy_head_dispatch(avx512, o, vc + (int64_t)t * d + h * hd, att[t], hd);
        }
        cr_matmul_vec(dt, xb, xb2, mat_at(w->wo, dt, l, d, d), w->bo + (int64_t)l * d, d, d, nt);
        for (int i = 0; i < d; i++) x[i] += xb[i];
        cr_layer_norm(xb, x, w->ln_2_weight + (int64_t)l * d, w->ln_2_bias + (int64_t)l * d, d);
        cr_matmul_vec(dt, hb, xb, mat_at(w->fc1_weight, dt, l, F, d), w->fc1_bias + (int64_t)l * F, d, F, nt);
        cr_gelu(hb2, hb, F);
        cr_matmul_vec(dt, xb, hb2, mat_at(w->fc2_weight, dt, l, d, F), w->fc2_bias + (int64_t)l * d, F, d, nt);
        for (int i = 0; i < d; i++) x[i] += xb[i];
    }
    cr_layer_norm(xb, x, w->ln_f_weight, w->ln_f_bias, d);
    /* project_lm_head_parallel / _q8 / _q4, lib.rs:3952-4015, 4203-4233 */
    int64_t req = 3 * (int64_t)d + (int64_t)d * d + (int64_t)V * d + V;
    if (w->classifier_len >= req) {
        const float *cw = w->classifier_weights;
        const float *lnw = cw, *lnb = cw + d, *dw = cw + 2 * d, *db = cw + 2 * d + (int64_t)d * d;
        const float *decw = cw + 3 * d + (int64_t)d * d, *decb = decw + (int64_t)V * d;
        cr_matmul_vec(CR_FP32, hb, xb, dw, db, d, d, nt);
        cr_gelu(hb2, hb, d);
        cr_layer_norm(hb, hb2, lnw, lnb, d);
        cr_matmul_vec(CR_FP32, s->logits, hb, decw, decb, d, V, nt);
    } else {
        float *zb = calloc((size_t)V, 4);
        cr_matmul_vec(dt == CR_Q8_0 ? CR_Q8_0 : CR_FP32, s->logits, xb, w->token_embedding_table, zb, d, V, nt);
        free(zb);
    }
    free(x); free(xb); free(xb2); free(q); free(k); free(v); free(att); free(hb); free(hb2);
    return 0;
}

/* SimpleRng, lib.rs:3506-3511: xorshift64 (13, 7, 17); seed 0 is replaced */
uint64_t cr_rng_seed(uint64_t seed) { return seed == 0 ? 0x123456789abcdefULL : seed; }

uint32_t cr_rng_next_u32(uint64_t *state) {
    uint64_t x = *state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return (uint32_t)(x & 0xffffffffULL);
}

float cr_rng_next_f32(uint64_t *state) { return (float)cr_rng_next_u32(state) / (float)UINT32_MAX; }

/* sample, lib.rs:3513-3530: only ids 4..=23 and <eos> (2) stay; T <= 0 is
 * argmax (first maximum); otherwise logits / T, softmax, inverse CDF. */
int32_t cr_sample(float *logits, int32_t V, float temperature, uint64_t *rng) {
    for (int i = 0; i < V; i++)
        if (!((i >= 4 && i <= 23) || i == 2)) logits[i] = -INFINITY;
    if (temperature <= 0.0f) {
        float mv = logits[0];
        int mi = 0;
        for (int i = 1; i < V; i++)
            if (logits[i] > mv) { mv = logits[i]; mi = i; }
        return mi;
    }
    const float inv_temp = 1.0f / temperature;
    for (int i = 0; i < V; i++)
        if (logits[i] != -INFINITY) logits[i] *= inv_temp;
    cr_softmax(logits, V);
    const float r = cr_rng_next_f32(rng);
    float cum = 0.0f;
    for (int i = 0; i < V; i++) {
        if (isnan(logits[i]) || logits[i] == 0.0f) continue;
        cum += logits[i];
        if (r <= cum) return i;
    }
    return 4;
}

/* generate_sequence_parallel / _q8 / _q4, lib.rs:6551-6827, from the token
 * ids the reference derives from the prompt (Tokenizer::encode minus the
 * trailing <eos>; [0] if empty).  max_new < 0 means no limit.  Returns the
 * number of generated tokens (written to out, at most out_cap) or < 0. */
int32_t cr_generate(const cr_config *cfg, const cr_weights *w, const int32_t *prompt, int32_t n_prompt,
                    float temperature, int32_t max_new, uint64_t seed, int32_t max_seq_len, int32_t nt,
                    int32_t *out, int32_t out_cap) {
    cr_run_state *s = cr_run_state_new(cfg, max_seq_len);
    int pos = 0, rc = 0;
    for (int i = 0; i < n_prompt && pos < max_seq_len; i++) {
        if ((rc = cr_forward_step(cfg, w, prompt[i], pos, s, nt)) != 0) goto done;
        pos++;
    }
    {
        uint64_t rng = cr_rng_seed(seed);
        int limit = max_new >= 0 ? (pos + max_new < max_seq_len ? pos + max_new : max_seq_len) : max_seq_len;
        int n = 0;
        float *lg = malloc(sizeof(float) * cfg->vocab_size);
        while (pos < limit) {
            memcpy(lg, s->logits, sizeof(float) * cfg->vocab_size);
            int tok = cr_sample(lg, cfg->vocab_size, temperature, &rng);
            if (tok == 2) break;
            if (n >= out_cap) { rc = -5; break; }
            out[n++] = tok;
            if ((rc = cr_forward_step(cfg, w, tok, pos, s, nt)) != 0) break;
            pos++;
        }
        free(lg);
        if (!rc) rc = n;
    }
done:
    cr_run_state_free(s);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* Metrics, lib.rs:2271-2346                                                  */
/* ------------------------------------------------------------------------ */

float cr_cosine_similarity(const float *a, const float *b, int64_t n) {
    float dot = 0, na = 0, nb = 0;
    for (int64_t i = 0; i < n; i++) { dot += a[i] * b[i]; na += a[i] * a[i]; nb += b[i] * b[i]; }
    float den = sqrtf(na) * sqrtf(nb);
    return den > 1e-12f ? dot / den : 1.0f;
}

float cr_rmse(const float *a, const float *b, int64_t n) {
    if (n == 0) return 0.0f;
    double s = 0;
    for (int64_t i = 0; i < n; i++) { double df = (double)(a[i] - b[i]); s += df * df; }
    return (float)sqrt(s / (double)n);
}

/* Iterator::max_by keeps the LAST of equal maxima (lib.rs:2306-2307). */
static int argmax_last(const float *x, int n) {
    int best = 0;
    for (int i = 1; i < n; i++) if (!(x[i] < x[best])) best = i;
    return best;
}

float cr_top1_match_rate(const float *a, const float *b, int64_t n, int32_t V) {
    if (V == 0) return 1.0f;
    int64_t nt = n / V;
    if (nt == 0) return 1.0f;
    int64_t m = 0;
    for (int64_t t = 0; t < nt; t++) m += argmax_last(a + t * V, V) == argmax_last(b + t * V, V);
    return (float)m / (float)nt;
}

float cr_kl_divergence(const float *a, const float *b, int64_t n, int32_t V) {
    if (V == 0) return 0.0f;
    int64_t nt = n / V;
    if (nt == 0) return 0.0f;
    float total = 0.0f;
    for (int64_t t = 0; t < nt; t++) {
        const float *r = a + t * V, *s = b + t * V;
        float mr = -INFINITY, ms = -INFINITY;
        for (int i = 0; i < V; i++) { mr = fmaxf(mr, r[i]); ms = fmaxf(ms, s[i]); }
        float sr = 0, ss = 0;
        for (int i = 0; i < V; i++) { sr += expf(r[i] - mr); ss += expf(s[i] - ms); }
        float kl = 0;
        for (int i = 0; i < V; i++) {
            float p = fmaxf(expf(r[i] - mr) / sr, 1e-12f), qq = fmaxf(expf(s[i] - ms) / ss, 1e-12f);
            kl += p * (logf(p) - logf(qq));
        }
        total += kl;
    }
    return total / (float)nt;
}
