/*
 * levo_oracle.c — CPU restatement of the reference's hot-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (the checker). Built by oracle/Makefile with
 * -std=c11 -ffp-contract=off so that every a*b+c below rounds twice, exactly
 * like the reference's ISO C++17 build for baseline x86-64
 * (CMakeLists.txt:8-10) and ggml's ISO C11 CPU backend.
 */
#define _GNU_SOURCE
#include "levo_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* F16 <-> F32                                                                */
/* ------------------------------------------------------------------------- */

/* IEEE binary32 -> binary16, round to nearest, ties to even (what
 * ggml_fp32_to_fp16_row produces with F16C or with its software fallback). */
uint16_t lo_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t exp = (x >> 23) & 0xffu;
    uint32_t mant = x & 0x7fffffu;
    if (exp == 0xffu) {
        if (mant != 0) return (uint16_t)(sign | 0x7e00u | (mant >> 13));
        return (uint16_t)(sign | 0x7c00u);
    }
    if (exp >= 143u) return (uint16_t)(sign | 0x7c00u); /* >= 2^16: overflow */
    if (exp >= 113u) {                                    /* normal half */
        uint32_t h = ((exp - 112u) << 10) | (mant >> 13);
        const uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* may carry to inf */
        return (uint16_t)(sign | h);
    }
    if (exp < 102u) return (uint16_t)sign; /* < 2^-25 rounds to zero */
    /* subnormal half: value = M * 2^(exp-150), unit 2^-24 */
    mant |= 0x800000u;
    const uint32_t shift = 126u - exp; /* 14 .. 24 */
    uint32_t h = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

float lo_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    const uint32_t mant = h & 0x3ffu;
    uint32_t x;
    if (exp == 0) {
        const float v = ldexpf((float)mant, -24); /* exact */
        memcpy(&x, &v, sizeof x);
        x |= sign;
    } else if (exp == 0x1fu) {
        x = sign | 0x7f800000u | (mant << 13);
    } else {
        x = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &x, sizeof f);
    return f;
}

void lo_fp32_to_fp16_row(const float * x, uint16_t * y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = lo_fp32_to_fp16(x[i]);
}

void lo_fp16_to_fp32_row(const uint16_t * x, float * y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = lo_fp16_to_fp32(x[i]);
}

/* ------------------------------------------------------------------------- */
/* Row-partitioned worker threads (ggml-cpu hands row i to thread i % nth).   */
/* ------------------------------------------------------------------------- */

typedef void (*lo_row_fn)(void * ctx, int ith, int nth, pthread_barrier_t * barrier);

typedef struct {
    lo_row_fn fn;
    void * ctx;
    int ith, nth;
    pthread_barrier_t * barrier;
} lo_thread_arg;

static void * lo_thread_main(void * p) {
    lo_thread_arg * a = (lo_thread_arg *)p;
    a->fn(a->ctx, a->ith, a->nth, a->barrier);
    return NULL;
}

static void lo_parallel(lo_row_fn fn, void * ctx, int n_threads) {
    if (n_threads < 1) n_threads = 1;
    if (n_threads == 1) {
        fn(ctx, 0, 1, NULL);
        return;
    }
    pthread_barrier_t barrier;
    pthread_barrier_init(&barrier, NULL, (unsigned)n_threads);
    pthread_t * threads = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)n_threads);
    lo_thread_arg * args = (lo_thread_arg *)malloc(sizeof(lo_thread_arg) * (size_t)n_threads);
    for (int i = 0; i < n_threads; ++i) {
        args[i].fn = fn;
        args[i].ctx = ctx;
        args[i].ith = i;
        args[i].nth = n_threads;
        args[i].barrier = &barrier;
    }
    for (int i = 1; i < n_threads; ++i) pthread_create(&threads[i], NULL, lo_thread_main, &args[i]);
    lo_thread_main(&args[0]);
    for (int i = 1; i < n_threads; ++i) pthread_join(threads[i], NULL);
    pthread_barrier_destroy(&barrier);
    free(threads);
    free(args);
}

static void lo_sync(pthread_barrier_t * barrier) {
    if (barrier) pthread_barrier_wait(barrier);
}

/* ------------------------------------------------------------------------- */
/* SnakeBeta (src/levo-audio-ops.cpp:146-151)                                 */
/* ------------------------------------------------------------------------- */

typedef struct {
    const float * x;
    const float * alpha;
    const float * beta;
    float * work;
    float * y;
    int64_t channels, time;
} lo_snake_ctx;

/* Five unfused passes, one per ggml node, each over the thread's rows with a
 * barrier in between (ggml computes one node at a time). The intermediate
 * lives in one buffer updated in place, as ggml's graph allocator does for
 * unary ops whose parent has no other consumer. */
static void lo_snake_rows(void * p, int ith, int nth, pthread_barrier_t * barrier) {
    const lo_snake_ctx * c = (const lo_snake_ctx *)p;
    const int64_t T = c->time;
    for (int64_t ch = ith; ch < c->channels; ch += nth) { /* ggml_mul(input, alpha) */
        const float a = c->alpha[ch];
        const float * x = c->x + ch * T;
        float * w = c->work + ch * T;
        for (int64_t t = 0; t < T; ++t) w[t] = x[t] * a;
    }
    lo_sync(barrier);
    for (int64_t ch = ith; ch < c->channels; ch += nth) { /* ggml_sin */
        float * w = c->work + ch * T;
        for (int64_t t = 0; t < T; ++t) w[t] = sinf(w[t]);
    }
    lo_sync(barrier);
    for (int64_t ch = ith; ch < c->channels; ch += nth) { /* ggml_sqr */
        float * w = c->work + ch * T;
        for (int64_t t = 0; t < T; ++t) w[t] = w[t] * w[t];
    }
    lo_sync(barrier);
    for (int64_t ch = ith; ch < c->channels; ch += nth) { /* ggml_div(periodic, beta) */
        const float b = c->beta[ch];
        float * w = c->work + ch * T;
        for (int64_t t = 0; t < T; ++t) w[t] = w[t] / b;
    }
    lo_sync(barrier);
    for (int64_t ch = ith; ch < c->channels; ch += nth) { /* ggml_add(input, .) */
        const float * x = c->x + ch * T;
        const float * w = c->work + ch * T;
        float * y = c->y + ch * T;
        for (int64_t t = 0; t < T; ++t) y[t] = x[t] + w[t];
    }
}

void lo_snake_beta_f32(const float * x, const float * alpha_log, const float * beta_log,
                       float * y, int64_t channels, int64_t time, int n_threads) {
    float * alpha = (float *)malloc(sizeof(float) * (size_t)channels);
    float * beta = (float *)malloc(sizeof(float) * (size_t)channels);
    float * work = (float *)malloc(sizeof(float) * (size_t)(channels * time));
    for (int64_t c = 0; c < channels; ++c) {
        alpha[c] = expf(alpha_log[c]);                /* ggml_exp(alpha_log) */
        const float e = expf(beta_log[c]);            /* ggml_exp(beta_log) */
        beta[c] = e * 1.0f + 1.0e-9f;                 /* ggml_scale_bias(., 1, 1e-9) */
    }
    lo_snake_ctx ctx = {x, alpha, beta, work, y, channels, time};
    lo_parallel(lo_snake_rows, &ctx, n_threads);
    free(work);
    free(beta);
    free(alpha);
}

/* ------------------------------------------------------------------------- */
/* Residual add + RMSNorm / LayerNorm                                         */
/* ------------------------------------------------------------------------- */

/* ggml-cpu rms_norm row (scalar algorithm): sum of x*x in ggml_float (double)
 * in index order, mean = sum/n rounded to float, scale = 1/sqrtf(mean + eps). */
static float lo_rms_scale(const float * h, int64_t n, float eps) {
    double sum = 0.0;
    for (int64_t i = 0; i < n; ++i) sum += (double)(h[i] * h[i]);
    const float mean = (float)(sum / (double)n);
    return 1.0f / sqrtf(mean + eps);
}

/* ggml-cpu norm row: mean from a ggml_float sum, y = x - mean, variance from
 * a ggml_float sum of y*y, scale = 1/sqrtf(variance + eps), y *= scale. */
static void lo_norm_row(const float * h, float * y, int64_t n, float eps) {
    double sum = 0.0;
    for (int64_t i = 0; i < n; ++i) sum += (double)h[i];
    const float mean = (float)(sum / (double)n);
    double sum2 = 0.0;
    for (int64_t i = 0; i < n; ++i) {
        const float v = h[i] - mean;
        y[i] = v;
        sum2 += (double)(v * v);
    }
    const float variance = (float)(sum2 / (double)n);
    const float scale = 1.0f / sqrtf(variance + eps);
    for (int64_t i = 0; i < n; ++i) y[i] = y[i] * scale;
}

typedef struct {
    const void * x;
    const void * delta;
    const void * w;
    const void * b;
    void * h_out;
    void * y;
    int64_t rows, dim;
    float eps;
} lo_norm_ctx;

static void lo_rms_f16_rows(void * p, int ith, int nth, pthread_barrier_t * barrier) {
    (void)barrier;
    const lo_norm_ctx * c = (const lo_norm_ctx *)p;
    const int64_t D = c->dim;
    float * h = (float *)malloc(sizeof(float) * (size_t)D);
    for (int64_t r = ith; r < c->rows; r += nth) {
        const uint16_t * x = (const uint16_t *)c->x + r * D;
        const uint16_t * d = c->delta ? (const uint16_t *)c->delta + r * D : NULL;
        const uint16_t * w = (const uint16_t *)c->w;
        uint16_t * ho = c->h_out ? (uint16_t *)c->h_out + r * D : NULL;
        uint16_t * y = (uint16_t *)c->y + r * D;
        for (int64_t i = 0; i < D; ++i) {
            /* ggml_add on F16 tensors: F32 sum rounded to F16 (src/levo-kv.cpp:462,507) */
            const uint16_t h16 = d ? lo_fp32_to_fp16(lo_fp16_to_fp32(x[i]) + lo_fp16_to_fp32(d[i])) : x[i];
            if (ho) ho[i] = h16;
            h[i] = lo_fp16_to_fp32(h16); /* cast_f32 (src/levo-kv.cpp:157) */
        }
        const float scale = lo_rms_scale(h, D, c->eps);
        for (int64_t i = 0; i < D; ++i) {
            const uint16_t n16 = lo_fp32_to_fp16(h[i] * scale); /* cast_f16 (:158) */
            /* ggml_mul F16 x F16 weight -> F16 (:159) */
            y[i] = lo_fp32_to_fp16(lo_fp16_to_fp32(n16) * lo_fp16_to_fp32(w[i]));
        }
    }
    free(h);
}

static void lo_rms_f32_rows(void * p, int ith, int nth, pthread_barrier_t * barrier) {
    (void)barrier;
    const lo_norm_ctx * c = (const lo_norm_ctx *)p;
    const int64_t D = c->dim;
    float * h = (float *)malloc(sizeof(float) * (size_t)D);
    for (int64_t r = ith; r < c->rows; r += nth) {
        const float * x = (const float *)c->x + r * D;
        const float * d = c->delta ? (const float *)c->delta + r * D : NULL;
        const float * w = (const float *)c->w;
        float * ho = c->h_out ? (float *)c->h_out + r * D : NULL;
        float * y = (float *)c->y + r * D;
        for (int64_t i = 0; i < D; ++i) {
            h[i] = d ? x[i] + d[i] : x[i];
            if (ho) ho[i] = h[i];
        }
        const float scale = lo_rms_scale(h, D, c->eps);
        for (int64_t i = 0; i < D; ++i) y[i] = (h[i] * scale) * w[i];
    }
    free(h);
}

static void lo_ln_f32_rows(void * p, int ith, int nth, pthread_barrier_t * barrier) {
    (void)barrier;
    const lo_norm_ctx * c = (const lo_norm_ctx *)p;
    const int64_t D = c->dim;
    float * h = (float *)malloc(sizeof(float) * (size_t)D);
    float * n = (float *)malloc(sizeof(float) * (size_t)D);
    for (int64_t r = ith; r < c->rows; r += nth) {
        const float * x = (const float *)c->x + r * D;
        const float * d = c->delta ? (const float *)c->delta + r * D : NULL;
        const float * g = (const float *)c->w;
        const float * b = (const float *)c->b;
        float * ho = c->h_out ? (float *)c->h_out + r * D : NULL;
        float * y = (float *)c->y + r * D;
        for (int64_t i = 0; i < D; ++i) {
            h[i] = d ? x[i] + d[i] : x[i];
            if (ho) ho[i] = h[i];
        }
        lo_norm_row(h, n, D, c->eps);                                    /* ggml_norm */
        for (int64_t i = 0; i < D; ++i) y[i] = (n[i] * g[i]) + b[i];     /* ggml_mul, ggml_add */
    }
    free(n);
    free(h);
}

static void lo_ln_f16_rows(void * p, int ith, int nth, pthread_barrier_t * barrier) {
    (void)barrier;
    const lo_norm_ctx * c = (const lo_norm_ctx *)p;
    const int64_t D = c->dim;
    float * h = (float *)malloc(sizeof(float) * (size_t)D);
    float * n = (float *)malloc(sizeof(float) * (size_t)D);
    for (int64_t r = ith; r < c->rows; r += nth) {
        const uint16_t * x = (const uint16_t *)c->x + r * D;
        const uint16_t * d = c->delta ? (const uint16_t *)c->delta + r * D : NULL;
        const uint16_t * g = (const uint16_t *)c->w;
        const uint16_t * b = (const uint16_t *)c->b;
        uint16_t * ho = c->h_out ? (uint16_t *)c->h_out + r * D : NULL;
        uint16_t * y = (uint16_t *)c->y + r * D;
        for (int64_t i = 0; i < D; ++i) {
            const uint16_t h16 = d ? lo_fp32_to_fp16(lo_fp16_to_fp32(x[i]) + lo_fp16_to_fp32(d[i])) : x[i];
            if (ho) ho[i] = h16;
            h[i] = lo_fp16_to_fp32(h16);
        }
        lo_norm_row(h, n, D, c->eps);
        for (int64_t i = 0; i < D; ++i)
            y[i] = lo_fp32_to_fp16((n[i] * lo_fp16_to_fp32(g[i])) + lo_fp16_to_fp32(b[i]));
    }
    free(n);
    free(h);
}

void lo_residual_rms_norm_f16(const uint16_t * x, const uint16_t * delta, const uint16_t * weight,
                              uint16_t * h_out, uint16_t * y, int64_t rows, int64_t dim,
                              float eps, int n_threads) {
    lo_norm_ctx ctx = {x, delta, weight, NULL, h_out, y, rows, dim, eps};
    lo_parallel(lo_rms_f16_rows, &ctx, n_threads);
}

void lo_residual_rms_norm_f32(const float * x, const float * delta, const float * weight,
                              float * h_out, float * y, int64_t rows, int64_t dim,
                              float eps, int n_threads) {
    lo_norm_ctx ctx = {x, delta, weight, NULL, h_out, y, rows, dim, eps};
    lo_parallel(lo_rms_f32_rows, &ctx, n_threads);
}

void lo_residual_layer_norm_f32(const float * x, const float * delta, const float * gamma,
                                const float * beta, float * h_out, float * y, int64_t rows,
                                int64_t dim, float eps, int n_threads) {
    lo_norm_ctx ctx = {x, delta, gamma, beta, h_out, y, rows, dim, eps};
    lo_parallel(lo_ln_f32_rows, &ctx, n_threads);
}

void lo_residual_layer_norm_f16(const uint16_t * x, const uint16_t * delta, const uint16_t * gamma,
                                const uint16_t * beta, uint16_t * h_out, uint16_t * y,
                                int64_t rows, int64_t dim, float eps, int n_threads) {
    lo_norm_ctx ctx = {x, delta, gamma, beta, h_out, y, rows, dim, eps};
    lo_parallel(lo_ln_f16_rows, &ctx, n_threads);
}

/* Entry b, channel c of a per-batch modulation vector: ggml_add(dynamic,
 * learned) of modulation_chunk (src/levo-flow-estimator.cpp:95-104), or the
 * dynamic part alone. */
static float lo_batch_value(const lo_batch_vector * v, int64_t b, int64_t c) {
    const float dyn = v->dynamic[b * v->stride + c];
    return v->learned ? dyn + v->learned[c] : dyn;
}

/* A Flow estimator block boundary (src/levo-flow-estimator.cpp:221-233,
 * 243-261), one ggml op at a time:
 *   current = (delta * gate) + x     ggml_add(ggml_mul(out, gate), residual) :221-227, 243-246
 *   t = (norm(current) * gamma) + beta   layer_norm :106-109
 *   y = (t * (scale + 1)) + shift    add_scale_shift :89-93 (ggml_scale_bias(scale, 1, 1))
 * with gate / scale / shift taken at batch entry b = row / rows_per_batch. */
void lo_residual_layer_norm_modulated_f32(const float * x, const float * delta, const lo_batch_vector * gate,
                                          const float * gamma, const float * beta,
                                          const lo_batch_vector * scale, const lo_batch_vector * shift,
                                          float * h_out, float * y, int64_t rows, int64_t rows_per_batch,
                                          int64_t dim, float eps) {
    float * h = (float *)malloc(sizeof(float) * (size_t)dim);
    float * n = (float *)malloc(sizeof(float) * (size_t)dim);
    for (int64_t r = 0; r < rows; ++r) {
        const int64_t b = r / rows_per_batch;
        const float * xr = x + r * dim;
        const float * dr = delta ? delta + r * dim : NULL;
        for (int64_t c = 0; c < dim; ++c) {
            if (!dr) h[c] = xr[c];
            else if (gate) h[c] = (dr[c] * lo_batch_value(gate, b, c)) + xr[c];
            else h[c] = xr[c] + dr[c];
            if (h_out) h_out[r * dim + c] = h[c];
        }
        lo_norm_row(h, n, dim, eps);
        for (int64_t c = 0; c < dim; ++c) {
            float t = (n[c] * gamma[c]) + beta[c];
            if (scale) {
                const float one_plus = lo_batch_value(scale, b, c) + 1.0f;
                t = (t * one_plus) + lo_batch_value(shift, b, c);
            }
            y[r * dim + c] = t;
        }
    }
    free(n);
    free(h);
}

/* ------------------------------------------------------------------------- */
/* CFG                                                                        */
/* ------------------------------------------------------------------------- */

void lo_apply_cfg(const float * cond, const float * uncond, float * out, int64_t n, float scale) {
    for (int64_t i = 0; i < n; ++i) out[i] = uncond[i] + scale * (cond[i] - uncond[i]);
}

/* ------------------------------------------------------------------------- */
/* mt19937_64 and the sampler                                                 */
/* ------------------------------------------------------------------------- */

#define LO_MT_N 312
#define LO_MT_M 156

void lo_mt_seed(lo_mt19937_64 * rng, uint64_t seed) {
    rng->state[0] = seed;
    for (int i = 1; i < LO_MT_N; ++i) {
        const uint64_t prev = rng->state[i - 1];
        rng->state[i] = 6364136223846793005ULL * (prev ^ (prev >> 62)) + (uint64_t)i;
    }
    rng->index = LO_MT_N;
}

uint64_t lo_mt_next(lo_mt19937_64 * rng) {
    if (rng->index >= LO_MT_N) {
        const uint64_t upper = 0xFFFFFFFF80000000ULL; /* w - r = 33 high bits */
        const uint64_t lower = 0x000000007FFFFFFFULL; /* r = 31 low bits */
        for (int i = 0; i < LO_MT_N; ++i) {
            const uint64_t y = (rng->state[i] & upper) | (rng->state[(i + 1) % LO_MT_N] & lower);
            uint64_t next = rng->state[(i + LO_MT_M) % LO_MT_N] ^ (y >> 1);
            if (y & 1u) next ^= 0xB5026F5AA96619E9ULL;
            rng->state[i] = next;
        }
        rng->index = 0;
    }
    uint64_t z = rng->state[rng->index++];
    z ^= (z >> 29) & 0x5555555555555555ULL;
    z ^= (z << 17) & 0x71D67FFFEDA60000ULL;
    z ^= (z << 37) & 0xFFF7EEE000000000ULL;
    z ^= z >> 43;
    return z;
}

void lo_mt_discard(lo_mt19937_64 * rng, uint64_t count) {
    for (uint64_t i = 0; i < count; ++i) (void)lo_mt_next(rng);
}

/* manual_uniform (src/levo-sampling.cpp:12-18): (53 random bits + 0.5) / 2^53. */
double lo_manual_uniform(lo_mt19937_64 * rng, uint64_t * draws) {
    const double denom = 9007199254740992.0;
    if (draws) ++*draws;
    return ((double)(lo_mt_next(rng) >> 11) + 0.5) / denom;
}

/* src/levo-sampling.cpp:39-47: each distinct id in [0, limit) is divided once. */
int lo_repetition_penalty(float * logits, int64_t vocab, const int64_t * recent, int64_t n_recent,
                          float penalty, int64_t vocabulary_limit) {
    if (!(penalty > 0.0f) || !isfinite(penalty)) return LO_ERR_PENALTY;
    const int64_t limit = vocabulary_limit == 0 ? vocab : (vocabulary_limit < vocab ? vocabulary_limit : vocab);
    if (limit <= 0 || n_recent <= 0) return LO_OK;
    unsigned char * seen = (unsigned char *)calloc((size_t)limit, 1);
    for (int64_t i = 0; i < n_recent; ++i) {
        const int64_t t = recent[i];
        if (t >= 0 && t < limit && !seen[t]) {
            seen[t] = 1;
            logits[t] /= penalty;
        }
    }
    free(seen);
    return LO_OK;
}

static int lo_desc_float(const void * a, const void * b) {
    const float x = *(const float *)a, y = *(const float *)b;
    return (x < y) - (x > y);
}

/* Threshold of the stable descending sort (src/levo-sampling.cpp:85-89): the
 * value at rank top_k-1, i.e. the top_k-th largest value with multiplicity. */
static float lo_kth_largest(const float * v, int64_t n, int64_t k) {
    float * copy = (float *)malloc(sizeof(float) * (size_t)n);
    memcpy(copy, v, sizeof(float) * (size_t)n);
    qsort(copy, (size_t)n, sizeof(float), lo_desc_float);
    const float t = copy[k - 1];
    free(copy);
    return t;
}

int64_t lo_top_k_candidates(const float * logits, int64_t vocab, int64_t top_k,
                            int64_t * best, int64_t * candidates, int64_t cap) {
    if (vocab <= 0) return LO_ERR_EMPTY;
    for (int64_t i = 0; i < vocab; ++i)
        if (isnan(logits[i])) return LO_ERR_NAN;
    const int filter = top_k > 0 && top_k < vocab;
    const float threshold = filter ? lo_kth_largest(logits, vocab, top_k) : -INFINITY;
    int64_t count = 0;
    int64_t b = -1;
    for (int64_t i = 0; i < vocab; ++i) {
        if (filter && logits[i] < threshold) continue;
        if (count < cap) candidates[count] = i;
        ++count;
        if (b < 0 || logits[b] < logits[i]) b = i; /* std::max_element keeps the first max */
    }
    *best = b;
    return count;
}

int lo_sample_top_k(const float * input, int64_t vocab, int64_t top_k, float temperature,
                    int use_sampling, lo_mt19937_64 * rng, uint64_t * draws, int64_t * token) {
    if (vocab <= 0) return LO_ERR_EMPTY;
    if (!isfinite(temperature) || temperature < 0.0f) return LO_ERR_TEMPERATURE;
    int64_t * cand = (int64_t *)malloc(sizeof(int64_t) * (size_t)vocab);
    int64_t best = 0;
    const int64_t n = lo_top_k_candidates(input, vocab, top_k, &best, cand, vocab);
    if (n < 0) {
        free(cand);
        return (int)n;
    }
    if (!use_sampling || temperature == 0.0f) {
        *token = best;
        free(cand);
        return LO_OK;
    }
    float max_logit = -INFINITY;
    for (int64_t i = 0; i < n; ++i)
        if (max_logit < input[cand[i]]) max_logit = input[cand[i]]; /* std::max */
    double * weights = (double *)malloc(sizeof(double) * (size_t)n);
    double total = 0.0;
    for (int64_t i = 0; i < n; ++i) {
        const float value = input[cand[i]];
        if (isinf(value) && value < 0) weights[i] = 0.0;
        else weights[i] = exp((double)((value - max_logit) / temperature));
        total += weights[i];
    }
    if (!(total > 0.0) || !isfinite(total)) {
        *token = best;
    } else {
        const double target = lo_manual_uniform(rng, draws) * total;
        double cumulative = 0.0;
        int64_t chosen = cand[n - 1];
        for (int64_t i = 0; i < n; ++i) {
            cumulative += weights[i];
            if (target < cumulative) {
                chosen = cand[i];
                break;
            }
        }
        *token = chosen;
    }
    free(weights);
    free(cand);
    return LO_OK;
}

int lo_sample_streams(const float * logits, int64_t n_streams, int64_t vocab,
                      int use_sampling, float temperature, int64_t top_k_mixed,
                      int64_t top_k_detail, float repetition_penalty,
                      const int64_t * recent, int64_t n_recent,
                      const int64_t * ignore_tokens, int64_t n_ignore,
                      lo_mt19937_64 * rng, uint64_t * draws, int64_t * tokens) {
    float * adjusted = (float *)malloc(sizeof(float) * (size_t)(vocab > 0 ? vocab : 1));
    int status = LO_OK;
    for (int64_t q = 0; q < n_streams && status == LO_OK; ++q) {
        memcpy(adjusted, logits + q * vocab, sizeof(float) * (size_t)vocab);
        if (recent) {
            status = lo_repetition_penalty(adjusted, vocab, recent + q * n_recent, n_recent,
                                           repetition_penalty, vocab == 0 ? 0 : vocab - 1);
            if (status != LO_OK) break;
        }
        if (q == 0)
            for (int64_t i = 0; i < n_ignore; ++i)
                if (ignore_tokens[i] >= 0 && ignore_tokens[i] < vocab) adjusted[ignore_tokens[i]] = -INFINITY;
        const int64_t k = q == 0 ? top_k_mixed : top_k_detail;
        status = lo_sample_top_k(adjusted, vocab, k, temperature, use_sampling, rng, draws, &tokens[q]);
    }
    free(adjusted);
    return status;
}

/* ------------------------------------------------------------------------- */
/* Flow Euler / CFG                                                           */
/* ------------------------------------------------------------------------- */

void lo_flow_incontext(float * state, const float * noise, const float * context,
                       int64_t n_prefix, float time, float sigma_min) {
    const float noise_scale = 1.0f - (1.0f - sigma_min) * time;
    for (int64_t e = 0; e < n_prefix; ++e) state[e] = noise_scale * noise[e] + time * context[e];
}

void lo_flow_cfg_euler(float * state, const float * v_uncond, const float * v_cond, int64_t n,
                       float guidance, float dt) {
    for (int64_t e = 0; e < n; ++e) {
        const float v = v_cond ? v_uncond[e] + guidance * (v_cond[e] - v_uncond[e]) : v_uncond[e];
        state[e] += dt * v;
    }
}

/* ------------------------------------------------------------------------- */
/* Q8_0 / Q4_0 block formats (ggml public layout): {f16 d; int8 qs[32]} = 34 B */
/* and {f16 d; u8 qs[16]} = 18 B, little-endian.                              */
/* ------------------------------------------------------------------------- */

/* float -> int8 as x86-64 does it for (int8_t)f: cvttss2si (int32, invalid ->
 * 0x80000000) then the low byte. Only non-finite products reach the invalid
 * case (a block whose |max| is so small that 1/d overflows). */
static int8_t lo_trunc_i8(float f) {
    if (!(fabsf(f) < 2147483648.0f)) return 0;
    return (int8_t)(int32_t)f;
}

void lo_quantize_row_q8_0(const float * x, void * out, int64_t k) {
    unsigned char * y = (unsigned char *)out;
    const int64_t nb = k / 32;
    for (int64_t i = 0; i < nb; ++i) {
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const float v = fabsf(x[i * 32 + j]);
            amax = amax > v ? amax : v; /* MAX(amax, fabsf(v)) */
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t dh = lo_fp32_to_fp16(d);
        unsigned char * blk = y + i * 34;
        blk[0] = (unsigned char)(dh & 0xffu);
        blk[1] = (unsigned char)(dh >> 8);
        for (int j = 0; j < 32; ++j) {
            const float x0 = x[i * 32 + j] * id;
            blk[2 + j] = (unsigned char)lo_trunc_i8(roundf(x0));
        }
    }
}

void lo_quantize_row_q4_0(const float * x, void * out, int64_t k) {
    unsigned char * y = (unsigned char *)out;
    const int64_t nb = k / 32;
    for (int64_t i = 0; i < nb; ++i) {
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const float v = x[i * 32 + j];
            if (amax < fabsf(v)) {
                amax = fabsf(v);
                max = v;
            }
        }
        const float d = max / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t dh = lo_fp32_to_fp16(d);
        unsigned char * blk = y + i * 18;
        blk[0] = (unsigned char)(dh & 0xffu);
        blk[1] = (unsigned char)(dh >> 8);
        for (int j = 0; j < 16; ++j) {
            const float x0 = x[i * 32 + j] * id;
            const float x1 = x[i * 32 + 16 + j] * id;
            int q0 = lo_trunc_i8(x0 + 8.5f);
            int q1 = lo_trunc_i8(x1 + 8.5f);
            q0 = q0 < 15 ? q0 : 15;
            q1 = q1 < 15 ? q1 : 15;
            blk[2 + j] = (unsigned char)((uint8_t)q0 | (uint8_t)((uint8_t)q1 << 4));
        }
    }
}

void lo_dequantize_row_q8_0(const void * in, float * y, int64_t k) {
    const unsigned char * x = (const unsigned char *)in;
    const int64_t nb = k / 32;
    for (int64_t i = 0; i < nb; ++i) {
        const unsigned char * blk = x + i * 34;
        const float d = lo_fp16_to_fp32((uint16_t)(blk[0] | (blk[1] << 8)));
        for (int j = 0; j < 32; ++j) y[i * 32 + j] = (float)(int8_t)blk[2 + j] * d;
    }
}

void lo_dequantize_row_q4_0(const void * in, float * y, int64_t k) {
    const unsigned char * x = (const unsigned char *)in;
    const int64_t nb = k / 32;
    for (int64_t i = 0; i < nb; ++i) {
        const unsigned char * blk = x + i * 18;
        const float d = lo_fp16_to_fp32((uint16_t)(blk[0] | (blk[1] << 8)));
        for (int j = 0; j < 16; ++j) {
            const int x0 = (blk[2 + j] & 0x0f) - 8;
            const int x1 = (blk[2 + j] >> 4) - 8;
            y[i * 32 + j] = (float)x0 * d;
            y[i * 32 + 16 + j] = (float)x1 * d;
        }
    }
}

static size_t lo_row_size(int type, int64_t n) {
    if (type == LO_TYPE_Q8_0) return (size_t)(n / 32) * 34u;
    if (type == LO_TYPE_Q4_0) return (size_t)(n / 32) * 18u;
    if (type == LO_TYPE_Q4_K) return (size_t)(n / 256) * 144u;
    if (type == LO_TYPE_Q5_K) return (size_t)(n / 256) * 176u;
    if (type == LO_TYPE_Q6_K) return (size_t)(n / 256) * 210u;
    return 0;
}

size_t lo_quantize_chunk(int type, const float * src, void * dst, int64_t start, int64_t nrows,
                         int64_t n_per_row) {
    const int kq = type == LO_TYPE_Q4_K || type == LO_TYPE_Q5_K || type == LO_TYPE_Q6_K;
    const size_t row_size = lo_row_size(type, n_per_row);
    if (row_size == 0 || n_per_row % (kq ? 256 : 32) != 0 || start % n_per_row != 0) return 0;
    const int64_t start_row = start / n_per_row;
    unsigned char * out = (unsigned char *)dst + (size_t)start_row * row_size;
    const int64_t n = nrows * n_per_row;
    if (type == LO_TYPE_Q8_0) lo_quantize_row_q8_0(src + start, out, n);
    else if (type == LO_TYPE_Q4_0) lo_quantize_row_q4_0(src + start, out, n);
    else if (type == LO_TYPE_Q4_K) lo_quantize_row_q4_K(src + start, out, n);
    else if (type == LO_TYPE_Q5_K) lo_quantize_row_q5_K(src + start, out, n);
    else lo_quantize_row_q6_K(src + start, out, n);
    return (size_t)nrows * row_size;
}

size_t lo_quantize_f16_rows_padded(int type, const uint16_t * src, int64_t nrows, int64_t src_cols,
                                   int64_t dst_cols, void * dst) {
    if (dst_cols < src_cols) return 0;
    float * values = (float *)calloc((size_t)(nrows * dst_cols), sizeof(float));
    for (int64_t r = 0; r < nrows; ++r)
        lo_fp16_to_fp32_row(src + r * src_cols, values + r * dst_cols, src_cols);
    const size_t n = lo_quantize_chunk(type, values, dst, 0, nrows, dst_cols);
    free(values);
    return n;
}

/* ------------------------------------------------------------------------- */
/* Seeded synthetic inputs (src/levo-render.cpp:87-112)                       */
/* ------------------------------------------------------------------------- */

static uint64_t lo_splitmix64(uint64_t * state) {
    *state += 0x9e3779b97f4a7c15ULL;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

static double lo_uniform_open(uint64_t * state) {
    return ((double)(lo_splitmix64(state) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

void lo_gaussian_noise(float * out, int64_t count, uint64_t seed) {
    uint64_t state = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < count; i += 2) {
        const double radius = sqrt(-2.0 * log(lo_uniform_open(&state)));
        const double angle = two_pi * lo_uniform_open(&state);
        out[i] = (float)(radius * cos(angle));
        if (i + 1 < count) out[i + 1] = (float)(radius * sin(angle));
    }
}

/* ------------------------------------------------------------------------- */
/* Q8_0 x Q8_0 matrix-vector product (ggml CPU mul_mat, generic vec_dot)      */
/* ------------------------------------------------------------------------- */

void lo_mul_mat_q8_0(const void * w, const float * x, float * y, int64_t rows, int64_t k, int64_t n_vec) {
    const int64_t nb = k / 32;
    unsigned char * xq = (unsigned char *)malloc((size_t)(nb * 34));
    if (!xq) return;
    for (int64_t v = 0; v < n_vec; ++v) {
        lo_quantize_row_q8_0(x + v * k, xq, k);
        for (int64_t r = 0; r < rows; ++r) {
            const unsigned char * wr = (const unsigned char *)w + r * nb * 34;
            float sumf = 0.0f;
            for (int64_t ib = 0; ib < nb; ++ib) {
                const unsigned char * bw = wr + ib * 34;
                const unsigned char * bx = xq + ib * 34;
                int sumi = 0;
                for (int j = 0; j < 32; ++j) sumi += (int)(int8_t)bw[2 + j] * (int)(int8_t)bx[2 + j];
                const float dw = lo_fp16_to_fp32((uint16_t)(bw[0] | (bw[1] << 8)));
                const float dx = lo_fp16_to_fp32((uint16_t)(bx[0] | (bx[1] << 8)));
                sumf += (float)sumi * (dw * dx);
            }
            y[v * rows + r] = sumf;
        }
    }
    free(xq);
}

/* ------------------------------------------------------------------------- */
/* K-quant super-blocks (ggml public layout, QK_K = 256, little-endian):      */
/*   block_q4_K {f16 d; f16 dmin; u8 scales[12]; u8 qs[128]}            144 B */
/*   block_q5_K {f16 d; f16 dmin; u8 scales[12]; u8 qh[32]; u8 qs[128]} 176 B */
/*   block_q6_K {u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d}           210 B */
/*   block_q8_K {f32 d; i8 qs[256]; i16 bsums[16]}                      292 B */
/* Routed to by the Q6_K / Q5_K_M / Q4_K_M profiles                          */
/* (src/levo-quantization.h:47-55, 96-118).                                  */
/* ------------------------------------------------------------------------- */

/* ggml's nearest_int: fval + 1.5 * 2^23 rounds to an integer (ties to even)
 * for |fval| < 2^22, read back from the mantissa bits. */
static int lo_nearest_int(float fval) {
    const float val = fval + 12582912.0f;
    int32_t i;
    memcpy(&i, &val, sizeof(i));
    return (i & 0x007fffff) - 0x00400000;
}

static float lo_h(const unsigned char * p) { return lo_fp16_to_fp32((uint16_t)(p[0] | (p[1] << 8))); }

/* get_scale_min_k4: sub-block j's 6-bit scale and min from the 12 packed
 * bytes (j < 4: low 6 bits of bytes j and j + 4; j >= 4: a nibble of byte
 * j + 4 and the top 2 bits of bytes j - 4 and j). */
static void lo_scale_min_k4(int j, const unsigned char * q, int * d, int * m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4);
    }
}

void lo_quantize_row_q8_K(const float * x, void * out, int64_t k) {
    unsigned char * y = (unsigned char *)out;
    const int64_t nb = k / 256;
    for (int64_t i = 0; i < nb; ++i, x += 256) {
        unsigned char * blk = y + i * 292;
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < 256; ++j) {
            const float ax = fabsf(x[j]);
            if (ax > amax) {
                amax = ax;
                max = x[j];
            }
        }
        if (!amax) {  /* the reference leaves bsums as they were; zero here */
            memset(blk, 0, 292);
            continue;
        }
        const float iscale = -127.0f / max;
        int8_t qs[256];
        for (int j = 0; j < 256; ++j) {
            const int v = lo_nearest_int(iscale * x[j]);
            qs[j] = (int8_t)(v < 127 ? v : 127);
        }
        const float d = 1.0f / iscale;
        memcpy(blk, &d, 4);
        memcpy(blk + 4, qs, 256);
        for (int j = 0; j < 16; ++j) {
            int sum = 0;
            for (int ii = 0; ii < 16; ++ii) sum += qs[j * 16 + ii];
            const int16_t s16 = (int16_t)sum;
            memcpy(blk + 260 + 2 * j, &s16, 2);
        }
    }
}

/* ---- K-quant block quantizers: ggml's quantize_row_q{4,5,6}_K_ref as
 * reached from ggml_quantize_chunk(type, src, dst, start, nrows, n_per_row,
 * NULL) (tools/levo-quantize.cpp:386-388; no importance matrix). Restated
 * from ggml's published source (ggml-quants.c at the reference's pinned
 * submodule 8846b79e): make_qkx2_quants (Q4_K / Q5_K) and make_qx_quants
 * with rmse_type 1 (Q6_K). These routines live in ggml-base, built for the
 * baseline x86-64 ISA (no FMA instructions), so every float operation rounds
 * on its own, as this library does (-ffp-contract=off). Inputs are finite
 * (write_tensor rejects non-finite tensors, tools/levo-quantize.cpp:330). */

#define LO_GROUP_MAX_EPS 1e-15f

/* make_qkx2_quants: an affine code L in [0, nmax] with scale and min found by
 * a grid of nstep + 1 trial inverse scales around nmax / (max - min), each
 * refined by a weighted least-squares fit of (scale, min) to the codes; the
 * trial with the smallest weighted squared error wins. `min` and the trial
 * scales follow each accepted trial (as in ggml). Returns the scale and
 * stores -min in *the_min. */
static float lo_make_qkx2_quants(int n, int nmax, const float * x, const float * weights, uint8_t * L,
                                 float * the_min, uint8_t * Laux, float rmin, float rdelta, int nstep) {
    float min = x[0];
    float max = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        const float w = weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -min;
        return 0.f;
    }
    float iscale = nmax / (max - min);
    float scale = 1 / iscale;
    float best_mad = 0;
    for (int i = 0; i < n; ++i) {
        const int l = lo_nearest_int(iscale * (x[i] - min));
        L[i] = (uint8_t)(l < 0 ? 0 : l > nmax ? nmax : l);
        float diff = scale * L[i] + min - x[i];
        diff = diff * diff;
        const float w = weights[i];
        best_mad += w * diff;
    }
    if (nstep < 1) {
        *the_min = -min;
        return scale;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = lo_nearest_int(iscale * (x[i] - min));
            l = l < 0 ? 0 : l > nmax ? nmax : l;
            Laux[i] = (uint8_t)l;
            const float w = weights[i];
            sum_l += w * l;
            sum_l2 += w * l * l;
            sum_xl += w * l * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float mad = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                diff = diff * diff;
                const float w = weights[i];
                mad += w * diff;
            }
            if (mad < best_mad) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_mad = mad;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

/* make_qx_quants(n, nmax, x, L, rmse_type = 1, qw = NULL): symmetric codes
 * L - nmax in [-nmax, nmax - 1] from the signed extreme, weights x^2, the
 * least-squares scale, then 18 trial inverse scales -(nmax + 0.1 is) / max
 * (is = -9..9, not 0), keeping the one that maximizes sumlx^2 / suml2. */
static float lo_make_qx_quants(int n, int nmax, const float * x, int8_t * L) {
    float max = 0;
    float amax = 0;
    for (int i = 0; i < n; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    if (amax < LO_GROUP_MAX_EPS) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = -nmax / max;
    float sumlx = 0;
    float suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = lo_nearest_int(iscale * x[i]);
        l = l < -nmax ? -nmax : l > nmax - 1 ? nmax - 1 : l;
        L[i] = (int8_t)(l + nmax);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    float scale = suml2 ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / max;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; ++i) {
            int l = lo_nearest_int(iscale * x[i]);
            l = l < -nmax ? -nmax : l > nmax - 1 ? nmax - 1 : l;
            const float w = x[i] * x[i];
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                int l = lo_nearest_int(iscale * x[i]);
                l = l < -nmax ? -nmax : l > nmax - 1 ? nmax - 1 : l;
                L[i] = (int8_t)(nmax + l);
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

static uint16_t lo_h16(float f) { return lo_fp32_to_fp16(f); }

static void lo_put_h(unsigned char * p, float f) {
    const uint16_t h = lo_h16(f);
    p[0] = (unsigned char)(h & 0xff);
    p[1] = (unsigned char)(h >> 8);
}

/* quantize_row_q4_K_ref (nmax 15, rmin -1, rdelta 0.1, 20 steps) and
 * quantize_row_q5_K_ref (nmax 31, rmin -0.5, rdelta 0.1, 15 steps): per
 * 32-value sub-block weights sqrt(mean x^2) + |x|, make_qkx2_quants; the
 * eight scales and mins quantized to 6 bits against the largest of each
 * (d = max_scale / 63, dmin = max_min / 63, stored F16); every value then
 * re-coded as nearest_int((x + dmin*m) / (d*sc)) (a sub-block whose quantized
 * scale is 0 keeps its make_qkx2_quants codes). */
static void lo_quantize_row_q45_K(int q5, const float * x, void * out, int64_t k) {
    unsigned char * y = (unsigned char *)out;
    const int nmax = q5 ? 31 : 15;
    const int bsz = q5 ? 176 : 144;
    for (int64_t i = 0; i < k / 256; ++i, x += 256) {
        unsigned char * blk = y + i * bsz;
        uint8_t L[256], Laux[32];
        float weights[32], mins[8], scales[8];
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < 8; ++j) {
            float sum_x2 = 0;
            for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
            const float av_x = sqrtf(sum_x2 / 32);
            for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(x[32 * j + l]);
            scales[j] = q5 ? lo_make_qkx2_quants(32, nmax, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, -0.5f, 0.1f, 15)
                           : lo_make_qkx2_quants(32, nmax, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, -1.f, 0.1f, 20);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
        const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
        unsigned char * sc = blk + 4;
        memset(sc, 0, 12);
        for (int j = 0; j < 8; ++j) {
            uint8_t ls = (uint8_t)lo_nearest_int(inv_scale * scales[j]);
            uint8_t lm = (uint8_t)lo_nearest_int(inv_min * mins[j]);
            ls = ls < 63 ? ls : 63;
            lm = lm < 63 ? lm : 63;
            if (j < 4) {
                sc[j] = ls;
                sc[j + 4] = lm;
            } else {
                sc[j + 4] = (unsigned char)((ls & 0xF) | ((lm & 0xF) << 4));
                sc[j - 4] |= (unsigned char)((ls >> 4) << 6);
                sc[j - 0] |= (unsigned char)((lm >> 4) << 6);
            }
        }
        lo_put_h(blk, max_scale / 63.f);
        lo_put_h(blk + 2, max_min / 63.f);
        const float d16 = lo_h(blk), dmin16 = lo_h(blk + 2);
        for (int j = 0; j < 8; ++j) {
            int s, m;
            lo_scale_min_k4(j, sc, &s, &m);
            const float d = d16 * s;
            if (!d) continue;
            const float dm = dmin16 * m;
            for (int ii = 0; ii < 32; ++ii) {
                int l = lo_nearest_int((x[32 * j + ii] + dm) / d);
                l = l < 0 ? 0 : l > nmax ? nmax : l;
                L[32 * j + ii] = (uint8_t)l;
            }
        }
        if (!q5) {
            unsigned char * q = blk + 16;
            for (int j = 0; j < 256; j += 64, q += 32)
                for (int l = 0; l < 32; ++l) q[l] = (unsigned char)(L[j + l] | (L[j + l + 32] << 4));
        } else {
            unsigned char * qh = blk + 16;
            unsigned char * ql = blk + 48;
            memset(qh, 0, 32);
            unsigned m1 = 1, m2 = 2;
            for (int n = 0; n < 256; n += 64, ql += 32, m1 <<= 2, m2 <<= 2) {
                for (int j = 0; j < 32; ++j) {
                    int l1 = L[n + j];
                    if (l1 > 15) {
                        l1 -= 16;
                        qh[j] |= (unsigned char)m1;
                    }
                    int l2 = L[n + j + 32];
                    if (l2 > 15) {
                        l2 -= 16;
                        qh[j] |= (unsigned char)m2;
                    }
                    ql[j] = (unsigned char)(l1 | (l2 << 4));
                }
            }
        }
    }
}

void lo_quantize_row_q4_K(const float * x, void * y, int64_t k) { lo_quantize_row_q45_K(0, x, y, k); }
void lo_quantize_row_q5_K(const float * x, void * y, int64_t k) { lo_quantize_row_q45_K(1, x, y, k); }

/* quantize_row_q6_K_ref: 16-value sub-blocks, make_qx_quants(16, 32, ., 1);
 * the scale with the largest magnitude (first of equal magnitudes) sets
 * iscale = -128 / max_scale, d = F16(1 / iscale), 8-bit sub-block scales
 * min(127, nearest_int(iscale * scale)); values re-coded as
 * clamp(nearest_int(x / (d * sc)), -32, 31) + 32 (a zero quantized scale
 * keeps the make_qx_quants codes); a block whose scales are all below 1e-15
 * is all zero. */
void lo_quantize_row_q6_K(const float * x, void * out, int64_t k) {
    unsigned char * y = (unsigned char *)out;
    for (int64_t i = 0; i < k / 256; ++i, x += 256) {
        unsigned char * blk = y + i * 210;
        int8_t L[256];
        float scales[16];
        float max_scale = 0, max_abs_scale = 0;
        for (int ib = 0; ib < 16; ++ib) {
            const float scale = lo_make_qx_quants(16, 32, x + 16 * ib, L + 16 * ib);
            scales[ib] = scale;
            const float abs_scale = fabsf(scale);
            if (abs_scale > max_abs_scale) {
                max_abs_scale = abs_scale;
                max_scale = scale;
            }
        }
        if (max_abs_scale < LO_GROUP_MAX_EPS) {
            memset(blk, 0, 210);
            lo_put_h(blk + 208, 0.f);
            continue;
        }
        const float iscale = -128.f / max_scale;
        lo_put_h(blk + 208, 1 / iscale);
        int8_t * sc = (int8_t *)(blk + 192);
        for (int ib = 0; ib < 16; ++ib) {
            const int v = lo_nearest_int(iscale * scales[ib]);
            sc[ib] = (int8_t)(v < 127 ? v : 127);
        }
        const float d16 = lo_h(blk + 208);
        for (int j = 0; j < 16; ++j) {
            const float d = d16 * sc[j];
            if (!d) continue;
            for (int ii = 0; ii < 16; ++ii) {
                int l = lo_nearest_int(x[16 * j + ii] / d);
                l = l < -32 ? -32 : l > 31 ? 31 : l;
                L[16 * j + ii] = (int8_t)(l + 32);
            }
        }
        unsigned char * ql = blk;
        unsigned char * qh = blk + 128;
        for (int j = 0; j < 256; j += 128, ql += 64, qh += 32) {
            for (int l = 0; l < 32; ++l) {
                const uint8_t q1 = L[j + l + 0] & 0xF;
                const uint8_t q2 = L[j + l + 32] & 0xF;
                const uint8_t q3 = L[j + l + 64] & 0xF;
                const uint8_t q4 = L[j + l + 96] & 0xF;
                ql[l + 0] = (unsigned char)(q1 | (q3 << 4));
                ql[l + 32] = (unsigned char)(q2 | (q4 << 4));
                qh[l] = (unsigned char)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4) |
                                        ((L[j + l + 96] >> 4) << 6));
            }
        }
    }
}

/* dequantize_row_q4_K / q5_K: y = d1 * q - m1 with d1 = d * sc, m1 = dmin * m,
 * every operation rounded on its own (ggml-base built for the baseline x86-64
 * ISA, as for the quantizers). d (F16, 11 significant bits) times a 6-bit scale
 * times a code below 32 needs at most 22 bits, so d1 * q is exact in F32 and a
 * contracted build gives the same bits. */
void lo_dequantize_row_q4_K(const void * in, float * y, int64_t k) {
    const unsigned char * x = (const unsigned char *)in;
    for (int64_t i = 0; i < k / 256; ++i) {
        const unsigned char * blk = x + i * 144;
        const float d = lo_h(blk), min = lo_h(blk + 2);
        const unsigned char * sc = blk + 4;
        const unsigned char * q = blk + 16;
        for (int j = 0; j < 4; ++j, q += 32) {
            int s0, m0, s1, m1;
            lo_scale_min_k4(2 * j, sc, &s0, &m0);
            lo_scale_min_k4(2 * j + 1, sc, &s1, &m1);
            const float d1 = d * (float)s0, mn1 = min * (float)m0;
            const float d2 = d * (float)s1, mn2 = min * (float)m1;
            for (int l = 0; l < 32; ++l) *y++ = d1 * (float)(q[l] & 0xF) - mn1;
            for (int l = 0; l < 32; ++l) *y++ = d2 * (float)(q[l] >> 4) - mn2;
        }
    }
}

void lo_dequantize_row_q5_K(const void * in, float * y, int64_t k) {
    const unsigned char * x = (const unsigned char *)in;
    for (int64_t i = 0; i < k / 256; ++i) {
        const unsigned char * blk = x + i * 176;
        const float d = lo_h(blk), min = lo_h(blk + 2);
        const unsigned char * sc = blk + 4;
        const unsigned char * qh = blk + 16;
        const unsigned char * ql = blk + 48;
        unsigned u1 = 1, u2 = 2;
        for (int j = 0; j < 4; ++j, ql += 32, u1 <<= 2, u2 <<= 2) {
            int s0, m0, s1, m1;
            lo_scale_min_k4(2 * j, sc, &s0, &m0);
            lo_scale_min_k4(2 * j + 1, sc, &s1, &m1);
            const float d1 = d * (float)s0, mn1 = min * (float)m0;
            const float d2 = d * (float)s1, mn2 = min * (float)m1;
            for (int l = 0; l < 32; ++l) *y++ = d1 * (float)((ql[l] & 0xF) + ((qh[l] & u1) ? 16 : 0)) - mn1;
            for (int l = 0; l < 32; ++l) *y++ = d2 * (float)((ql[l] >> 4) + ((qh[l] & u2) ? 16 : 0)) - mn2;
        }
    }
}

/* Q6_K element e of a block: 6-bit code (low 4 bits in ql, high 2 in qh) - 32. */
static int lo_q6_code(const unsigned char * blk, int e) {
    const int n = e / 128, r = e % 128, quarter = r / 32, l = r % 32;
    const unsigned char * ql = blk + 64 * n;
    const unsigned char * qh = blk + 128 + 32 * n;
    const int lo = quarter & 1 ? ql[l + 32] : ql[l];
    const int nib = quarter < 2 ? (lo & 0xF) : (lo >> 4);
    return (nib | (((qh[l] >> (2 * quarter)) & 3) << 4)) - 32;
}

void lo_dequantize_row_q6_K(const void * in, float * y, int64_t k) {
    const unsigned char * x = (const unsigned char *)in;
    for (int64_t i = 0; i < k / 256; ++i) {
        const unsigned char * blk = x + i * 210;
        const float d = lo_h(blk + 208);
        const int8_t * sc = (const int8_t *)(blk + 192);
        /* y = d * sc * q, left to right (two roundings) */
        for (int e = 0; e < 256; ++e) *y++ = d * (float)sc[e / 16] * (float)lo_q6_code(blk, e);
    }
}

/* ggml_vec_dot_q{4,5,6}_K_q8_K, generic loops: per super-block the integer
 * sums of scale * (q_w * q_x) in 8 lanes (element l goes to lane l % 8), then
 * sums[lane] += (d_w * d_x) * aux32[lane]; for Q4_K / Q5_K also
 * sumi = sum_j bsums[j] * min[j / 2] and sumf -= (dmin_w * d_x) * sumi; at
 * the end sumf += sums[0..7] in order. */
static float lo_vec_dot_kquant(int type, const unsigned char * w, const unsigned char * xq, int64_t nb) {
    float sums[8] = {0};
    float sumf = 0.0f;
    const int wbytes = type == LO_TYPE_Q4_K ? 144 : type == LO_TYPE_Q5_K ? 176 : 210;
    for (int64_t i = 0; i < nb; ++i) {
        const unsigned char * blk = w + i * wbytes;
        const unsigned char * bx = xq + i * 292;
        float dx;
        memcpy(&dx, bx, 4);
        const int8_t * q8 = (const int8_t *)(bx + 4);
        int a[256];
        int scales[16];
        int mins[8] = {0};
        if (type == LO_TYPE_Q6_K) {
            for (int e = 0; e < 256; ++e) a[e] = lo_q6_code(blk, e);
            for (int j = 0; j < 16; ++j) scales[j] = ((const int8_t *)(blk + 192))[j];
        } else {
            const unsigned char * sc = blk + 4;
            const unsigned char * qh = blk + 16;
            const unsigned char * ql = blk + (type == LO_TYPE_Q5_K ? 48 : 16);
            for (int j = 0; j < 4; ++j) {
                for (int l = 0; l < 32; ++l) {
                    a[64 * j + l] = ql[32 * j + l] & 0xF;
                    a[64 * j + 32 + l] = ql[32 * j + l] >> 4;
                    if (type == LO_TYPE_Q5_K) {
                        a[64 * j + l] += (qh[l] >> (2 * j)) & 1 ? 16 : 0;
                        a[64 * j + 32 + l] += (qh[l] >> (2 * j + 1)) & 1 ? 16 : 0;
                    }
                }
            }
            for (int j = 0; j < 8; ++j) lo_scale_min_k4(j, sc, &scales[j], &mins[j]);
        }
        const int sub = type == LO_TYPE_Q6_K ? 16 : 32;  /* elements per scale */
        int32_t aux32[8] = {0};
        for (int e = 0; e < 256; ++e) aux32[e % 8] += scales[e / sub] * (int16_t)(q8[e] * a[e]);
        const float d = (type == LO_TYPE_Q6_K ? lo_h(blk + 208) : lo_h(blk)) * dx;
        for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux32[l];
        if (type != LO_TYPE_Q6_K) {
            int sumi = 0;
            for (int j = 0; j < 16; ++j) {
                int16_t b;
                memcpy(&b, bx + 260 + 2 * j, 2);
                sumi += b * mins[j / 2];
            }
            const float dmin = lo_h(blk + 2) * dx;
            sumf -= dmin * (float)sumi;
        }
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

int64_t lo_kquant_block_bytes(int type) {
    switch (type) {
        case LO_TYPE_Q4_K: return 144;
        case LO_TYPE_Q5_K: return 176;
        case LO_TYPE_Q6_K: return 210;
        case LO_TYPE_Q8_K: return 292;
        default: return 0;
    }
}

void lo_dequantize_row_kquant(int type, const void * x, float * y, int64_t k) {
    if (type == LO_TYPE_Q4_K) lo_dequantize_row_q4_K(x, y, k);
    else if (type == LO_TYPE_Q5_K) lo_dequantize_row_q5_K(x, y, k);
    else if (type == LO_TYPE_Q6_K) lo_dequantize_row_q6_K(x, y, k);
}

float lo_vec_dot_kquant_q8_K(int type, const void * w, const void * xq, int64_t k) {
    return lo_vec_dot_kquant(type, (const unsigned char *)w, (const unsigned char *)xq, k / 256);
}

void lo_mul_mat_kquant(int type, const void * w, const float * x, float * y, int64_t rows, int64_t k,
                       int64_t n_vec) {
    const int64_t nb = k / 256;
    const int64_t wrow = nb * lo_kquant_block_bytes(type);
    unsigned char * xq = (unsigned char *)malloc((size_t)(nb * 292));
    if (!xq) return;
    for (int64_t v = 0; v < n_vec; ++v) {
        lo_quantize_row_q8_K(x + v * k, xq, k);
        for (int64_t r = 0; r < rows; ++r)
            y[v * rows + r] = lo_vec_dot_kquant(type, (const unsigned char *)w + r * wrow, xq, nb);
    }
    free(xq);
}

/* ------------------------------------------------------------------------- */
/* Conv1d (im2col + F32 mul_mat + bias), stride 1                            */
/* ------------------------------------------------------------------------- */

typedef struct {
    const float * x;
    int64_t c_in, t_in;
    const float * w;
    int64_t c_out, kernel;
    const float * bias;
    int64_t padding, dilation, t_out;
    float * y;
    int64_t co0, co1;
} lo_conv_job;

static void * lo_conv_rows(void * arg) {
    const lo_conv_job * j = (const lo_conv_job *)arg;
    const int64_t kk = j->c_in * j->kernel;
    float * col = (float *)malloc((size_t)kk * sizeof(float));
    if (!col) return NULL;
    for (int64_t t = 0; t < j->t_out; ++t) {
        /* the im2col column of output t */
        for (int64_t ci = 0; ci < j->c_in; ++ci) {
            for (int64_t k = 0; k < j->kernel; ++k) {
                const int64_t ti = t + k * j->dilation - j->padding;
                col[ci * j->kernel + k] = (ti >= 0 && ti < j->t_in) ? j->x[ci * j->t_in + ti] : 0.0f;
            }
        }
        for (int64_t co = j->co0; co < j->co1; ++co) {
            const float * wr = j->w + co * kk;
            float sum = 0.0f;
            for (int64_t e = 0; e < kk; ++e) sum += wr[e] * col[e];
            j->y[co * j->t_out + t] = j->bias ? sum + j->bias[co] : sum;
        }
    }
    free(col);
    return NULL;
}

void lo_conv1d_f32(const float * x, int64_t c_in, int64_t t_in, const float * w, int64_t c_out, int64_t kernel,
                   const float * bias, int64_t padding, int64_t dilation, float * y, int threads) {
    const int64_t t_out = t_in + 2 * padding - dilation * (kernel - 1);
    if (t_out <= 0) return;
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t tid[64];
    lo_conv_job jobs[64];
    const int64_t per = (c_out + threads - 1) / threads;
    int started = 0;
    for (int i = 0; i < threads; ++i) {
        lo_conv_job * j = &jobs[i];
        j->x = x; j->c_in = c_in; j->t_in = t_in; j->w = w; j->c_out = c_out; j->kernel = kernel;
        j->bias = bias; j->padding = padding; j->dilation = dilation; j->t_out = t_out; j->y = y;
        j->co0 = i * per;
        j->co1 = (i + 1) * per < c_out ? (i + 1) * per : c_out;
        if (j->co0 >= j->co1) break;
        if (threads == 1 || pthread_create(&tid[i], NULL, lo_conv_rows, j) != 0) {
            lo_conv_rows(j);
            tid[i] = 0;
        }
        started = i + 1;
    }
    for (int i = 0; i < started; ++i) if (threads > 1 && tid[i]) pthread_join(tid[i], NULL);
}

/* ------------------------------------------------------------------------- */
/* ConvTranspose1d (ggml_conv_transpose_1d + crop + bias)                     */
/* ------------------------------------------------------------------------- */

void lo_conv_transpose1d_f32(const float * x, int64_t c_in, int64_t t_in, const float * w, int64_t c_out,
                             int64_t kernel, int64_t stride, int64_t padding, const float * bias, float * y) {
    const int64_t t_full = (t_in - 1) * stride + kernel;
    const int64_t t_out = t_full - 2 * padding;
    if (t_out <= 0) return;
    float * full = (float *)calloc((size_t)t_full, sizeof(float));
    float * col = (float *)malloc((size_t)c_in * sizeof(float));
    if (!full || !col) {
        free(full);
        free(col);
        return;
    }
    for (int64_t co = 0; co < c_out; ++co) {
        memset(full, 0, (size_t)t_full * sizeof(float));
        for (int64_t i = 0; i < t_in; ++i) {
            for (int64_t ci = 0; ci < c_in; ++ci) col[ci] = x[ci * t_in + i];
            for (int64_t k = 0; k < kernel; ++k) {
                float v = 0.0f;
                for (int64_t ci = 0; ci < c_in; ++ci) v += w[(ci * c_out + co) * kernel + k] * col[ci];
                full[i * stride + k] += v;
            }
        }
        for (int64_t t = 0; t < t_out; ++t) {
            y[co * t_out + t] = bias ? full[t + padding] + bias[co] : full[t + padding];
        }
    }
    free(full);
    free(col);
}
