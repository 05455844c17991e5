/*
 * Oracle: plain-C restatement of the reference's CPU path for the speculative verify
 * step. TEST INFRASTRUCTURE ONLY (the checker and the CPU baseline); the product never
 * links it.
 *
 * Build: -O3 -ffp-contract=off, no fast-math. Floating-point expressions keep the
 * reference's evaluation order exactly: Rust never contracts a*b+c into an FMA, never
 * reassociates, and `iter().sum::<f32>()` is a left fold. Math functions go to glibc
 * (expf, sinf, cosf, sqrtf, pow), as Rust std does on Linux.
 *
 * Parity pins: see tests/test_oracle_*.py (known answers from the reference's own unit
 * tests, f64 brute force, closed forms, and an independent Hugging Face Qwen2 model).
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static __thread char g_err[512];

static int fail(const char* msg) {
    snprintf(g_err, sizeof g_err, "%s", msg);
    return -1;
}

const char* or_last_error(void) { return g_err; }

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + ts.tv_nsec * 1e-9;
}

/* ---------------------------------------------------------------------------------------
 * bf16 helpers: src/kernels.rs:8-15, 45-48
 * ------------------------------------------------------------------------------------- */
static inline float bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline float bf16_at(const uint8_t* p, size_t i) {
    return bf16_to_f32((uint16_t)(p[2 * i] | (p[2 * i + 1] << 8)));
}

/* src/quant.rs:26-33: round to nearest bf16, ties to even; NaN passes through. */
float or_bf16_round(float v) {
    uint32_t bits;
    memcpy(&bits, &v, 4);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return v;
    uint32_t lsb = (bits >> 16) & 1u;
    uint32_t r = (bits + 0x7fffu + lsb) & 0xffff0000u;
    float f;
    memcpy(&f, &r, 4);
    return f;
}

/* ---------------------------------------------------------------------------------------
 * Formats: src/weights.rs:14-55, 158-227
 * ------------------------------------------------------------------------------------- */
size_t or_row_bytes(or_fmt f, size_t cols) {
    if (f.bits == 16) return cols * 2;
    return cols * (size_t)f.bits / 8 + cols / (size_t)f.group * 2;
}

int or_validate(or_fmt f, const size_t* cols, size_t n) {
    if (f.bits == 16) return 0;
    if (f.bits != 8 && f.bits != 4) return fail("quantization supports 8 or 4 bits");
    if (f.group < 16 || f.group > 256 || f.group % 16 != 0)
        return fail("group size must be a multiple of 16 between 16 and 256");
    for (size_t i = 0; i < n; i++)
        if (cols[i] % (size_t)f.group != 0) return fail("group size does not divide a matrix width");
    return 0;
}

enum { T_INPUT_NORM, T_DOWN, T_GATE, T_UP, T_POST_NORM, T_K_B, T_K_W, T_O_W, T_Q_B, T_Q_W, T_V_B, T_V_W, N_T };

/* matrix_shape (src/weights.rs:188-211): rows, cols of the seven matrices; 0 for vectors. */
static void slot_shape(const or_cfg* c, int slot, size_t* rows, size_t* cols, size_t* vec_len) {
    size_t h = c->hidden, i = c->inter, kv = c->kv_heads * c->head_dim;
    *rows = *cols = *vec_len = 0;
    switch (slot) {
        case T_INPUT_NORM: case T_POST_NORM: case T_Q_B: *vec_len = h; break;
        case T_K_B: case T_V_B: *vec_len = kv; break;
        case T_DOWN: *rows = h; *cols = i; break;
        case T_GATE: case T_UP: *rows = i; *cols = h; break;
        case T_K_W: case T_V_W: *rows = kv; *cols = h; break;
        case T_O_W: case T_Q_W: *rows = h; *cols = h; break;
    }
}

size_t or_layer_layout(const or_cfg* c, size_t* ranges24) {
    size_t off = 0;
    for (int s = 0; s < N_T; s++) {
        size_t rows, cols, vl;
        slot_shape(c, s, &rows, &cols, &vl);
        size_t len = rows ? rows * or_row_bytes(c->format, cols) : vl * 2;
        ranges24[2 * s] = off;
        ranges24[2 * s + 1] = len;
        off += len;
    }
    return off;
}

/* ---------------------------------------------------------------------------------------
 * Dot products: src/kernels.rs:27-92
 * ------------------------------------------------------------------------------------- */
static inline float sum8(const float* acc) {
    /* `acc.iter().sum::<f32>()`: a left fold. */
    float s = -0.0f;
    for (int k = 0; k < 8; k++) s = s + acc[k];
    return s;
}

float or_dot_bf16(const uint8_t* w, const float* x, size_t n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t nc = n / 8;
    for (size_t c = 0; c < nc; c++)
        for (int k = 0; k < 8; k++) acc[k] = acc[k] + bf16_at(w, c * 8 + k) * x[c * 8 + k];
    float sum = sum8(acc);
    for (size_t i = nc * 8; i < n; i++) sum = sum + bf16_at(w, i) * x[i];
    return sum;
}

float or_dot_q8(const uint8_t* row, const float* x, size_t cols, size_t group) {
    const uint8_t* scales = row + cols;
    float total = 0.0f;
    for (size_t g = 0; g < cols / group; g++) {
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        const uint8_t* q = row + g * group;
        const float* xg = x + g * group;
        for (size_t c = 0; c < group / 8; c++)
            for (int k = 0; k < 8; k++) acc[k] = acc[k] + (float)(int8_t)q[c * 8 + k] * xg[c * 8 + k];
        total = total + bf16_at(scales, g) * sum8(acc);
    }
    return total;
}

float or_dot_q4(const uint8_t* row, const float* x, size_t cols, size_t group) {
    const uint8_t* scales = row + cols / 2;
    size_t half = group / 2;
    float total = 0.0f;
    for (size_t g = 0; g < cols / group; g++) {
        const uint8_t* bytes = row + g * half;
        const float* lo = x + g * group;
        const float* hi = lo + half;
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (size_t c = 0; c < half / 8; c++)
            for (int k = 0; k < 8; k++) {
                uint8_t b = bytes[c * 8 + k];
                float p_lo = (float)((int)(b & 15) - 8) * lo[c * 8 + k];
                float p_hi = (float)((int)(b >> 4) - 8) * hi[c * 8 + k];
                acc[k] = acc[k] + (p_lo + p_hi);
            }
        total = total + bf16_at(scales, g) * sum8(acc);
    }
    return total;
}

/* src/kernels.rs:95-121 */
void or_dequant_row(or_fmt f, const uint8_t* raw, float* out, size_t cols) {
    if (f.bits == 16) {
        for (size_t i = 0; i < cols; i++) out[i] = bf16_at(raw, i);
        return;
    }
    size_t group = f.group;
    const uint8_t* scales = raw + cols * f.bits / 8;
    for (size_t g = 0; g < cols / group; g++) {
        float s = bf16_at(scales, g);
        if (f.bits == 8) {
            for (size_t j = 0; j < group; j++) out[g * group + j] = (float)(int8_t)raw[g * group + j] * s;
        } else {
            size_t half = group / 2;
            for (size_t j = 0; j < half; j++) {
                uint8_t b = raw[g * half + j];
                out[g * group + j] = (float)((int)(b & 15) - 8) * s;
                out[g * group + j + half] = (float)((int)(b >> 4) - 8) * s;
            }
        }
    }
}

static float dot_fmt(or_fmt f, const uint8_t* row, const float* x, size_t cols) {
    if (f.bits == 16) return or_dot_bf16(row, x, cols);
    if (f.bits == 8) return or_dot_q8(row, x, cols, f.group);
    return or_dot_q4(row, x, cols, f.group);
}

/* ---------------------------------------------------------------------------------------
 * Pool: src/pool.rs:77-137. Persistent workers; tasks handed out from an atomic counter;
 * the caller takes part; one job at a time.
 * ------------------------------------------------------------------------------------- */
typedef void (*task_fn)(void* ctx, size_t task);

struct or_pool {
    int workers;
    pthread_t* th;
    pthread_mutex_t mu;
    pthread_cond_t start, done;
    uint64_t generation;
    int pending, shutdown;
    task_fn fn;
    void* ctx;
    size_t n_tasks;
    atomic_size_t next;
};

static void run_tasks(or_pool* p) {
    for (;;) {
        size_t i = atomic_fetch_add_explicit(&p->next, 1, memory_order_relaxed);
        if (i >= p->n_tasks) break;
        p->fn(p->ctx, i);
    }
}

static void* worker_main(void* arg) {
    or_pool* p = (or_pool*)arg;
    uint64_t seen = 0;
    pthread_mutex_lock(&p->mu);
    for (;;) {
        while (!p->shutdown && p->generation == seen) pthread_cond_wait(&p->start, &p->mu);
        if (p->shutdown) break;
        seen = p->generation;
        pthread_mutex_unlock(&p->mu);
        run_tasks(p);
        pthread_mutex_lock(&p->mu);
        if (--p->pending == 0) pthread_cond_signal(&p->done);
    }
    pthread_mutex_unlock(&p->mu);
    return NULL;
}

or_pool* or_pool_new(int threads) {
    or_pool* p = (or_pool*)calloc(1, sizeof *p);
    p->workers = (threads < 1 ? 1 : threads) - 1;
    pthread_mutex_init(&p->mu, NULL);
    pthread_cond_init(&p->start, NULL);
    pthread_cond_init(&p->done, NULL);
    p->th = (pthread_t*)calloc(p->workers + 1, sizeof(pthread_t));
    for (int i = 0; i < p->workers; i++) pthread_create(&p->th[i], NULL, worker_main, p);
    return p;
}

void or_pool_free(or_pool* p) {
    if (!p) return;
    pthread_mutex_lock(&p->mu);
    p->shutdown = 1;
    pthread_cond_broadcast(&p->start);
    pthread_mutex_unlock(&p->mu);
    for (int i = 0; i < p->workers; i++) pthread_join(p->th[i], NULL);
    free(p->th);
    free(p);
}

static void pool_run(or_pool* p, size_t n_tasks, task_fn fn, void* ctx) {
    if (n_tasks == 0) return;
    if (p->workers == 0 || n_tasks == 1) {
        for (size_t i = 0; i < n_tasks; i++) fn(ctx, i);
        return;
    }
    pthread_mutex_lock(&p->mu);
    p->fn = fn;
    p->ctx = ctx;
    p->n_tasks = n_tasks;
    atomic_store(&p->next, 0);
    p->pending = p->workers;
    p->generation++;
    pthread_cond_broadcast(&p->start);
    pthread_mutex_unlock(&p->mu);
    run_tasks(p);
    pthread_mutex_lock(&p->mu);
    while (p->pending > 0) pthread_cond_wait(&p->done, &p->mu);
    pthread_mutex_unlock(&p->mu);
}

/* ---------------------------------------------------------------------------------------
 * matmul_rows: src/kernels.rs:123-203. ROW_BLOCK = 16 rows per task; for t > 1 the task
 * computes [rows][t] and the result is transposed into [t][rows]. The split never changes
 * a value: every output is one row's dot with one input.
 * ------------------------------------------------------------------------------------- */
#define ROW_BLOCK 16

typedef struct {
    or_fmt f;
    const uint8_t* w;
    size_t rows, cols, row_bytes, t;
    const float* x;
    float* out; /* t == 1: y[rows]; else tmp[rows][t] */
} mm_ctx;

static void mm_task(void* vctx, size_t task) {
    mm_ctx* c = (mm_ctx*)vctx;
    size_t r0 = task * ROW_BLOCK, r1 = r0 + ROW_BLOCK < c->rows ? r0 + ROW_BLOCK : c->rows;
    for (size_t r = r0; r < r1; r++) {
        const uint8_t* wr = c->w + r * c->row_bytes;
        if (c->t == 1) {
            c->out[r] = dot_fmt(c->f, wr, c->x, c->cols);
        } else {
            for (size_t tt = 0; tt < c->t; tt++) c->out[r * c->t + tt] = dot_fmt(c->f, wr, c->x + tt * c->cols, c->cols);
        }
    }
}

void or_matmul(or_pool* p, or_fmt f, const uint8_t* w, size_t rows, size_t cols, const float* x, size_t t, float* y) {
    mm_ctx c = {f, w, rows, cols, or_row_bytes(f, cols), t, x, NULL};
    size_t n_tasks = (rows + ROW_BLOCK - 1) / ROW_BLOCK;
    if (t == 1) {
        c.out = y;
        pool_run(p, n_tasks, mm_task, &c);
        return;
    }
    float* tmp = (float*)malloc(rows * t * sizeof(float));
    c.out = tmp;
    pool_run(p, n_tasks, mm_task, &c);
    for (size_t tt = 0; tt < t; tt++)
        for (size_t r = 0; r < rows; r++) y[tt * rows + r] = tmp[r * t + tt];
    free(tmp);
}

/* ---------------------------------------------------------------------------------------
 * Small kernels: src/kernels.rs:206-270
 * ------------------------------------------------------------------------------------- */
static void add_bias_bf16(float* y, const uint8_t* bias, size_t n, size_t t) {
    for (size_t r = 0; r < t; r++)
        for (size_t i = 0; i < n; i++) y[r * n + i] = y[r * n + i] + bf16_at(bias, i);
}

void or_rms_norm_bf16(const float* x, size_t len, const uint8_t* w, size_t n, float eps, float* out) {
    for (size_t r = 0; r < len / n; r++) {
        const float* xr = x + r * n;
        float* o = out + r * n;
        float ss = -0.0f;
        for (size_t i = 0; i < n; i++) ss = ss + xr[i] * xr[i];
        float mean_sq = ss / (float)n;
        float inv = 1.0f / sqrtf(mean_sq + eps);
        for (size_t i = 0; i < n; i++) o[i] = xr[i] * inv * bf16_at(w, i);
    }
}

void or_rms_norm_f32(const float* x, const float* w, size_t n, float eps, float* out) {
    float ss = -0.0f;
    for (size_t i = 0; i < n; i++) ss = ss + x[i] * x[i];
    float mean_sq = ss / (float)n;
    float inv = 1.0f / sqrtf(mean_sq + eps);
    for (size_t i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}

void or_rope_inplace(float* head, const float* inv_freq, size_t hd, size_t pos) {
    size_t half = hd / 2;
    for (size_t i = 0; i < half; i++) {
        float angle = (float)pos * inv_freq[i];
        float s = sinf(angle), c = cosf(angle);
        float a = head[i], b = head[i + half];
        head[i] = a * c - b * s;
        head[i + half] = b * c + a * s;
    }
}

void or_softmax_inplace(float* v, size_t n) {
    float max = -INFINITY;
    for (size_t i = 0; i < n; i++) max = fmaxf(max, v[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        v[i] = expf(v[i] - max);
        sum = sum + v[i];
    }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; i++) v[i] = v[i] * inv;
}

float or_silu(float x) { return x / (1.0f + expf(-x)); }

/* src/spec.rs:41-49 (same rule as Sampler greedy, src/model.rs:328-336): the first index
 * of the maximum. */
uint32_t or_argmax(const float* v, size_t n) {
    size_t best = 0;
    for (size_t i = 0; i < n; i++)
        if (v[i] > v[best]) best = i;
    return (uint32_t)best;
}

/* ---------------------------------------------------------------------------------------
 * Sampler: src/model.rs:300-366
 * ------------------------------------------------------------------------------------- */
/* Sampler::new (:309-311): top_k at least 1, state seed * 0x9E3779B97F4A7C15 | 1. */
void or_sampler_init(or_sampler* s, float temperature, size_t top_k, float top_p, uint64_t seed) {
    s->temperature = temperature;
    s->top_k = top_k < 1 ? 1 : top_k;
    s->top_p = top_p;
    s->state = (seed * 0x9E3779B97F4A7C15ull) | 1;
}

/* Sampler::next_uniform (:317-324): xorshift64*, (r >> 40) / 2^24 in f32. */
float or_sampler_uniform(or_sampler* s) {
    s->state ^= s->state >> 12;
    s->state ^= s->state << 25;
    s->state ^= s->state >> 27;
    uint64_t r = s->state * 0x2545F4914F6CDD1Dull;
    return (float)(uint32_t)(r >> 40) / (float)(1u << 24);
}

static const float* g_sort_logits;
/* descending logit; equal logits keep index order (the reference's selection leaves their order
 * unspecified) */
static int desc_logit(const void* a, const void* b) {
    uint32_t i = *(const uint32_t*)a, j = *(const uint32_t*)b;
    float x = g_sort_logits[i], y = g_sort_logits[j];
    if (x > y) return -1;
    if (x < y) return 1;
    return i < j ? -1 : (i > j ? 1 : 0);
}

/* Sampler::sample (:326-365). */
uint32_t or_sampler_sample(or_sampler* s, const float* logits, size_t n) {
    if (s->temperature <= 0.0f) return or_argmax(logits, n);
    size_t k = s->top_k < n ? s->top_k : n;
    uint32_t* idx = (uint32_t*)malloc(n * sizeof(uint32_t));
    float* probs = (float*)malloc(k * sizeof(float));
    for (size_t i = 0; i < n; i++) idx[i] = (uint32_t)i;
    g_sort_logits = logits;
    qsort(idx, n, sizeof(uint32_t), desc_logit);
    float max = logits[idx[0]];
    for (size_t i = 0; i < k; i++) probs[i] = expf((logits[idx[i]] - max) / s->temperature);
    float sum = 0.0f;
    for (size_t i = 0; i < k; i++) sum += probs[i];
    for (size_t i = 0; i < k; i++) probs[i] /= sum;
    /* nucleus cut */
    float cum = 0.0f;
    size_t keep = k;
    for (size_t i = 0; i < k; i++) {
        cum += probs[i];
        if (cum >= s->top_p) {
            keep = i + 1;
            break;
        }
    }
    float total = 0.0f;
    for (size_t i = 0; i < keep; i++) total += probs[i];
    float r = or_sampler_uniform(s) * total;
    uint32_t out = idx[keep - 1];
    for (size_t i = 0; i < keep; i++) {
        r -= probs[i];
        if (r <= 0.0f) {
            out = idx[i];
            break;
        }
    }
    free(idx);
    free(probs);
    return out;
}

/* ---------------------------------------------------------------------------------------
 * Quantizer: src/quant.rs:35-145, 158-251
 * ------------------------------------------------------------------------------------- */
static const float CLIPS[9] = {1.0f, 0.95f, 0.9f, 0.85f, 0.8f, 0.75f, 0.7f, 0.65f, 0.6f};

/* Rust f32::round: half away from zero (C roundf). f32::clamp(-qmax, qmax). */
static inline float qround(float v, float qmax) {
    float r = roundf(v);
    if (r < -qmax) r = -qmax;
    if (r > qmax) r = qmax;
    return r;
}

static float quantize_group(int bits, const float* w, size_t n, int clip_search, int8_t* q, double* err_out) {
    float qmax = bits == 8 ? 127.0f : 7.0f;
    float amax = 0.0f;
    for (size_t i = 0; i < n; i++) amax = fmaxf(amax, fabsf(w[i]));
    int finite = isfinite(amax);
    if (amax == 0.0f || !finite) {
        double e = -0.0;
        for (size_t i = 0; i < n; i++) e = e + (double)(w[i] * w[i]);
        memset(q, 0, n);
        *err_out = e;
        return 0.0f;
    }
    int n_clips = clip_search ? 9 : 1;
    double best_err = INFINITY;
    float best_s = 0.0f;
    for (int ci = 0; ci < n_clips; ci++) {
        float s = or_bf16_round(CLIPS[ci] * amax / qmax);
        if (s == 0.0f) continue;
        float inv = 1.0f / s;
        double err = 0.0;
        for (size_t i = 0; i < n; i++) {
            float d = w[i] - qround(w[i] * inv, qmax) * s;
            err = err + (double)(d * d);
        }
        if (err < best_err) {
            best_err = err;
            best_s = s;
        }
    }
    if (best_s == 0.0f) {
        double e = -0.0;
        for (size_t i = 0; i < n; i++) e = e + (double)(w[i] * w[i]);
        memset(q, 0, n);
        *err_out = e;
        return 0.0f;
    }
    float inv = 1.0f / best_s;
    for (size_t i = 0; i < n; i++) q[i] = (int8_t)qround(w[i] * inv, qmax);
    *err_out = best_err;
    return best_s;
}

void or_quantize_row(or_fmt f, const float* row, size_t cols, int clip_search, uint8_t* out, double* err,
                     double* norm) {
    size_t group = f.group;
    uint8_t* data = out;
    uint8_t* scales = out + cols * f.bits / 8;
    int8_t q[256];
    double e_sum = 0.0, n_sum = 0.0;
    for (size_t g = 0; g < cols / group; g++) {
        const float* wg = row + g * group;
        double e;
        float s = quantize_group(f.bits, wg, group, clip_search, q, &e);
        e_sum = e_sum + e;
        double nn = -0.0;
        for (size_t i = 0; i < group; i++) nn = nn + (double)(wg[i] * wg[i]);
        n_sum = n_sum + nn;
        uint32_t sb;
        memcpy(&sb, &s, 4);
        scales[2 * g] = (uint8_t)((sb >> 16) & 0xff);
        scales[2 * g + 1] = (uint8_t)(sb >> 24);
        if (f.bits == 8) {
            for (size_t j = 0; j < group; j++) data[g * group + j] = (uint8_t)q[j];
        } else {
            size_t half = group / 2;
            for (size_t j = 0; j < half; j++)
                data[g * half + j] = (uint8_t)((uint8_t)(q[j] + 8) | ((uint8_t)(q[j + half] + 8) << 4));
        }
    }
    if (err) *err = e_sum;
    if (norm) *norm = n_sum;
}

typedef struct {
    or_fmt f;
    const uint8_t* src;
    uint8_t* dst;
    size_t rows, cols;
    int clip;
} qm_ctx;

static void qm_task(void* vctx, size_t task) {
    qm_ctx* c = (qm_ctx*)vctx;
    size_t r0 = task * 8, r1 = r0 + 8 < c->rows ? r0 + 8 : c->rows;
    size_t rb_out = or_row_bytes(c->f, c->cols);
    float* fbuf = (float*)malloc(c->cols * sizeof(float));
    for (size_t r = r0; r < r1; r++) {
        for (size_t i = 0; i < c->cols; i++) fbuf[i] = bf16_at(c->src + r * c->cols * 2, i);
        or_quantize_row(c->f, fbuf, c->cols, c->clip, c->dst + r * rb_out, NULL, NULL);
    }
    free(fbuf);
}

static void quantize_matrix(or_pool* p, or_fmt f, const uint8_t* src, size_t rows, size_t cols, int clip,
                            uint8_t* dst) {
    qm_ctx c = {f, src, dst, rows, cols, clip};
    pool_run(p, (rows + 7) / 8, qm_task, &c);
}

/* JSON string escaping of Json::Str(..).to_text() (src/json.rs:84-99). */
static size_t json_escape(const char* s, char* out) {
    size_t o = 0;
    if (out) out[o] = '"';
    o++;
    for (const unsigned char* p = (const unsigned char*)s; *p; p++) {
        char buf[8];
        const char* rep = NULL;
        switch (*p) {
            case '"': rep = "\\\""; break;
            case '\\': rep = "\\\\"; break;
            case '\n': rep = "\\n"; break;
            case '\r': rep = "\\r"; break;
            case '\t': rep = "\\t"; break;
            default:
                if (*p < 0x20) {
                    snprintf(buf, sizeof buf, "\\u%04x", *p);
                    rep = buf;
                }
        }
        if (rep) {
            size_t l = strlen(rep);
            if (out) memcpy(out + o, rep, l);
            o += l;
        } else {
            if (out) out[o] = (char)*p;
            o++;
        }
    }
    if (out) out[o] = '"';
    return o + 1;
}

int or_quantize_model(const or_cfg* q, const char* qtext, const uint8_t* bf16_layers, const uint8_t* bf16_embed,
                      const uint8_t* norm_raw, int clip_search, int threads, uint8_t* out, size_t out_cap,
                      size_t* out_len) {
    or_cfg b = *q;
    b.format.bits = 16;
    b.embed_format.bits = 16;
    size_t src_r[24], dst_r[24];
    size_t src_total = or_layer_layout(&b, src_r);
    size_t dst_total = or_layer_layout(q, dst_r);
    size_t embed_bytes = (size_t)q->vocab * or_row_bytes(q->embed_format, q->hidden);
    size_t norm_bytes = (size_t)q->hidden * 2;
    /* Header (src/weights.rs:345-358). */
    size_t esc = json_escape(qtext, NULL);
    char* json = (char*)malloc(esc + 256);
    int n0 = snprintf(json, 64, "{\"format\":\"layerstream-quant-1\",\"config_json\":");
    json_escape(qtext, json + n0);
    size_t jl = n0 + esc;
    jl += snprintf(json + jl, 200, ",\"layer_bytes\":%zu,\"embed_bytes\":%zu,\"norm_bytes\":%zu}", dst_total,
                   embed_bytes, norm_bytes);
    size_t total = 8 + jl + (size_t)q->layers * dst_total + embed_bytes + norm_bytes;
    *out_len = total;
    if (!out) {
        free(json);
        return 0;
    }
    if (out_cap < total) {
        free(json);
        return fail("output buffer too small");
    }
    memcpy(out, "LSQ1", 4);
    uint32_t l32 = (uint32_t)jl;
    out[4] = l32 & 0xff;
    out[5] = (l32 >> 8) & 0xff;
    out[6] = (l32 >> 16) & 0xff;
    out[7] = (l32 >> 24) & 0xff;
    memcpy(out + 8, json, jl);
    free(json);
    uint8_t* w = out + 8 + jl;
    or_pool* p = or_pool_new(threads);
    for (int64_t l = 0; l < q->layers; l++) {
        const uint8_t* in = bf16_layers + (size_t)l * src_total;
        for (int s = 0; s < N_T; s++) {
            size_t rows, cols, vl;
            slot_shape(q, s, &rows, &cols, &vl);
            if (!rows)
                memcpy(w + dst_r[2 * s], in + src_r[2 * s], src_r[2 * s + 1]);
            else
                quantize_matrix(p, q->format, in + src_r[2 * s], rows, cols, clip_search, w + dst_r[2 * s]);
        }
        w += dst_total;
    }
    /* Embedding in batches of 4096 rows (src/quant.rs:227-241); batching never changes bytes. */
    quantize_matrix(p, q->embed_format, bf16_embed, q->vocab, q->hidden, clip_search, w);
    w += embed_bytes;
    memcpy(w, norm_raw, norm_bytes);
    or_pool_free(p);
    return 0;
}

/* ---------------------------------------------------------------------------------------
 * Model: src/model.rs:16-299
 * ------------------------------------------------------------------------------------- */
#define PREFILL_CHUNK 128
#define HEAD_ROWS 4096

struct or_model {
    or_cfg cfg;
    size_t ranges[24], total;
    const uint8_t* layers;
    const uint8_t* embed;
    float* final_norm;
    or_pool* pool;
    float** k_cache;
    float** v_cache;
    float* inv_freq;
    size_t max_ctx, pos;
};

or_model* or_model_new(const or_cfg* c, const uint8_t* layers, const uint8_t* embed, const uint8_t* norm_raw,
                       int threads, size_t max_ctx) {
    or_model* m = (or_model*)calloc(1, sizeof *m);
    m->cfg = *c;
    m->total = or_layer_layout(c, m->ranges);
    m->layers = layers;
    m->embed = embed;
    m->final_norm = (float*)malloc(c->hidden * sizeof(float));
    for (int64_t i = 0; i < c->hidden; i++) m->final_norm[i] = bf16_at(norm_raw, i);
    m->pool = or_pool_new(threads);
    size_t kv = c->kv_heads * c->head_dim;
    m->k_cache = (float**)calloc(c->layers, sizeof(float*));
    m->v_cache = (float**)calloc(c->layers, sizeof(float*));
    for (int64_t l = 0; l < c->layers; l++) {
        m->k_cache[l] = (float*)calloc(max_ctx * kv, sizeof(float));
        m->v_cache[l] = (float*)calloc(max_ctx * kv, sizeof(float));
    }
    size_t half = c->head_dim / 2;
    m->inv_freq = (float*)malloc(half * sizeof(float));
    for (size_t i = 0; i < half; i++)
        m->inv_freq[i] = (float)(1.0 / pow((double)c->rope_theta, (double)(2 * i) / (double)c->head_dim));
    m->max_ctx = max_ctx;
    m->pos = 0;
    return m;
}

void or_model_free(or_model* m) {
    if (!m) return;
    for (int64_t l = 0; l < m->cfg.layers; l++) {
        free(m->k_cache[l]);
        free(m->v_cache[l]);
    }
    free(m->k_cache);
    free(m->v_cache);
    free(m->inv_freq);
    free(m->final_norm);
    or_pool_free(m->pool);
    free(m);
}

size_t or_model_pos(const or_model* m) { return m->pos; }
size_t or_model_max_ctx(const or_model* m) { return m->max_ctx; }
void or_model_reset(or_model* m) { m->pos = 0; }

int or_model_truncate(or_model* m, size_t pos) {
    if (pos > m->pos) return fail("cannot truncate beyond the cached tokens");
    m->pos = pos;
    return 0;
}

static int check_request(const or_model* m, const uint32_t* tok, size_t n) {
    if (n == 0) return fail("no tokens to process");
    if (m->pos + n > m->max_ctx) return fail("context is full");
    for (size_t i = 0; i < n; i++)
        if ((int64_t)tok[i] >= m->cfg.vocab) return fail("token id is outside the vocabulary");
    return 0;
}

static const uint8_t* slot(const or_model* m, size_t l, int s) {
    return m->layers + l * m->total + m->ranges[2 * s];
}

/* layer_forward: src/model.rs:224-299 */
static void layer_forward(or_model* m, size_t l, float* x, size_t t, size_t pos0, float* h_buf, float* q, float* k,
                          float* v, float* attn, float* proj, float* gate, float* up, float* scores) {
    const or_cfg* c = &m->cfg;
    size_t h = c->hidden, kvd = c->kv_heads * c->head_dim, hd = c->head_dim, inter = c->inter;
    size_t group = c->heads / c->kv_heads;
    or_fmt f = c->format;
    float* kc = m->k_cache[l];
    float* vc = m->v_cache[l];

    or_rms_norm_bf16(x, t * h, slot(m, l, T_INPUT_NORM), h, c->eps, h_buf);
    or_matmul(m->pool, f, slot(m, l, T_Q_W), h, h, h_buf, t, q);
    add_bias_bf16(q, slot(m, l, T_Q_B), h, t);
    or_matmul(m->pool, f, slot(m, l, T_K_W), kvd, h, h_buf, t, k);
    add_bias_bf16(k, slot(m, l, T_K_B), kvd, t);
    or_matmul(m->pool, f, slot(m, l, T_V_W), kvd, h, h_buf, t, v);
    add_bias_bf16(v, slot(m, l, T_V_B), kvd, t);

    for (size_t i = 0; i < t; i++) {
        size_t pos = pos0 + i;
        for (int64_t hh = 0; hh < c->heads; hh++) or_rope_inplace(q + i * h + hh * hd, m->inv_freq, hd, pos);
        for (int64_t g = 0; g < c->kv_heads; g++) or_rope_inplace(k + i * kvd + g * hd, m->inv_freq, hd, pos);
        memcpy(kc + pos * kvd, k + i * kvd, kvd * sizeof(float));
        memcpy(vc + pos * kvd, v + i * kvd, kvd * sizeof(float));
    }

    float scale = 1.0f / sqrtf((float)hd);
    for (size_t i = 0; i < t; i++) {
        size_t ctx = pos0 + i + 1;
        for (int64_t hh = 0; hh < c->heads; hh++) {
            size_t g = hh / group;
            const float* qh = q + i * h + hh * hd;
            for (size_t j = 0; j < ctx; j++) {
                const float* kj = kc + j * kvd + g * hd;
                float s = -0.0f;
                for (size_t d = 0; d < hd; d++) s = s + qh[d] * kj[d];
                scores[j] = s * scale;
            }
            or_softmax_inplace(scores, ctx);
            float* out = attn + i * h + hh * hd;
            for (size_t d = 0; d < hd; d++) out[d] = 0.0f;
            for (size_t j = 0; j < ctx; j++) {
                const float* vj = vc + j * kvd + g * hd;
                float p = scores[j];
                for (size_t d = 0; d < hd; d++) out[d] = out[d] + p * vj[d];
            }
        }
    }
    or_matmul(m->pool, f, slot(m, l, T_O_W), h, h, attn, t, proj);
    for (size_t i = 0; i < t * h; i++) x[i] = x[i] + proj[i];

    or_rms_norm_bf16(x, t * h, slot(m, l, T_POST_NORM), h, c->eps, h_buf);
    or_matmul(m->pool, f, slot(m, l, T_GATE), inter, h, h_buf, t, gate);
    or_matmul(m->pool, f, slot(m, l, T_UP), inter, h, h_buf, t, up);
    for (size_t i = 0; i < t * inter; i++) gate[i] = or_silu(gate[i]) * up[i];
    or_matmul(m->pool, f, slot(m, l, T_DOWN), h, inter, gate, t, proj);
    for (size_t i = 0; i < t * h; i++) x[i] = x[i] + proj[i];
}

/* forward_chunk: src/model.rs:161-220. logits: n_logits * vocab (may be NULL). */
static int forward_chunk(or_model* m, const uint32_t* tok, size_t t, size_t n_logits, float* logits) {
    const or_cfg* c = &m->cfg;
    size_t h = c->hidden, kv = c->kv_heads * c->head_dim, inter = c->inter;
    size_t rb = or_row_bytes(c->embed_format, h);
    float* x = (float*)malloc(t * h * sizeof(float));
    for (size_t i = 0; i < t; i++) or_dequant_row(c->embed_format, m->embed + (size_t)tok[i] * rb, x + i * h, h);
    float* buf = (float*)malloc((t * (4 * h + 2 * kv + 2 * inter) + m->max_ctx) * sizeof(float));
    float *hb = buf, *q = hb + t * h, *k = q + t * h, *v = k + t * kv, *attn = v + t * kv, *proj = attn + t * h,
          *gate = proj + t * h, *up = gate + t * inter, *scores = up + t * inter;
    for (int64_t l = 0; l < c->layers; l++) layer_forward(m, l, x, t, m->pos, hb, q, k, v, attn, proj, gate, up, scores);
    if (n_logits > 0 && logits) {
        size_t n = n_logits, vocab = c->vocab;
        float* hf = (float*)malloc(n * h * sizeof(float));
        for (size_t j = 0; j < n; j++) or_rms_norm_f32(x + (t - n + j) * h, m->final_norm, h, c->eps, hf + j * h);
        float* tmp = (float*)malloc(n * HEAD_ROWS * sizeof(float));
        for (size_t first = 0; first < vocab; first += HEAD_ROWS) {
            size_t rows = vocab - first < HEAD_ROWS ? vocab - first : HEAD_ROWS;
            or_matmul(m->pool, c->embed_format, m->embed + first * rb, rows, h, hf, n, tmp);
            for (size_t j = 0; j < n; j++) memcpy(logits + j * vocab + first, tmp + j * rows, rows * sizeof(float));
        }
        free(tmp);
        free(hf);
    }
    free(buf);
    free(x);
    m->pos += t;
    return 0;
}

int or_model_forward(or_model* m, const uint32_t* tok, size_t n, float* logits) {
    if (check_request(m, tok, n)) return -1;
    size_t n_chunks = (n + PREFILL_CHUNK - 1) / PREFILL_CHUNK;
    for (size_t ci = 0; ci < n_chunks; ci++) {
        size_t a = ci * PREFILL_CHUNK, len = n - a < PREFILL_CHUNK ? n - a : PREFILL_CHUNK;
        int last = ci + 1 == n_chunks;
        forward_chunk(m, tok + a, len, last ? 1 : 0, last ? logits : NULL);
    }
    return 0;
}

int or_model_forward_multi(or_model* m, const uint32_t* tok, size_t n, size_t n_logits, float* logits) {
    if (check_request(m, tok, n)) return -1;
    if (n_logits == 0 || n_logits > n) return fail("asked for logits at more positions than tokens");
    if (n > PREFILL_CHUNK) return fail("forward_multi takes at most 128 tokens at a time");
    return forward_chunk(m, tok, n, n_logits, logits);
}

/* ---------------------------------------------------------------------------------------
 * Drafts and speculative decoding: src/spec.rs:52-152
 * ------------------------------------------------------------------------------------- */
/* SplitMix64 finalizer (Steele, Lea, Flood 2014). */
static inline uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint32_t or_scripted_draft(const or_drafter* d, size_t idx) {
    uint64_t h1 = mix64(d->seed ^ mix64((uint64_t)idx));
    uint64_t h2 = mix64(h1);
    double u = (double)(h1 >> 11) * (1.0 / 9007199254740992.0);
    if (idx < d->n_greedy) {
        uint32_t g = d->greedy[idx];
        if (u < d->p_accept) return g;
        uint64_t r = h2 % (d->vocab - 1);
        return (uint32_t)(r >= g ? r + 1 : r);
    }
    return (uint32_t)(h2 % d->vocab);
}

#define MAX_DRAFT 32

static int contains(const uint32_t* v, size_t n, uint32_t x) {
    for (size_t i = 0; i < n; i++)
        if (v[i] == x) return 1;
    return 0;
}

int or_speculative_greedy(or_model* target, or_drafter* dr, const uint32_t* prompt, size_t n_prompt, size_t max_new,
                          size_t k, const uint32_t* eos, size_t n_eos, uint32_t* out, size_t* out_len,
                          or_spec_stats* st) {
    or_model* draft = dr->model;
    memset(st, 0, sizeof *st);
    *out_len = 0;
    if (k == 0 || k > MAX_DRAFT) return fail("k must be between 1 and 32");
    if (n_prompt == 0 || max_new == 0) return fail("need a prompt and at least one token to generate");
    if (target->pos != 0 || (draft && draft->pos != 0)) return fail("both models must start with an empty cache");
    if (draft && target->cfg.vocab != draft->cfg.vocab) return fail("the draft and the target must share a vocabulary");
    size_t need = n_prompt + max_new + k;
    if (need > target->max_ctx || (draft && need > draft->max_ctx)) return fail("prompt + max_new + k exceed the context limit");
    size_t vocab = target->cfg.vocab;
    float* logits = (float*)malloc((k + 1) * vocab * sizeof(float));
    float* dlog = draft ? (float*)malloc(draft->cfg.vocab * sizeof(float)) : NULL;
    size_t len = 0;

    double t0 = now_s();
    if (or_model_forward(target, prompt, n_prompt, logits)) goto err;
    if (draft && or_model_forward(draft, prompt, n_prompt, dlog)) goto err;
    st->first_secs = now_s() - t0;

    uint32_t a = or_argmax(logits, vocab);
    out[len++] = a;
    int stop = contains(eos, n_eos, a);
    double t_dec = now_s();
    uint32_t drafts[MAX_DRAFT], block[MAX_DRAFT + 1];
    while (!stop && len < max_new) {
        size_t kk = k < max_new - len - 1 ? k : max_new - len - 1;
        double ts = now_s();
        uint32_t cur = a;
        for (size_t i = 0; i < kk; i++) {
            uint32_t d;
            if (draft) {
                if (or_model_forward(draft, &cur, 1, dlog)) goto err;
                d = or_argmax(dlog, draft->cfg.vocab);
                st->draft_forwards++;
            } else {
                d = or_scripted_draft(dr, len + i);
            }
            drafts[i] = d;
            cur = d;
        }
        st->draft_secs += now_s() - ts;
        block[0] = a;
        memcpy(block + 1, drafts, kk * sizeof(uint32_t));
        size_t p = target->pos;
        ts = now_s();
        if (or_model_forward_multi(target, block, kk + 1, kk + 1, logits)) goto err;
        st->target_secs += now_s() - ts;
        st->target_passes++;
        size_t mm = 0;
        while (mm < kk && or_argmax(logits + mm * vocab, vocab) == drafts[mm]) mm++;
        uint32_t next = or_argmax(logits + mm * vocab, vocab);
        st->drafted += kk;
        st->accepted += mm;
        for (size_t i = 0; i <= mm; i++) {
            uint32_t tok = i < mm ? drafts[i] : next;
            out[len++] = tok;
            if (contains(eos, n_eos, tok) || len == max_new) {
                stop = 1;
                break;
            }
        }
        size_t want = p + mm + 1;
        or_model_truncate(target, want);
        if (draft) {
            if (draft->pos > want) {
                or_model_truncate(draft, want);
            } else if (draft->pos < want) {
                ts = now_s();
                if (or_model_forward(draft, block + (draft->pos - p), mm + 1 - (draft->pos - p), dlog)) goto err;
                st->draft_forwards++;
                st->draft_secs += now_s() - ts;
            }
        }
        a = next;
    }
    st->decode_secs = now_s() - t_dec;
    *out_len = len;
    free(logits);
    free(dlog);
    return 0;
err:
    *out_len = len;
    free(logits);
    free(dlog);
    return -1;
}

int or_plain_greedy(or_model* m, const uint32_t* prompt, size_t n_prompt, size_t max_new, const uint32_t* eos,
                    size_t n_eos, uint32_t* out, size_t* out_len) {
    size_t vocab = m->cfg.vocab;
    float* logits = (float*)malloc(vocab * sizeof(float));
    *out_len = 0;
    if (or_model_forward(m, prompt, n_prompt, logits)) {
        free(logits);
        return -1;
    }
    for (size_t i = 0; i < max_new; i++) {
        uint32_t t = or_argmax(logits, vocab);
        out[(*out_len)++] = t;
        if (contains(eos, n_eos, t) || i + 1 == max_new) break;
        if (or_model_forward(m, &t, 1, logits)) {
            free(logits);
            return -1;
        }
    }
    free(logits);
    return 0;
}
