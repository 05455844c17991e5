/*
 * Oracle: a plain-C restatement of the reference's CPU path for the speculative
 * verify step. TEST INFRASTRUCTURE ONLY: tests, the smoke check and the CPU
 * baseline leg of the benchmark may call it, as the checker. The product
 * (layerstream_amd) never links or calls it.
 *
 * Every function follows the reference file:line named in its comment, in the
 * same floating-point operation order, compiled with -ffp-contract=off and no
 * fast-math, calling glibc expf/sinf/cosf/sqrtf/pow like Rust std does on Linux.
 */
#ifndef LS_ORACLE_H
#define LS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* WeightFormat (src/weights.rs:14-21): bits 16 = Bf16, 8/4 = Quant{bits, group}. */
typedef struct {
    int32_t bits;
    int32_t group;
} or_fmt;

/* Config (src/weights.rs:57-74). */
typedef struct {
    or_fmt format;
    or_fmt embed_format;
    int64_t hidden, inter, layers, heads, kv_heads, head_dim, vocab;
    float eps, rope_theta;
} or_cfg;

/* ---- formats / quant helpers ---- */
size_t or_row_bytes(or_fmt f, size_t cols);                 /* src/weights.rs:26-31 */
int or_validate(or_fmt f, const size_t* cols, size_t n);    /* src/weights.rs:34-47 */
size_t or_layer_layout(const or_cfg* c, size_t* ranges24);  /* src/weights.rs:215-227; returns total */
float or_bf16_round(float v);                               /* src/quant.rs:26-33 */
void or_quantize_row(or_fmt f, const float* row, size_t cols, int clip_search, uint8_t* out,
                     double* err, double* norm);            /* src/quant.rs:79-104 */
/* quantize_model (src/quant.rs:158-251) over in-memory parts; writes the .lsq image to out.
 * qcfg carries the quantized formats, qconfig_text the config text with layerstream_quant
 * (src/quant.rs:137-145). With out == NULL only *out_len (the image size) is set. */
int or_quantize_model(const or_cfg* qcfg, const char* qconfig_text, const uint8_t* bf16_layers,
                      const uint8_t* bf16_embed, const uint8_t* norm_raw, int clip_search, int threads,
                      uint8_t* out, size_t out_cap, size_t* out_len);

/* ---- kernels (src/kernels.rs) ---- */
float or_dot_bf16(const uint8_t* w, const float* x, size_t n);              /* :27-43 */
float or_dot_q8(const uint8_t* row, const float* x, size_t cols, size_t g); /* :53-68 */
float or_dot_q4(const uint8_t* row, const float* x, size_t cols, size_t g); /* :74-92 */
void or_dequant_row(or_fmt f, const uint8_t* raw, float* out, size_t cols); /* :95-121 */
void or_rms_norm_bf16(const float* x, size_t len, const uint8_t* w, size_t n, float eps, float* out); /* :217-228 */
void or_rms_norm_f32(const float* x, const float* w, size_t n, float eps, float* out);                /* :231-238 */
void or_rope_inplace(float* head, const float* inv_freq, size_t hd, size_t pos);                       /* :242-252 */
void or_softmax_inplace(float* v, size_t n);                                                            /* :254-265 */
float or_silu(float x);                                                                                 /* :268-270 */
uint32_t or_argmax(const float* v, size_t n);                                                           /* src/spec.rs:41-49 */
/* Sampler (src/model.rs:300-366). */
typedef struct {
    float temperature;
    size_t top_k;
    float top_p;
    uint64_t state;
} or_sampler;
void or_sampler_init(or_sampler* s, float temperature, size_t top_k, float top_p, uint64_t seed);
float or_sampler_uniform(or_sampler* s);
uint32_t or_sampler_sample(or_sampler* s, const float* logits, size_t n);

/* ---- pool (src/pool.rs) and matmul (src/kernels.rs:123-203) ---- */
typedef struct or_pool or_pool;
or_pool* or_pool_new(int threads);
void or_pool_free(or_pool* p);
void or_matmul(or_pool* p, or_fmt f, const uint8_t* w, size_t rows, size_t cols, const float* x, size_t t,
               float* y);

/* ---- model (src/model.rs) ---- */
typedef struct or_model or_model;
/* layers: cfg.layers consecutive layer blocks (layout of or_layer_layout); embed: vocab rows in
 * embed_format; norm_raw: hidden bf16 values. The buffers are borrowed for the model's life. */
or_model* or_model_new(const or_cfg* c, const uint8_t* layers, const uint8_t* embed, const uint8_t* norm_raw,
                       int threads, size_t max_ctx);
void or_model_free(or_model* m);
size_t or_model_pos(const or_model* m);
size_t or_model_max_ctx(const or_model* m);
void or_model_reset(or_model* m);
int or_model_truncate(or_model* m, size_t pos);
/* logits: vocab floats (may be NULL). */
int or_model_forward(or_model* m, const uint32_t* tok, size_t n, float* logits);
/* logits: n_logits * vocab floats. */
int or_model_forward_multi(or_model* m, const uint32_t* tok, size_t n, size_t n_logits, float* logits);
const char* or_last_error(void);

/* ---- speculative decoding (src/spec.rs:57-152) ---- */
typedef struct {
    uint64_t target_passes, drafted, accepted, draft_forwards;
    double target_secs, draft_secs, first_secs, decode_secs;
} or_spec_stats;

/* Draft source: either a draft model (as the reference) or a scripted generator that proposes
 * the known greedy continuation g with probability p_accept per position. */
typedef struct {
    or_model* model;         /* non-NULL: draft model, the reference's behaviour */
    const uint32_t* greedy;  /* scripted: g[0..n_greedy) = the target's greedy output tokens */
    size_t n_greedy;
    double p_accept;
    uint64_t seed;
    uint64_t vocab;
} or_drafter;

/* Scripted proposal for output index `idx` (the token that would become out[idx]). */
uint32_t or_scripted_draft(const or_drafter* d, size_t idx);

int or_speculative_greedy(or_model* target, or_drafter* draft, const uint32_t* prompt, size_t n_prompt,
                          size_t max_new, size_t k, const uint32_t* eos, size_t n_eos, uint32_t* out,
                          size_t* out_len, or_spec_stats* stats);
/* Plain greedy (tests/spec.rs:44-57 with Sampler::greedy, src/model.rs:328-336). */
int or_plain_greedy(or_model* m, const uint32_t* prompt, size_t n_prompt, size_t max_new, const uint32_t* eos,
                    size_t n_eos, uint32_t* out, size_t* out_len);

#ifdef __cplusplus
}
#endif
#endif
