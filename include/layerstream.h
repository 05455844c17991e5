/*
 * layerstream_amd: MI355X (gfx950) speculative-decoding verify engine for Qwen2-architecture
 * models with tied embeddings, behind a C ABI.
 *
 * The reference (themaker00001/layerstream) is a Rust crate with no FFI; each entry point
 * below names the reference interface it replaces (file:line in that crate), with the same
 * argument meaning and error behaviour: bad requests return an error code and set a
 * thread-local message (ls_last_error), they never abort.
 *
 * Conventions: every function returns 0 on success and a negative LS_E* code on error unless
 * its comment says otherwise. Handles are not thread-safe (one caller thread per model, as the
 * reference's `&mut self`). Output buffers are caller-owned; no pointer is retained across
 * calls except where stated (a memory source borrows its buffers for its whole life).
 */
#ifndef LAYERSTREAM_H
#define LAYERSTREAM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LS_OK 0
#define LS_E_INVALID (-1) /* bad request or argument (the reference's Err(String)) */
#define LS_E_FORMAT (-2)  /* malformed config, header or file */
#define LS_E_IO (-3)      /* file read failure */
#define LS_E_DEVICE (-4)  /* HIP runtime failure */
#define LS_E_STATE (-5)   /* call out of order (provider schedule, model in use) */

/* Last error message of this thread (empty if none). Valid until the next call. */
const char* ls_last_error(void);
/* Library version string. */
const char* ls_version(void);

/* ---------------------------------------------------------------------------------------
 * Formats. WeightFormat (src/weights.rs:14-55): bits 16 = bf16; 8 or 4 = symmetric integers
 * with one bf16 scale per `group` weights, the scales after the packed integers of each row.
 * ------------------------------------------------------------------------------------- */
typedef struct {
    int32_t bits;  /* 16, 8 or 4 */
    int32_t group; /* 0 for bf16; 16..256, a multiple of 16 */
} ls_format;

/* Config (src/weights.rs:57-156). */
typedef struct {
    ls_format format;       /* the seven layer matrices */
    ls_format embed_format; /* the tied embedding table / output head */
    int64_t hidden, inter, layers, heads, kv_heads, head_dim, vocab, max_pos;
    float eps, rope_theta;
} ls_config;

/* WeightFormat::row_bytes (src/weights.rs:26-31). Returns the byte count. */
size_t ls_row_bytes(ls_format f, size_t cols);
/* WeightFormat::validate (src/weights.rs:34-47). */
int ls_format_validate(ls_format f, const size_t* cols, size_t n_cols);
/* Config::from_json (src/weights.rs:77-141), including the layerstream_quant key. */
int ls_config_from_json(const char* config_json, ls_config* out);
/* layer_layout_for (src/weights.rs:215-227): 12 (offset, length) pairs in slot order
 * input_norm, down, gate, up, post_norm, k_b, k_w, o_w, q_b, q_w, v_b, v_w. Returns the block
 * size in bytes (0 on error). */
size_t ls_layer_layout(const ls_config* cfg, size_t ranges[24]);
/* inject_quant (src/quant.rs:137-145). Writes NUL-terminated text to out (cap bytes);
 * *out_len = length without the NUL. embed_bits == 0 shares the layers' format. */
int ls_inject_quant(const char* config_json, int bits, int group, int embed_bits, int embed_group, char* out,
                    size_t cap, size_t* out_len);

/* ---------------------------------------------------------------------------------------
 * Quantizer: quantize_row (src/quant.rs:79-104) and quantize_model (src/quant.rs:158-251).
 * ------------------------------------------------------------------------------------- */
/* One row: out receives ls_row_bytes(f, cols) bytes. err/norm may be NULL. */
int ls_quantize_row(ls_format f, const float* row, size_t cols, int clip_search, uint8_t* out, double* err,
                    double* norm);
/* A whole in-memory bf16 model into a `.lsq` image (src/weights.rs:327-358 layout): header,
 * layer blocks, embedding table, final norm. bf16_config_json is the model's config.json text.
 * With out == NULL only *out_len is set. threads <= 0 uses every core. rel_rmse may be NULL. */
int ls_quantize_model(const char* bf16_config_json, const uint8_t* bf16_layers, const uint8_t* bf16_embed,
                      const uint8_t* final_norm_bf16, ls_format fmt, ls_format embed_fmt, int clip_search,
                      int threads, uint8_t* out, size_t out_cap, size_t* out_len, double* rel_rmse);

/* Synthetic Qwen2 weights for benchmarks and tests (no reference counterpart: the reference
 * reads real checkpoints). SplitMix64(seed) counter stream -> Box-Muller N(0, std) -> bf16
 * round-to-nearest-even for every matrix and the q/k/v biases; RMSNorm weights are
 * 1 + N(0, std). Layer blocks in slot order. Sizes: layers = cfg.layers * block bytes,
 * embed = vocab * hidden * 2, norm = hidden * 2. cfg must be bf16. */
int ls_synth_bf16_model(const ls_config* cfg, uint64_t seed, float std_dev, uint8_t* layers, uint8_t* embed,
                        uint8_t* final_norm, int threads);

/* ---------------------------------------------------------------------------------------
 * Sources: trait Source (src/source.rs:23-33).
 * ------------------------------------------------------------------------------------- */
typedef struct ls_source ls_source;

/* Borrowed in-memory model parts (the caller keeps them alive until ls_source_free):
 * cfg.layers consecutive layer blocks, the embedding table, the bf16 final norm. */
int ls_source_from_memory(const char* config_json, const uint8_t* layers, size_t layers_len,
                          const uint8_t* embed, size_t embed_len, const uint8_t* final_norm_bf16,
                          size_t norm_len, ls_source** out);
/* ModelFiles::open_quantized + FileSource (src/weights.rs:389-424, src/source.rs:90-182):
 * a `.lsq` file read with positioned reads. */
int ls_source_open_lsq(const char* path, ls_source** out);
/* A `.lsq` image already in memory (borrowed), with the same checks as the file. */
int ls_source_from_lsq_image(const uint8_t* image, size_t len, ls_source** out);
/* A copy of src's layers and embedding table in pinned host memory (hipHostMalloc), for the
 * streaming mode's direct host -> device DMA ("pinned host buffers"). src may be freed after. */
int ls_source_pinned_copy(const ls_source* src, ls_source** out);
void ls_source_free(ls_source* s);
int ls_source_config(const ls_source* s, ls_config* out);
/* IoStats::bytes_read (src/source.rs:13-21). */
uint64_t ls_source_bytes_read(const ls_source* s);

/* ---------------------------------------------------------------------------------------
 * Model (src/model.rs:16-140) on one MI355X. The provider decides where weights live
 * (src/provider.rs:39-55): RESIDENT keeps every layer in HBM (ResidentProvider :61-137);
 * STREAM keeps `slots` device layer slots fed from pinned host staging buffers by
 * hipMemcpyAsync on a side stream, in the fixed schedule order layer 0..L-1 then the head
 * chunks (StreamProvider :161-352).
 * ------------------------------------------------------------------------------------- */
typedef struct ls_model ls_model;

#define LS_MODE_RESIDENT 0
#define LS_MODE_STREAM 1

/* Model::new (src/model.rs:58-77). The source must outlive the model. device = HIP device
 * ordinal. */
int ls_model_create(ls_source* src, int mode, int slots, size_t max_ctx, int device, ls_model** out);
void ls_model_free(ls_model* m);
/* Model::{pos, max_ctx, reset} (src/model.rs:84-103). */
size_t ls_model_pos(const ls_model* m);
size_t ls_model_max_ctx(const ls_model* m);
void ls_model_reset(ls_model* m);
/* Model::truncate (src/model.rs:137-140): forget cached tokens after pos. The reference asserts
 * pos <= cached; here that is LS_E_INVALID. O(1): rejected K/V rows are overwritten later. */
int ls_model_truncate(ls_model* m, size_t pos);
/* Model::forward (src/model.rs:111-119): push tokens in 128-token chunks and return the
 * logits of the last one. logits (vocab floats) and argmax may each be NULL. */
int ls_model_forward(ls_model* m, const uint32_t* tokens, size_t n, float* logits, uint32_t* argmax);
/* Model::forward_multi (src/model.rs:124-133): one weight pass over n <= 128 tokens, logits at
 * the last n_logits positions (n_logits * vocab floats, may be NULL) and their argmax (first
 * index of the maximum, src/spec.rs:41-49; may be NULL). */
int ls_model_forward_multi(ls_model* m, const uint32_t* tokens, size_t n, size_t n_logits, float* logits,
                           uint32_t* argmax);
/* One greedy verify step of speculative decoding, fused on the device: forward_multi over
 * block[0..n) with n = kk + 1 (block = [a, d_1 .. d_kk]), the per-position argmax, the
 * longest-prefix acceptance of src/spec.rs:119-127 and the rollback truncate(p + m + 1) of
 * src/spec.rs:137-139. Only *accepted (m) and *next (the correction or bonus token) return
 * to the host. */
int ls_model_verify_greedy(ls_model* m, const uint32_t* block, size_t n, uint32_t* accepted, uint32_t* next);
/* A draft model's proposals (src/spec.rs:100-107: kk single-token forwards, each fed the argmax
 * of the one before): out[i] is the argmax after consuming first, out[0] .. out[i - 1], and the
 * model advances by k positions, exactly as k calls of ls_model_forward with argmax. Over resident
 * weights the k passes run chained on the device with one host wait (LS_E_STATE otherwise);
 * 1 <= k <= 32. The reference has no such call: its draft loop sits inside speculative_greedy;
 * here the model drafter (ls_drafter_from_model) runs that loop through this call. */
int ls_model_draft_chain(ls_model* m, uint32_t first, size_t k, uint32_t* out);

/* Several independent sequences over one copy of the weights. The reference has one KV cache
 * per Model (src/model.rs:16-26, 67-68); this model holds n_seq of them (each max_ctx tokens)
 * and its own position per sequence. Every call above acts on the selected sequence (0 at
 * creation). ls_model_create(...) is ls_model_create_batch(..., 1, ...). */
int ls_model_create_batch(ls_source* src, int mode, int slots, size_t max_ctx, int device, int n_seq, ls_model** out);
int ls_model_n_seq(const ls_model* m);
int ls_model_select(ls_model* m, int seq);
/* One verify pass over a block for every sequence (blocks concatenated in sequence order, lens[s]
 * tokens for sequence s, each 1..33): the weights are read once for all of them. accepted[s] and
 * next[s] are what ls_model_verify_greedy would return for that sequence alone, bit for bit, and
 * each sequence is truncated to p_s + accepted[s] + 1 (src/spec.rs:116-139 per sequence). */
int ls_model_verify_greedy_batch(ls_model* m, const uint32_t* blocks, const size_t* lens, int n_seq, uint32_t* accepted,
                                 uint32_t* next);

/* Provider report (src/provider.rs:29-37). */
typedef struct {
    uint64_t resident_weight_bytes; /* device bytes held for weights */
    uint64_t bytes_read;            /* source bytes read so far */
    uint64_t wait_ns;               /* host time blocked waiting for streamed weights */
    uint64_t h2d_bytes;             /* bytes copied host -> device for streamed weights */
} ls_report;
int ls_model_report(const ls_model* m, ls_report* out);
/* Time of the last verify step in ms: host clock from its launch until its result is on the host
 * (LS_STEP_EVENTS=1 in the environment: HIP events around its launch on the device instead). */
double ls_model_last_step_ms(const ls_model* m);

/* Profiling of the weight-streaming matvec kernels: with enable != 0, HIP events bracket each
 * launch on the model's compute stream; ls_model_profile_read returns the launches, their summed
 * device time and their algorithmic bytes (weights in the stored format + f32 inputs + f32
 * outputs) since the last read, then resets. enable = 1 takes every matrix launch; enable = 2 only
 * each pass's dominant launch: the layer stack when a pass runs every layer in one launch (the
 * head is left out), else every matrix launch. */
typedef struct {
    uint64_t launches;
    double ms;
    double bytes;
    double flops;
} ls_kernel_stat;
int ls_model_profile(ls_model* m, int enable);
int ls_model_profile_read(ls_model* m, ls_kernel_stat* out);

/* Graph replay of the verify step (no counterpart in the reference, whose forward pass is a
 * CPU loop): with enable != 0 (the default) a resident model captures ls_model_verify_greedy
 * for each block length once into a HIP graph and replays it, so a step costs one launch on
 * the host. Results are bit-identical either way; profiling and streamed weights always run
 * the step launch by launch. */
int ls_model_use_graphs(ls_model* m, int enable);

/* Test hook for the error path of the in-launch waits (no counterpart in the reference). The next
 * device pass of this model (forward, forward_multi, verify_greedy or a batched verify) starts
 * with the control block's error word set, as if a bounded wait had given up: every wait of the
 * pass stops waiting at once, every kernel still runs to its end, and the call returns
 * LS_E_DEVICE with the positions unchanged. The control block is cleared afterwards, so the
 * following call runs normally. */
int ls_model_debug_fail_next(ls_model* m);

/* Measurement hook (no counterpart in the reference): with LS_PASS=1 and LS_PASS_TIMELINE=1 in the
 * environment when the model was created, every unit of the persistent layer pass records device
 * timestamps (100 MHz s_memrealtime) per (workgroup, layer, stage): word 0 start, 1 + w wavefront
 * w's input ready, 9 1/rms known, 10 products summed, 11 stores issued, 12 done, 13 producers'
 * flags seen, 14 and 15 stale re-fetch counts, 16 + w wavefront w's products done, 24 the flag's
 * store acknowledged (a timeline makes each unit wait for it). Copies up to cap words of the last
 * pass's stamps to out (NULL: none) and returns the number of words, [workgroup][layer][5
 * stages][32]; 0 when there is no timeline. Without the persistent pass, LS_STACK_TIMELINE=1 makes
 * every workgroup of the layer-stack launch record [workgroup][8] stamps: 0 entry, 1 input there
 * (after its wait; 0 when it has none), 2 done, and for the matrix roles 3 inputs loaded, 4 products
 * issued, 5 row-group sums done, 6 epilogue stores issued, 7 layer << 8 | role (0 q|k|v,
 * 1 attention, 2 o, 3 gate|up, 4 down); workgroups in launch order. Built for int8 weights at
 * head_dim 64 and 128 (the 0.5B and 3B shapes); other models refuse the timeline. */
size_t ls_model_debug_timeline(ls_model* m, uint64_t* out, size_t cap);
/* Debugging hook: a copy of one of the model's device buffers by name ("x", "xf", "ss", "q",
 * "af", "actf", "kcache", "vcache", "pass_area"), up to cap bytes (out may be NULL). Returns the
 * buffer's size in bytes, 0 on error. */
size_t ls_model_debug_read(ls_model* m, const char* name, void* out, size_t cap);

/* ---------------------------------------------------------------------------------------
 * Speculative decoding: speculative_greedy (src/spec.rs:57-152).
 * ------------------------------------------------------------------------------------- */
typedef struct {
    uint64_t target_passes, drafted, accepted, draft_forwards;
    double target_secs, draft_secs, first_secs, decode_secs;
} ls_spec_stats; /* SpecStats + SpecResult times (src/spec.rs:17-39) */

/* Draft source. The reference's draft is a `Model` (src/spec.rs:59); here any proposer plugs in
 * through two callbacks, and two built-ins are provided. */
typedef struct {
    void* ctx;
    /* Consume the prompt (src/spec.rs:84). */
    int (*prefill)(void* ctx, const uint32_t* prompt, size_t n);
    /* Propose kk tokens after `last` (src/spec.rs:100-107). Returns the forward calls made
     * (>= 0) or a negative error. */
    int (*propose)(void* ctx, uint32_t last, size_t kk, uint32_t* out);
    /* After a pass that accepted m drafts, the target consumed block[0..m] (positions p..p+m);
     * bring the draft to the same state (src/spec.rs:137-147). Returns forward calls made. */
    int (*commit)(void* ctx, const uint32_t* block, size_t p, size_t m);
} ls_drafter;

/* A draft model on the device, exactly as the reference uses one. */
int ls_drafter_from_model(ls_model* draft, ls_drafter* out);
/* A scripted proposer for benchmarks: for output index i it proposes greedy[i] with
 * probability p_accept, else a uniformly random other token (SplitMix64 counter stream keyed by
 * seed and i). The returned drafter owns a copy of greedy; free it with ls_drafter_free. */
int ls_drafter_scripted(const uint32_t* greedy, size_t n_greedy, double p_accept, uint64_t seed, uint64_t vocab,
                        ls_drafter* out);
/* The scripted proposal for output index i (for tests). */
uint32_t ls_drafter_scripted_token(const ls_drafter* d, size_t i);
void ls_drafter_free(ls_drafter* d);

/* speculative_greedy (src/spec.rs:57-152). out receives up to max_new tokens; *out_len the
 * count. Errors as the reference (:65-80): 1 <= k <= 32, a prompt, max_new >= 1, an empty target
 * cache, prompt + max_new + k <= max_ctx. */
int ls_speculative_greedy(ls_model* target, ls_drafter* draft, const uint32_t* prompt, size_t n_prompt,
                          size_t max_new, size_t k, const uint32_t* eos, size_t n_eos, uint32_t* out,
                          size_t* out_len, ls_spec_stats* stats);
/* The same loop in resumable form: begin runs the prompt pass (src/spec.rs:82-92), step runs
 * up to max_steps verify passes (0 = until generation ends; *done = 1 then), result copies the
 * tokens so far. Used by benchmarks to time exactly K verify passes. */
typedef struct ls_spec ls_spec;
int ls_spec_begin(ls_model* target, ls_drafter* draft, const uint32_t* prompt, size_t n_prompt, size_t max_new,
                  size_t k, const uint32_t* eos, size_t n_eos, ls_spec** out);
int ls_spec_step(ls_spec* s, size_t max_steps, int* done);
int ls_spec_result(const ls_spec* s, uint32_t* out, size_t cap, size_t* out_len, ls_spec_stats* stats);
/* Device time (ms, HIP events around each fused verify) and accepted count m of every verify
 * pass so far. Returns the number of passes; copies at most cap entries (arrays may be NULL). */
size_t ls_spec_step_log(const ls_spec* s, double* ms, uint32_t* accepted, size_t cap);
void ls_spec_free(ls_spec* s);

/* Plain greedy decoding with Sampler::greedy (src/model.rs:328-336), the parity baseline of
 * tests/spec.rs:44-57. */
int ls_greedy_generate(ls_model* m, const uint32_t* prompt, size_t n_prompt, size_t max_new, const uint32_t* eos,
                       size_t n_eos, uint32_t* out, size_t* out_len);

/* ---------------------------------------------------------------------------------------
 * Operator level: kernels::matmul (src/kernels.rs:196-203) on device buffers.
 * w_dev: the reference's row layout (rows * row_bytes); x_dev: t * cols f32; y_dev: t * rows
 * f32. stream: a hipStream_t (NULL = default stream). Synchronous on that stream.
 * ------------------------------------------------------------------------------------- */
int ls_matmul(ls_format f, const void* w_dev, size_t rows, size_t cols, const float* x_dev, size_t t,
              float* y_dev, void* stream);

/* ls_matmul without any device allocation. No counterpart in the reference: it is for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments and the same result bit for bit, but asynchronous: it enqueues its
 * kernels on `stream` and returns; synchronize the stream before reading y_dev. Everything
 * ls_matmul allocates per call (the tile-layout copy of the weights, the input fragments, the
 * split-K pieces and counters) sits in one static device array of 32 MiB per GPU, held until the
 * process ends; a call that needs more (for example a wide matrix in int8 above about 30 M
 * weights) returns LS_E_INVALID. Calls on one GPU share that array: calls that overlap in time on
 * one GPU (other streams, other threads) race and must be ordered by the caller. */
int ls_matmul_noalloc(ls_format f, const void* w_dev, size_t rows, size_t cols, const float* x_dev, size_t t,
                      float* y_dev, void* stream);

/* ---------------------------------------------------------------------------------------
 * Text and sampling around the engine, host side: the tokenizer (src/tokenizer.rs) and the
 * sampler (src/model.rs:300-366).
 * Variable-length outputs: *n (or *len) receives the full size; the data is copied only when
 * out is not NULL and cap is at least that size (call again with a larger buffer otherwise).
 * ------------------------------------------------------------------------------------- */
typedef struct ls_tokenizer ls_tokenizer;
/* Tokenizer::load (src/tokenizer.rs:67-180): vocab.json, merges.txt, tokenizer_config.json of
 * dir. LS_E_IO when a file is missing, LS_E_FORMAT for bad content. */
int ls_tokenizer_load(const char* dir, ls_tokenizer** out);
void ls_tokenizer_free(ls_tokenizer* t);
size_t ls_tokenizer_vocab_size(const ls_tokenizer* t);
/* Tokenizer::encode (src/tokenizer.rs:208-232): text (UTF-8, len bytes; LS_E_INVALID if not
 * valid UTF-8) to ids, added tokens such as <|im_start|> matched literally. */
int ls_tokenizer_encode(const ls_tokenizer* t, const char* text, size_t len, uint32_t* out, size_t cap, size_t* n);
/* Tokenizer::decode (src/tokenizer.rs:303-306): special tokens hidden, invalid UTF-8 replaced by
 * U+FFFD. */
int ls_tokenizer_decode(const ls_tokenizer* t, const uint32_t* ids, size_t n, char* out, size_t cap, size_t* len);
/* Tokenizer::token_bytes (src/tokenizer.rs:289-301). */
int ls_tokenizer_token_bytes(const ls_tokenizer* t, uint32_t id, int show_special, char* out, size_t cap, size_t* len);
/* Tokenizer::token_id (src/tokenizer.rs:200-202): 1 and *id when the token exists, else 0. */
int ls_tokenizer_token_id(const ls_tokenizer* t, const char* token, uint32_t* id);
/* Tokenizer::is_special (src/tokenizer.rs:204-206). */
int ls_tokenizer_is_special(const ls_tokenizer* t, uint32_t id);
/* The pre-token split of text (src/tokenizer.rs:356-437; the Qwen2 pattern with the Unicode
 * letter and number categories): ends[i] is the code point end of pre-token i. For tests. */
int ls_tokenizer_pretokens(const char* text, size_t len, uint32_t* ends, size_t cap, size_t* n);

/* StreamDecoder (src/tokenizer.rs:311-346): feed token bytes, get the text complete so far.
 * out must hold 3 * (n + 4) bytes (no partial copies: the decoder's state moves on). */
typedef struct ls_stream_decoder ls_stream_decoder;
int ls_stream_decoder_new(ls_stream_decoder** out);
void ls_stream_decoder_free(ls_stream_decoder* d);
int ls_stream_decoder_push(ls_stream_decoder* d, const char* bytes, size_t n, char* out, size_t cap, size_t* len);
int ls_stream_decoder_finish(ls_stream_decoder* d, char* out, size_t cap, size_t* len);

/* Sampler::new (src/model.rs:309-311) and Sampler::sample (:322-365): greedy at temperature <= 0
 * (the first maximum), else the top_k largest (at least 1; equal logits by lower index), softmax
 * at the temperature, the smallest prefix reaching top_p, and a draw from the seeded xorshift64*
 * stream. logits: n host floats. */
typedef struct ls_sampler ls_sampler;
int ls_sampler_new(float temperature, size_t top_k, float top_p, uint64_t seed, ls_sampler** out);
void ls_sampler_free(ls_sampler* s);
int ls_sampler_sample(ls_sampler* s, const float* logits, size_t n, uint32_t* token);

#ifdef __cplusplus
}
#endif
#endif
