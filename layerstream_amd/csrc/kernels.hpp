// Device kernels of the verify step and their host launchers (gfx950).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace ls {

// Weight matrix in the engine's device layout ("strips"): rows are grouped in strips of 64,
// one row per lane of a wavefront. For each strip the packed row data is cut into 16-byte
// chunks, stored chunk-major: [strip][chunk][64 lanes][16 B], so one wavefront load of a chunk
// reads 1 KiB of contiguous memory. Scales are [strip][group][64] bf16. Padding rows are zero
// (scale 0); padding bytes past the row decode to zero weights. The bytes are the reference's
// row bytes rearranged (no value changes).
struct DevMat {
    const uint8_t* data = nullptr;
    const uint16_t* scales = nullptr;
    int bits = 16, group = 0;
    int rows = 0, cols = 0;
    int n_strips = 0, n_chunks = 0, n_groups = 0;
};

constexpr int STRIP = 64;
constexpr int MAX_T = 16;  // tokens per matvec tile

size_t devmat_data_bytes(int bits, int rows, int cols);
size_t devmat_scale_count(int bits, int group, int rows, int cols);
int devmat_chunks(int bits, int cols);

// Host-side repack of `rows` reference rows (row_bytes each) into the strip layout.
void repack_rows_host(const uint8_t* raw, int bits, int group, int rows, int cols, uint8_t* data, uint16_t* scales,
                      int row_offset_in_dest, int dest_rows);
// Device-side repack (for streamed layers): same mapping, raw rows already on the device.
void repack_rows_device(const uint8_t* raw, int bits, int group, int rows, int cols, uint8_t* data, uint16_t* scales,
                        int row_offset_in_dest, int dest_rows, hipStream_t s);

// y = W x for t <= MAX_T inputs. Split over K in `splits` ranges; partial sums
// part[split][t][rows_pad] are reduced in split order by the epilogue kernels below.
int matvec_splits(const DevMat& W, int t);
void matvec(const DevMat& W, const float* x, int ldx, int t, float* part, int splits, hipStream_t s);

// Epilogues over the partial sums (all reduce splits 0..S-1 in order, then):
//   out[t][ldo] = sum (+ bias)                    (bias may be null)
//   x[t][ldx] += sum                               (residual)
void reduce_store(const float* part, int splits, int t, int rows, int rows_pad, const float* bias, float* out, int ldo,
                  hipStream_t s);
void reduce_residual(const float* part, int splits, int t, int rows, int rows_pad, float* x, int ldx, hipStream_t s);

// x[t][h] = dequantized embedding rows of tokens[t] (embedding in strip layout).
void embed_gather(const DevMat& E, const uint32_t* tokens, int t, float* x, hipStream_t s);
// out[r] = x[r] * (1 / sqrt(mean(x[r]^2) + eps)) * w for rows r < t.
void rms_norm(const float* x, const float* w, int n, float eps, int t, float* out, hipStream_t s);
// RoPE (rotate half) on the q and k heads of qkv[t][h + 2 kv] at positions pos0 + i with the
// host-computed cos/sin table [max_ctx][hd/2], then K/V rows appended at pos0 + i.
void rope_append_kv(float* qkv, int t, int heads, int kv_heads, int hd, int pos0, const float* cos_t, const float* sin_t,
                    float* k_cache, float* v_cache, hipStream_t s);
// Causal GQA attention for token i at position pos0 + i over cache rows [0, pos0 + i].
void attention(const float* qkv, int t, int heads, int kv_heads, int hd, int pos0, int max_ctx, const float* k_cache,
               const float* v_cache, float* scores, float* out, hipStream_t s);
// act[t][inter] = silu(gu[t][0:inter]) * gu[t][inter:2 inter]
void silu_mul(const float* gu, int t, int inter, float* act, hipStream_t s);
// amax[r] = first index of the maximum of logits[r][0:n] (src/spec.rs:41-49 tie and NaN rule).
void argmax_rows(const float* logits, int ld, int n, int rows, float* pval, int* pidx, uint32_t* amax, hipStream_t s);
// dst[i] = widened bf16 src[i] (little-endian bytes), i < n.
void bf16_to_f32_dev(const uint8_t* src, int n, float* dst, hipStream_t s);
// x[t][cols] = dequantized raw embedding rows raw[t][row_bytes] (reference row layout).
void embed_raw_rows(const uint8_t* raw, int bits, int group, int cols, int t, float* x, hipStream_t s);
// Greedy acceptance (src/spec.rs:119-127): m = first i < n-1 with amax[i] != block[i+1] (else
// n-1); next = amax[m]. Writes out[0] = m, out[1] = next.
void accept_greedy(const uint32_t* amax, const uint32_t* block, int n, uint32_t* out, hipStream_t s);

}  // namespace ls
