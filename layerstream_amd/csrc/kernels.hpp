// Small device kernels of the verify step (gfx950): attention and embedding helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace ls {

// Causal GQA attention for token i at position *pos0 + i over cache rows [0, *pos0 + i], split
// over the context in fixed chunks (pos0 is a device scalar, so the launch does not depend on
// it). q: [t][ldq] (heads * hd used). The output rows [t][heads * hd] are written as B
// fragments (fused.hpp) into `frags`, tile stride frag_tile_bytes(heads * hd). scratch holds
// attention_scratch_floats() floats; cnt holds ceil(t / 16) * heads counters, zero at the
// start and left at zero; `splits` workgroups share each (head, token tile).
size_t attention_scratch_floats(int t, int heads, int hd, int max_ctx);
int attention_splits(int max_ctx);
void attention(const float* q, int ldq, int t, int heads, int kv_heads, int hd, const int* pos0, int max_ctx, const float* k_cache,
               const float* v_cache, float* scratch, int* cnt, int splits, uint8_t* frags, hipStream_t s);
// dst[i] = widened bf16 src[i] (little-endian bytes), i < n.
void bf16_to_f32_dev(const uint8_t* src, int n, float* dst, hipStream_t s);
// x[t][cols] = dequantized raw embedding rows raw[t][row_bytes] (reference row layout).
void embed_raw_rows(const uint8_t* raw, int bits, int group, int cols, int t, float* x, hipStream_t s);

}  // namespace ls
