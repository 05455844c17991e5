// Small device kernels of the verify step (gfx950): attention and embedding helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace ls {

// Rows of several sequences in one attention launch. segs[z] = (first launch row, rows <= 16,
// sequence, unused) for segment z; a segment lies inside one 16-row tile and its rows are
// consecutive positions of one sequence. pos[row] is each launch row's position; sequence s
// reads the caches at k_cache / v_cache + s * seq_stride floats. All device memory.
struct AttnRows {
    const int4* segs = nullptr;
    int n_segs = 0;
    const int* pos = nullptr;
    size_t seq_stride = 0;
};

// Causal GQA attention (src/model.rs:261-282) for every launch row over its cache rows
// [0, position]. Without a segment table (rows.segs null) the rows are one sequence and row i
// sits at position *pos0 + i (pos0 is a device scalar, so the launch does not depend on it).
// q: [t][ldq] (heads * hd used). The output rows [t][heads * hd] are written as B fragments
// (fused.hpp) into `frags`, tile stride frag_tile_bytes(heads * hd). scratch holds
// attention_scratch_floats() floats; cnt holds one counter per (segment, head) (ceil(t / 16)
// segments without a table), zero at the start and left at zero.
constexpr int ATTN_SPLIT = 8;  // workgroups per (head, segment)
size_t attention_scratch_floats(int t, int heads, int hd, int max_ctx);
void attention(const float* q, int ldq, int t, int heads, int kv_heads, int hd, const int* pos0, const AttnRows& rows,
               const float* k_cache, const float* v_cache, float* scratch, int* cnt, uint8_t* frags, hipStream_t s);
// dst[i] = widened bf16 src[i] (little-endian bytes), i < n.
void bf16_to_f32_dev(const uint8_t* src, int n, float* dst, hipStream_t s);
// Several such vectors in one launch.
struct Widen {
    static constexpr int MAX = 8;
    const uint8_t* src[MAX] = {};
    float* dst[MAX] = {};
    int n[MAX] = {};
    int count = 0;
    void add(const uint8_t* s, int len, float* d) {
        src[count] = s;
        n[count] = len;
        dst[count] = d;
        count++;
    }
};
void bf16_to_f32_dev(const Widen& w, hipStream_t s);
// x[t][cols] = dequantized raw embedding rows raw[t][row_bytes] (reference row layout).
void embed_raw_rows(const uint8_t* raw, int bits, int group, int cols, int t, float* x, hipStream_t s);

}  // namespace ls
