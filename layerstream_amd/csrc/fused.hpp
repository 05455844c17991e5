// Fused MFMA kernels of the verify step (gfx950).
//
// Weights use the "tile" layout: rows in strips of 16 (the MFMA M dimension), columns padded to a
// multiple of 128 and cut into chunks of 16 bytes per lane ([strip][chunk][64 lanes][16 B]), so
// that a wavefront load of one chunk of one strip is 1 KiB of contiguous memory and each lane
// receives exactly the A operand of v_mfma_f32_16x16x32_bf16 for its row and k-block. A chunk
// covers 32 columns for bf16, 64 for int8 and 128 for int4. Scales are [strip][group][16 rows]
// bf16. Inputs reach the MFMA B operand as three bf16 terms whose sum is the f32 value exactly
// ("B fragments", [k-step][term][64 lanes][16 B]), so every product is exact and accumulation is
// f32.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace ls {

struct TMat {
    const uint8_t* data = nullptr;
    const uint16_t* scales = nullptr;
    int bits = 16, group = 0;
    int rows = 0, cols = 0;
    int n_strips = 0;   // padded to a multiple of 4 (64 rows) or more
    int n_chunks = 0;   // chunks per strip
    int n_groups = 0;   // groups per row, padding columns included
};

constexpr int FTOK = 16;  // tokens per launch tile (the MFMA N dimension)

__host__ __device__ inline int tile_chunk_cols(int bits) { return bits == 16 ? 32 : (bits == 8 ? 64 : 128); }
__host__ __device__ inline int tile_kpad(int cols) { return (cols + 127) / 128 * 128; }
// Rows are padded to a multiple of row_align (64, or 256 for the output head's 256-row blocks).
TMat tile_shape(int bits, int group, int rows, int cols, int row_align = 64);
size_t tile_data_bytes(const TMat& m);
size_t tile_scale_bytes(const TMat& m);
TMat tile_bind(const TMat& shape, uint8_t* data, uint16_t* scales);
// Rearrange `rows` reference rows (raw, on the device) into the tile layout. Source row r goes
// to destination row row_off + (r / block) * stride + r % block (block = rows: contiguous).
void tile_repack(const uint8_t* raw, int rows, const TMat& dst, int row_off, int block, int stride, hipStream_t s);
// Initialise padding: zero-weight bytes and zero scales over the whole matrix.
void tile_clear(const TMat& m, hipStream_t s);

// Embedding rows of tokens from a tile-layout table (src/kernels.rs:95-121 dequantization).
void tile_embed(const TMat& E, const uint32_t* tokens, int t, float* x, hipStream_t s);

// B fragments of x rows [i0, i0 + nt) (f32, row stride ldx), optionally RMS-normalised with w,
// written to global memory (kpad / 32 k-steps x 3 KiB).
void frag_build(const float* x, int ldx, int i0, int nt, int cols, const float* w, float eps, uint8_t* frags, hipStream_t s);

struct FusedArgs {
    // weights
    TMat W;
    // input: f32 rows (x) with optional RMSNorm weights, or prebuilt B fragments
    const float* x = nullptr;
    int ldx = 0;
    const float* norm = nullptr;
    float eps = 0;
    const uint8_t* frags = nullptr;
    int i0 = 0, nt = 0;  // token tile
    // epilogue data
    const float* bias = nullptr;
    float* out = nullptr;  // q rows / residual rows / logits
    int ldo = 0;
    float* kcache = nullptr;
    float* vcache = nullptr;
    const float* rope_cos = nullptr;
    const float* rope_sin = nullptr;
    const int* pos0 = nullptr;  // device scalar: position of token 0 of the step
    int heads = 0, kv_heads = 0, hd = 0;
    uint8_t* frag_out = nullptr;  // SiLU epilogue: act fragments
    float* arg_val = nullptr;     // argmax epilogue partials [block][16]
    int* arg_idx = nullptr;
    int row_base = 0;             // added to argmax row indices
    float* row0 = nullptr;        // head: logits of row 0 of this launch, per token
};

// QKV projection + bias + RoPE + K/V append (norm prologue). Rows: q heads, k heads, v heads.
void fused_qkv(const FusedArgs& a, hipStream_t s);
// y = W x, x[row] += y (norm-free prologue from f32 rows, or fragments).
void fused_residual(const FusedArgs& a, int ksplit, hipStream_t s);
// gate|up projection (row blocks of 64 interleaved gate, up) + SiLU(g) * u -> act fragments.
void fused_gate_up(const FusedArgs& a, hipStream_t s);
// Output head: logits of 256-row blocks, per-block argmax partials, optional logits store.
void fused_head(const FusedArgs& a, hipStream_t s);
int fused_head_blocks(const TMat& E);
// Final argmax over head-block partials (src/spec.rs:41-49 rule); row0 holds logits[.][0].
void head_argmax_final(const float* pv, const int* pi, int nblocks, const float* row0, int i0, int nt, uint32_t* amax,
                       hipStream_t s);

}  // namespace ls
