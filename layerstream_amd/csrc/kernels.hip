// Small device kernels of the verify step for gfx950 (CDNA4, wave64): attention and the
// embedding helpers of streamed tables. The weight-streaming kernels live in fused.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>

#include "kernels.hpp"

#include "attn_dev.hpp"
#include "frag_dev.hpp"
#include "fused.hpp"

namespace ls {

#define HIPCHECK(x)                                                                        \
    do {                                                                                   \
        hipError_t e_ = (x);                                                               \
        if (e_ != hipSuccess) throw std::runtime_error(std::string("HIP: ") + hipGetErrorString(e_)); \
    } while (0)

template <int HD>
__global__ __launch_bounds__(AWV * 64) void k_attn(AttnArgs a) {
    __shared__ __align__(16) uint8_t smem[attn_lds_bytes<HD>()];
    attn_body<HD, false>(a, blockIdx.x, blockIdx.y, blockIdx.z, Flow{}, smem);
}

template <int HD>
__global__ __launch_bounds__(AWV * 64, 2) void k_attn_grp(AttnArgs a) {  // one workgroup per CU (LDS)
    __shared__ __align__(16) uint8_t smem[attn_grp_lds_bytes<HD>()];
    attn_group_body<HD>(a, blockIdx.x, blockIdx.y, blockIdx.z, smem);
}

size_t attention_scratch_floats(int t, int heads, int hd, int) { return size_t(t) * heads * ASPLIT * (hd + 2); }

// A batch's segments run with the heads of a KV group together (k_attn_grp) unless
// LS_ATTN_GROUP=0 (one workgroup per head and split, k_attn; token tiles of one sequence always
// do): the same bits either way.
static bool attn_grouped() {
    static const bool on = [] {
        const char* e = std::getenv("LS_ATTN_GROUP");
        return !e || std::atoi(e) != 0;
    }();
    return on;
}

template <int HD>
static void launch_attn(const float* q, int ldq, int t, int heads, int kv_heads, const int* pos0, const AttnRows& rows,
                        const float* kc, const float* vc, float* scratch, int* cnt, uint8_t* frags, hipStream_t s) {
    const AttnArgs a = make_attn_args(q, ldq, t, heads, kv_heads, HD, pos0, rows, kc, vc, scratch, cnt, frags);
    const int nseg = rows.segs ? rows.n_segs : (t + ATQ - 1) / ATQ;
    // (the final merge holds a group's output rows in the LDS of the wavefront outputs)
    if (attn_grouped() && rows.segs && heads > kv_heads && heads / kv_heads <= AWV)
        hipLaunchKernelGGL(k_attn_grp<HD>, dim3(ASPLIT, kv_heads, nseg), dim3(AWV * 64), 0, s, a);
    else
        hipLaunchKernelGGL(k_attn<HD>, dim3(ASPLIT, heads, nseg), dim3(AWV * 64), 0, s, a);
    HIPCHECK(hipGetLastError());
}

void attention(const float* q, int ldq, int t, int heads, int kv_heads, int hd, const int* pos0, const AttnRows& rows,
               const float* k_cache, const float* v_cache, float* scratch, int* cnt, uint8_t* frags, hipStream_t s) {
    if (rows.segs && rows.n_segs <= 0) throw std::runtime_error("attention: empty segment table");
    switch (hd) {
        case 16: launch_attn<16>(q, ldq, t, heads, kv_heads, pos0, rows, k_cache, v_cache, scratch, cnt, frags, s); break;
        case 32: launch_attn<32>(q, ldq, t, heads, kv_heads, pos0, rows, k_cache, v_cache, scratch, cnt, frags, s); break;
        case 64: launch_attn<64>(q, ldq, t, heads, kv_heads, pos0, rows, k_cache, v_cache, scratch, cnt, frags, s); break;
        case 128: launch_attn<128>(q, ldq, t, heads, kv_heads, pos0, rows, k_cache, v_cache, scratch, cnt, frags, s); break;
        default: throw std::runtime_error("head_dim must be 16, 32, 64 or 128");
    }
}


__global__ void k_bf16_to_f32(const uint8_t* __restrict__ src, int n, float* __restrict__ dst) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = __uint_as_float(uint32_t(src[2 * i] | (src[2 * i + 1] << 8)) << 16);
}

void bf16_to_f32_dev(const uint8_t* src, int n, float* dst, hipStream_t s) {
    hipLaunchKernelGGL(k_bf16_to_f32, dim3((n + 255) / 256), dim3(256), 0, s, src, n, dst);
    HIPCHECK(hipGetLastError());
}

// Vector blockIdx.y of w, 256 elements per workgroup along x.
__global__ void k_bf16_to_f32_multi(Widen w) {
    const int v = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < w.n[v]) w.dst[v][i] = __uint_as_float(uint32_t(w.src[v][2 * i] | (w.src[v][2 * i + 1] << 8)) << 16);
}

void bf16_to_f32_dev(const Widen& w, hipStream_t s) {
    if (w.count <= 0) return;
    if (w.count > Widen::MAX) throw std::runtime_error("too many vectors for one widening launch");
    int n = 0;
    for (int v = 0; v < w.count; v++) n = std::max(n, w.n[v]);
    hipLaunchKernelGGL(k_bf16_to_f32_multi, dim3((n + 255) / 256, w.count), dim3(256), 0, s, w);
    HIPCHECK(hipGetLastError());
}

// Raw reference rows: data bytes, then one bf16 scale per group (src/kernels.rs:95-121).
__global__ void k_embed_raw(const uint8_t* __restrict__ raw, int bits, int group, int cols, float* __restrict__ x) {
    const int i = blockIdx.x;
    const int db = bits == 16 ? cols * 2 : cols * bits / 8;
    const int rb = db + (bits == 16 ? 0 : (cols / group) * 2);
    const uint8_t* row = raw + size_t(i) * rb;
    float* out = x + size_t(i) * cols;
    for (int c = threadIdx.x; c < cols; c += blockDim.x) {
        if (bits == 16) {
            out[c] = __uint_as_float(uint32_t(row[2 * c] | (row[2 * c + 1] << 8)) << 16);
            continue;
        }
        const int g = c / group;
        const float s = __uint_as_float(uint32_t(row[db + 2 * g] | (row[db + 2 * g + 1] << 8)) << 16);
        float q;
        if (bits == 8) {
            q = float(int32_t(int8_t(row[c])));
        } else {
            const int half = group / 2, j = c % group;
            const uint8_t b = row[g * half + (j < half ? j : j - half)];
            q = float(int32_t(j < half ? (b & 15) : (b >> 4)) - 8);
        }
        out[c] = q * s;
    }
}

void embed_raw_rows(const uint8_t* raw, int bits, int group, int cols, int t, float* x, hipStream_t s) {
    hipLaunchKernelGGL(k_embed_raw, dim3(t), dim3(256), 0, s, raw, bits, group, cols, x);
    HIPCHECK(hipGetLastError());
}

}  // namespace ls
