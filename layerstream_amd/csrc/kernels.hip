// Small device kernels of the verify step for gfx950 (CDNA4, wave64): attention, greedy
// acceptance and helpers. The weight-streaming kernels live in fused.hip.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <stdexcept>
#include <string>

#include "kernels.hpp"

namespace ls {

#define HIPCHECK(x)                                                                        \
    do {                                                                                   \
        hipError_t e_ = (x);                                                               \
        if (e_ != hipSuccess) throw std::runtime_error(std::string("HIP: ") + hipGetErrorString(e_)); \
    } while (0)

// ---------------------------------------------------------------------------------------
// Causal GQA attention (src/model.rs:261-282), split over the context in chunks of ACH keys
// (flash-decoding). The reference computes scores (q . k_j) * scale, a softmax (max,
// exp(x - max), sum, * 1/sum) and sum_j p_j v_j over every cached position; here each chunk
// yields (m, l, o) = (max score, sum of exp(s - m), sum of exp(s - m) v) and the combine
// rescales the chunks in chunk order. Chunk boundaries depend only on key positions, so a
// token's result does not depend on how many tokens share the launch.
// ---------------------------------------------------------------------------------------
constexpr int ACH = 64;  // keys per chunk
constexpr int ATQ = 16;  // query tokens per block

__global__ __launch_bounds__(256) void k_attn_chunk(const float* __restrict__ q, int ldq, int t, int heads, int kv_heads, int hd,
                                                    int pos0, float scale, const float* __restrict__ kc,
                                                    const float* __restrict__ vc, int nc_max, float* __restrict__ pm,
                                                    float* __restrict__ pl, float* __restrict__ po) {
    extern __shared__ float sm[];
    const int c = blockIdx.x, head = blockIdx.y, i0 = blockIdx.z * ATQ;
    const int kv = kv_heads * hd;
    const int g = head / (heads / kv_heads);
    const int j0 = c * ACH;
    const int nq = min(ATQ, t - i0);
    const int nk = min(ACH, pos0 + t - j0);  // keys that exist in this chunk
    float* Ks = sm;                       // [ACH][hd + 1]
    float* Vs = Ks + ACH * (hd + 1);      // [ACH][hd]
    float* Q = Vs + ACH * hd;             // [ATQ][hd]
    float* S = Q + ATQ * hd;              // [ATQ][ACH]
    for (int p = threadIdx.x; p < ACH * hd; p += 256) {
        const int j = p / hd, d = p % hd;
        float kx = 0.0f, vx = 0.0f;
        if (j < nk) {
            kx = kc[size_t(j0 + j) * kv + g * hd + d];
            vx = vc[size_t(j0 + j) * kv + g * hd + d];
        }
        Ks[j * (hd + 1) + d] = kx;
        Vs[j * hd + d] = vx;
    }
    for (int p = threadIdx.x; p < nq * hd; p += 256) {
        const int i = p / hd, d = p % hd;
        Q[i * hd + d] = q[size_t(i0 + i) * ldq + head * hd + d];
    }
    __syncthreads();
    for (int p = threadIdx.x; p < nq * ACH; p += 256) {
        const int i = p / ACH, j = p % ACH;
        float sc = -INFINITY;
        if (j < nk && j0 + j <= pos0 + i0 + i) {
            float a = 0.0f;
            for (int d = 0; d < hd; d++) a = __builtin_fmaf(Q[i * hd + d], Ks[j * (hd + 1) + d], a);
            sc = a * scale;
        }
        S[i * ACH + j] = sc;
    }
    __syncthreads();
    // One wavefront per query row: lane j holds key j (ACH == 64 == wave size).
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int i = w; i < nq; i += 4) {
        const float sc = S[i * ACH + lane];
        float m = sc;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        const float e = sc == -INFINITY ? 0.0f : expf(sc - m);
        float l = e;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o, 64);
        S[i * ACH + lane] = e;
        if (lane == 0) {
            const size_t at = (size_t(i0 + i) * heads + head) * nc_max + c;
            pm[at] = m;
            pl[at] = l;
        }
    }
    __syncthreads();
    for (int p = threadIdx.x; p < nq * hd; p += 256) {
        const int i = p / hd, d = p % hd;
        float o = 0.0f;
        for (int j = 0; j < ACH; j++) o = __builtin_fmaf(S[i * ACH + j], Vs[j * hd + d], o);
        po[((size_t(i0 + i) * heads + head) * nc_max + c) * hd + d] = o;
    }
}

// out[i][head] = sum_c o_c e^(m_c - M) / sum_c l_c e^(m_c - M) over the chunks token i sees.
__global__ void k_attn_combine(int heads, int hd, int pos0, int nc_max, const float* __restrict__ pm,
                               const float* __restrict__ pl, const float* __restrict__ po, float* __restrict__ out) {
    const int i = blockIdx.x, head = blockIdx.y;
    const int nci = (pos0 + i + 1 + ACH - 1) / ACH;
    const size_t base = (size_t(i) * heads + head) * nc_max;
    float M = -INFINITY;
    for (int c = 0; c < nci; c++) M = fmaxf(M, pm[base + c]);
    float L = 0.0f;
    for (int c = 0; c < nci; c++) L += pl[base + c] * expf(pm[base + c] - M);
    const float inv = 1.0f / L;
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float o = 0.0f;
        for (int c = 0; c < nci; c++) o = __builtin_fmaf(po[(base + c) * hd + d], expf(pm[base + c] - M), o);
        out[size_t(i) * heads * hd + head * hd + d] = o * inv;
    }
}

size_t attention_scratch_floats(int t, int heads, int hd, int max_ctx) {
    const size_t nc = (size_t(max_ctx) + ACH - 1) / ACH;
    return size_t(t) * heads * nc * (hd + 2);
}

void attention(const float* q, int ldq, int t, int heads, int kv_heads, int hd, int pos0, int max_ctx, const float* k_cache,
               const float* v_cache, float* scratch, float* out, hipStream_t s) {
    if (hd > 256) throw std::runtime_error("head_dim too large");
    const float scale = 1.0f / sqrtf(float(hd));
    const int nc_max = (max_ctx + ACH - 1) / ACH;
    const int nc = (pos0 + t + ACH - 1) / ACH;
    float* pm = scratch;
    float* pl = pm + size_t(t) * heads * nc_max;
    float* po = pl + size_t(t) * heads * nc_max;
    const size_t lds = sizeof(float) * (ACH * (hd + 1) + ACH * hd + ATQ * hd + ATQ * ACH);
    hipLaunchKernelGGL(k_attn_chunk, dim3(nc, heads, (t + ATQ - 1) / ATQ), dim3(256), lds, s, q, ldq, t, heads, kv_heads, hd, pos0,
                       scale, k_cache, v_cache, nc_max, pm, pl, po);
    HIPCHECK(hipGetLastError());
    hipLaunchKernelGGL(k_attn_combine, dim3(t, heads), dim3(64), 0, s, heads, hd, pos0, nc_max, pm, pl, po, out);
    HIPCHECK(hipGetLastError());
}

__global__ void k_bf16_to_f32(const uint8_t* __restrict__ src, int n, float* __restrict__ dst) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = __uint_as_float(uint32_t(src[2 * i] | (src[2 * i + 1] << 8)) << 16);
}

void bf16_to_f32_dev(const uint8_t* src, int n, float* dst, hipStream_t s) {
    hipLaunchKernelGGL(k_bf16_to_f32, dim3((n + 255) / 256), dim3(256), 0, s, src, n, dst);
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

__global__ void k_accept(const uint32_t* __restrict__ amax, const uint32_t* __restrict__ block, int n, uint32_t* out) {
    if (threadIdx.x != 0) return;
    int m = 0;
    while (m < n - 1 && amax[m] == block[m + 1]) m++;
    out[0] = uint32_t(m);
    out[1] = amax[m];
}

void accept_greedy(const uint32_t* amax, const uint32_t* block, int n, uint32_t* out, hipStream_t s) {
    hipLaunchKernelGGL(k_accept, dim3(1), dim3(64), 0, s, amax, block, n, out);
    HIPCHECK(hipGetLastError());
}

}  // namespace ls
