// Small device kernels of the verify step for gfx950 (CDNA4, wave64): attention and the
// embedding helpers of streamed tables. The weight-streaming kernels live in fused.hip.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <stdexcept>
#include <string>

#include "kernels.hpp"

#include "frag_dev.hpp"
#include "fused.hpp"

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
//
// One launch: grid (splits, heads, token tiles). Workgroup s takes chunks s, s + splits, ...
// of its (head, tile); the last of the `splits` workgroups to finish (an agent-scope counter)
// combines every chunk and writes the output rows as fragments. The grid does not depend on
// the position (read from the device), so the launch can be replayed from a graph.
// ---------------------------------------------------------------------------------------
constexpr int ACH = 64;  // keys per chunk
constexpr int ATQ = 16;  // query tokens per tile
constexpr int CPOL_SC1 = 16;
constexpr int BUF_DWORD3 = 0x00020000;
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_rsrc(const void* p, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, int(bytes), BUF_DWORD3);
}
// Coherent (sc1) float accesses; the buffer builtins move raw 32-bit words.
__device__ __forceinline__ void st_f32(float v, __amdgpu_buffer_rsrc_t r, int at) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, at, 0, CPOL_SC1);
}
__device__ __forceinline__ float ld_f32(__amdgpu_buffer_rsrc_t r, int at) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, at, 0, CPOL_SC1));
}

// DPT consecutive floats through the coherent buffer path (128-bit pieces when DPT allows).
template <int DPT>
__device__ __forceinline__ void store_dpt(const float* v, __amdgpu_buffer_rsrc_t r, int at) {
    if constexpr (DPT % 4 == 0) {
#pragma unroll
        for (int u = 0; u < DPT; u += 4)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, f32x4{v[u], v[u + 1], v[u + 2], v[u + 3]}), r,
                                                   at + 4 * u, 0, CPOL_SC1);
    } else {
#pragma unroll
        for (int u = 0; u < DPT; u++) st_f32(v[u], r, at + 4 * u);
    }
}
template <int DPT>
__device__ __forceinline__ void load_dpt(float* v, __amdgpu_buffer_rsrc_t r, int at) {
    if constexpr (DPT % 4 == 0) {
#pragma unroll
        for (int u = 0; u < DPT; u += 4) {
            const f32x4 x = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, at + 4 * u, 0, CPOL_SC1));
            v[u] = x[0];
            v[u + 1] = x[1];
            v[u + 2] = x[2];
            v[u + 3] = x[3];
        }
    } else {
#pragma unroll
        for (int u = 0; u < DPT; u++) v[u] = ld_f32(r, at + 4 * u);
    }
}

template <int HD>
struct AttnLds {
    static constexpr int KP = HD + 4;  // padded K row
    static constexpr int K = 0, V = K + ACH * KP, Q = V + ACH * HD, P = Q + ATQ * HD, END = P + ATQ * ACH;
};

template <int HD>
__global__ __launch_bounds__(256) void k_attn(const float* __restrict__ q, int ldq, int t, int heads, int kv_heads,
                                              const int* __restrict__ pos0p, float scale, const float* __restrict__ kc,
                                              const float* __restrict__ vc, int nc_max, float* pm, float* pl, float* po, int* cnt,
                                              uint8_t* __restrict__ frags, size_t frag_stride) {
    using LY = AttnLds<HD>;
    constexpr int KP = LY::KP, H4 = HD / 4, DPT = HD / 16;  // dims per thread in PV and combine
    extern __shared__ __align__(16) float sm[];
    __shared__ int flag;
    float* Ks = sm + LY::K;
    float* Vs = sm + LY::V;
    float* Qs = sm + LY::Q;
    float* Ps = sm + LY::P;
    const int S = gridDim.x, s = blockIdx.x, head = blockIdx.y, tile = blockIdx.z, i0 = tile * ATQ;
    const int tid = threadIdx.x, row = tid >> 4, sub = tid & 15;
    const int kv = kv_heads * HD, g = head / (heads / kv_heads);
    const int nq = min(ATQ, t - i0);
    const int pos0 = *pos0p;
    const int last_key = pos0 + i0 + nq - 1;
    const int nc = last_key / ACH + 1;
    const size_t rows_total = size_t(t) * heads;
    const __amdgpu_buffer_rsrc_t rm = coherent_rsrc(pm, rows_total * nc_max * 4);
    const __amdgpu_buffer_rsrc_t rl = coherent_rsrc(pl, rows_total * nc_max * 4);
    const __amdgpu_buffer_rsrc_t ro = coherent_rsrc(po, rows_total * nc_max * HD * 4);

    for (int p = tid; p < nq * H4; p += 256) {
        const int i = p / H4, d = 4 * (p % H4);
        *reinterpret_cast<float4*>(Qs + i * HD + d) = *reinterpret_cast<const float4*>(q + size_t(i0 + i) * ldq + head * HD + d);
    }
    for (int c = s; c < nc; c += S) {
        const int j0 = c * ACH, nk = min(ACH, last_key + 1 - j0);
        constexpr int NP = (ACH * H4 + 255) / 256;
        float4 kx[NP], vx[NP];
#pragma unroll
        for (int u = 0; u < NP; u++) {
            const int p = tid + u * 256, j = p / H4, d = 4 * (p % H4);
            kx[u] = vx[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (p < ACH * H4 && j < nk) {
                kx[u] = *reinterpret_cast<const float4*>(kc + size_t(j0 + j) * kv + g * HD + d);
                vx[u] = *reinterpret_cast<const float4*>(vc + size_t(j0 + j) * kv + g * HD + d);
            }
        }
        __syncthreads();  // the previous chunk is done with Ks, Vs and Ps
#pragma unroll
        for (int u = 0; u < NP; u++) {
            const int p = tid + u * 256, j = p / H4, d = 4 * (p % H4);
            if (p < ACH * H4) {
                *reinterpret_cast<float4*>(Ks + j * KP + d) = kx[u];
                *reinterpret_cast<float4*>(Vs + j * HD + d) = vx[u];
            }
        }
        __syncthreads();
        // Scores: thread (row, sub) owns keys sub + 16 u (rows 68 floats apart: the 16 lanes of a
        // row read distinct banks); each dot product runs over d in order.
        float sc[4];
        {
            float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (row < nq) {
#pragma unroll 4
                for (int d = 0; d < HD; d += 4) {
                    const float4 q4 = *reinterpret_cast<const float4*>(Qs + row * HD + d);
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const float4 k4 = *reinterpret_cast<const float4*>(Ks + (sub + 16 * u) * KP + d);
                        a[u] = __builtin_fmaf(q4.x, k4.x, a[u]);
                        a[u] = __builtin_fmaf(q4.y, k4.y, a[u]);
                        a[u] = __builtin_fmaf(q4.z, k4.z, a[u]);
                        a[u] = __builtin_fmaf(q4.w, k4.w, a[u]);
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int j = sub + 16 * u;
                sc[u] = (row < nq && j < nk && j0 + j <= pos0 + i0 + row) ? a[u] * scale : -INFINITY;
            }
        }
        // Chunk softmax over the 16 lanes of the row.
        float m = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        float l = 0.0f;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float e = sc[u] == -INFINITY ? 0.0f : expf(sc[u] - m);
            Ps[row * ACH + sub + 16 * u] = e;
            l += e;
        }
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) l += __shfl_xor(l, o, 64);
        if (sub == 0 && row < nq) {
            const int at = int(((size_t(i0 + row) * heads + head) * nc_max + c) * 4);
            st_f32(m, rm, at);
            st_f32(l, rl, at);
        }
        __syncthreads();
        // o = sum_j p_j v_j in key order; thread (row, sub) owns dims sub * DPT ..
        if (row < nq) {
            float o[DPT];
#pragma unroll
            for (int u = 0; u < DPT; u++) o[u] = 0.0f;
#pragma unroll 8
            for (int j = 0; j < ACH; j++) {
                const float pj = Ps[row * ACH + j];
#pragma unroll
                for (int u = 0; u < DPT; u++) o[u] = __builtin_fmaf(pj, Vs[j * HD + sub * DPT + u], o[u]);
            }
            store_dpt<DPT>(o, ro, int((((size_t(i0 + row) * heads + head) * nc_max + c) * HD + sub * DPT) * 4));
        }
    }

    // The last workgroup of (head, tile) combines the chunks.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        int* cn = cnt + size_t(tile) * heads + head;
        const int old = __hip_atomic_fetch_add(cn, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = old == S - 1;
        if (last) __hip_atomic_store(cn, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        flag = last;
    }
    __syncthreads();
    if (!flag) return;
    float* Es = sm;  // [ATQ][nc_max] chunk weights e^(m_c - M)
    float* Os = sm + size_t(ATQ) * nc_max;  // [ATQ][HD] output rows
    // One round of loads: (m, l) of the row's chunks (lane-strided) and the first CB chunks of
    // o for this thread's dims; then M, the weights e^(m_c - M) and L.
    constexpr int CB = 16;
    const int nci = row < nq ? (pos0 + i0 + row) / ACH + 1 : 0;
    const size_t base = (size_t(i0 + row) * heads + head) * nc_max;
    float ov[CB][DPT];
#pragma unroll
    for (int k = 0; k < CB; k++)
        if (k < nci) load_dpt<DPT>(ov[k], ro, int(((base + k) * HD + sub * DPT) * 4));
    float inv = 0.0f;
    {
        // (m, l) of chunks sub + 16 u (u < 4) stay in registers; longer contexts reload the rest.
        float mv[4], lv[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int c = sub + 16 * u;
            mv[u] = -INFINITY;
            lv[u] = 0.0f;
            if (c < nci) {
                mv[u] = ld_f32(rm, int((base + c) * 4));
                lv[u] = ld_f32(rl, int((base + c) * 4));
            }
        }
        float M = fmaxf(fmaxf(mv[0], mv[1]), fmaxf(mv[2], mv[3]));
        for (int c = 64 + sub; c < nci; c += 16) M = fmaxf(M, ld_f32(rm, int((base + c) * 4)));
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
        float L = 0.0f;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int c = sub + 16 * u;
            if (c < nci) {
                const float e = expf(mv[u] - M);
                Es[row * nc_max + c] = e;
                L = __builtin_fmaf(lv[u], e, L);
            }
        }
        for (int c = 64 + sub; c < nci; c += 16) {
            const float e = expf(ld_f32(rm, int((base + c) * 4)) - M);
            Es[row * nc_max + c] = e;
            L = __builtin_fmaf(ld_f32(rl, int((base + c) * 4)), e, L);
        }
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) L += __shfl_xor(L, o, 64);
        if (row < nq) inv = 1.0f / L;
    }
    __syncthreads();
    if (row < nq) {
        float o[DPT];
#pragma unroll
        for (int u = 0; u < DPT; u++) o[u] = 0.0f;
#pragma unroll
        for (int k = 0; k < CB; k++)
            if (k < nci) {
                const float e = Es[row * nc_max + k];
#pragma unroll
                for (int u = 0; u < DPT; u++) o[u] = __builtin_fmaf(ov[k][u], e, o[u]);
            }
        for (int c0 = CB; c0 < nci; c0 += 8) {
            float v[8][DPT];
#pragma unroll
            for (int k = 0; k < 8; k++)
                if (c0 + k < nci) load_dpt<DPT>(v[k], ro, int(((base + c0 + k) * HD + sub * DPT) * 4));
#pragma unroll
            for (int k = 0; k < 8; k++)
                if (c0 + k < nci) {
                    const float e = Es[row * nc_max + c0 + k];
#pragma unroll
                    for (int u = 0; u < DPT; u++) o[u] = __builtin_fmaf(v[k][u], e, o[u]);
                }
        }
#pragma unroll
        for (int u = 0; u < DPT; u++) Os[row * HD + sub * DPT + u] = o[u] * inv;
    }
    __syncthreads();
    uint8_t* tf = frags + size_t(tile) * frag_stride;
    for (int p = tid; p < nq * (HD / 8); p += 256) {
        const int i = p / (HD / 8), sl = p % (HD / 8), col = head * HD + 8 * sl;
        write_slot(tf, col / 32, i + 16 * ((col % 32) / 8), Os + i * HD + 8 * sl);
    }
}

size_t attention_scratch_floats(int t, int heads, int hd, int max_ctx) {
    const size_t nc = (size_t(max_ctx) + ACH - 1) / ACH;
    return size_t(t) * heads * nc * (hd + 2);
}

int attention_splits(int max_ctx) {
    const int nc = (max_ctx + ACH - 1) / ACH;
    return nc < 32 ? nc : 32;
}

template <int HD>
static void launch_attn(const float* q, int ldq, int t, int heads, int kv_heads, const int* pos0, int max_ctx, const float* kc,
                        const float* vc, float* scratch, int* cnt, int splits, uint8_t* frags, hipStream_t s) {
    const int nc_max = (max_ctx + ACH - 1) / ACH;
    float* pm = scratch;
    float* pl = pm + size_t(t) * heads * nc_max;
    float* po = pl + size_t(t) * heads * nc_max;
    using LY = AttnLds<HD>;
    const size_t combine = size_t(ATQ) * nc_max + size_t(ATQ) * HD;
    const size_t lds = sizeof(float) * (size_t(LY::END) > combine ? size_t(LY::END) : combine);
    if (lds > 150 * 1024) throw std::runtime_error("attention context too long for the combine buffer");
    const float scale = 1.0f / sqrtf(float(HD));
    hipLaunchKernelGGL(k_attn<HD>, dim3(splits, heads, (t + ATQ - 1) / ATQ), dim3(256), lds, s, q, ldq, t, heads, kv_heads, pos0,
                       scale, kc, vc, nc_max, pm, pl, po, cnt, frags, frag_tile_bytes(heads * HD));
    HIPCHECK(hipGetLastError());
}

void attention(const float* q, int ldq, int t, int heads, int kv_heads, int hd, const int* pos0, int max_ctx, const float* k_cache,
               const float* v_cache, float* scratch, int* cnt, int splits, uint8_t* frags, hipStream_t s) {
    if (splits < 1) throw std::runtime_error("attention needs at least one split");
    switch (hd) {
        case 16: launch_attn<16>(q, ldq, t, heads, kv_heads, pos0, max_ctx, k_cache, v_cache, scratch, cnt, splits, frags, s); break;
        case 32: launch_attn<32>(q, ldq, t, heads, kv_heads, pos0, max_ctx, k_cache, v_cache, scratch, cnt, splits, frags, s); break;
        case 64: launch_attn<64>(q, ldq, t, heads, kv_heads, pos0, max_ctx, k_cache, v_cache, scratch, cnt, splits, frags, s); break;
        case 128: launch_attn<128>(q, ldq, t, heads, kv_heads, pos0, max_ctx, k_cache, v_cache, scratch, cnt, splits, frags, s); break;
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
