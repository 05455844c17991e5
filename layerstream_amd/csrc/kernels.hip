// Small device kernels of the verify step for gfx950 (CDNA4, wave64): attention and the
// embedding helpers of streamed tables. The weight-streaming kernels live in fused.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
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
// Causal GQA attention (src/model.rs:261-282), flash-decoding over chunks of ACH keys. The
// reference computes scores (q . k_j) * scale, a softmax (max, exp(x - max), sum, * 1/sum) and
// sum_j p_j v_j over every cached position.
//
// One launch: grid (ASPLIT, heads, row segments). A segment is a run of at most 16 consecutive
// rows of one sequence inside one 16-row tile: every token tile of a single sequence, or the
// pieces of a batch of sequences cut at tile boundaries. Workgroup s takes chunks s,
// s + ASPLIT, ... of its (head, segment) in order and keeps a running (max, sum, output) per
// token (online softmax); the last of the ASPLIT workgroups to finish (an agent-scope counter)
// merges their states in workgroup order and writes the output rows as fragments. Scores and the weighted
// sum run on v_mfma_f32_16x16x4f32 (f32 products and sums): scores as [keys][tokens], one
// 16-key block per wavefront; the output as [dims][tokens], one 16-dim block per wavefront.
// Which chunks a workgroup takes depends only on key positions and ASPLIT, so a token's result
// does not depend on how many tokens share the launch. The grid does not depend on the
// position (read from the device), so the launch can be replayed from a graph.
// ---------------------------------------------------------------------------------------
constexpr int ACH = 64;    // keys per chunk
constexpr int ATQ = 16;    // query tokens per tile
constexpr int ASPLIT = 8;  // workgroups per (head, tile)
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
__device__ __forceinline__ void st_f32x4(f32x4 v, __amdgpu_buffer_rsrc_t r, int at) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, at, 0, CPOL_SC1);
}
__device__ __forceinline__ f32x4 ld_f32x4(__amdgpu_buffer_rsrc_t r, int at) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, at, 0, CPOL_SC1));
}

__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

// Row paddings keep the MFMA operand reads free of LDS bank conflicts: K and Q rows are read
// as float4 by 16 lanes of consecutive rows (stride HD + 4), V rows by lane groups g on rows
// 4 u + g (stride HD + 16).
template <int HD>
struct AttnLds {
    static constexpr int KP = HD + 4, VP = HD + 16, QP = HD + 4;
    static constexpr int K = 0, V = K + ACH * KP, Q = V + ACH * VP, P = Q + ATQ * QP, R = P + ACH * ATQ, END = R + 2 * 4 * ATQ;
};

// Segment z: without a table, token tile z of one sequence whose row 0 sits at *pos0; with
// one, segs[z] = (first row, rows, sequence, -) and each row's position is rows.pos[row].
template <int HD>
__global__ __launch_bounds__(256) void k_attn(const float* __restrict__ q, int ldq, int t, int heads, int kv_heads,
                                              const int* __restrict__ pos0p, AttnRows rows, float scale, const float* __restrict__ kc,
                                              const float* __restrict__ vc, float* pm, float* pl, float* po, int* cnt,
                                              uint8_t* __restrict__ frags, size_t frag_stride) {
    using LY = AttnLds<HD>;
    constexpr int KP = LY::KP, VP = LY::VP, QP = LY::QP, H4 = HD / 4;
    constexpr int DB = HD / 16;                  // 16-dim blocks
    constexpr int DBW = (DB + 3) / 4;            // dim blocks per wavefront
    constexpr int NP = (ACH * H4 + 255) / 256;   // float4 pieces of K (and of V) per thread
    extern __shared__ __align__(16) float sm[];
    __shared__ int flag;
    float* Ks = sm + LY::K;
    float* Vs = sm + LY::V;
    float* Qs = sm + LY::Q;
    float* Ps = sm + LY::P;   // [key][token]
    float* Rm = sm + LY::R;   // [wave][token] chunk maxima
    float* Rl = Rm + 4 * ATQ; // [wave][token] chunk sums
    const int s = blockIdx.x, head = blockIdx.y, seg = blockIdx.z;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, tok = lane & 15, g = lane >> 4;
    const int kv = kv_heads * HD, grp = head / (heads / kv_heads);
    int i0, nq, pos_first;  // first launch row, rows, position of the first row
    if (rows.segs) {
        const int4 sg = rows.segs[seg];
        i0 = sg.x;
        nq = sg.y;
        pos_first = rows.pos[i0];
        kc += size_t(sg.z) * rows.seq_stride;
        vc += size_t(sg.z) * rows.seq_stride;
    } else {
        i0 = seg * ATQ;
        nq = min(ATQ, t - i0);
        pos_first = *pos0p + i0;
    }
    const int tile = i0 / ATQ, tok0 = i0 % ATQ;  // fragment tile and token of the first row
    const int last_key = pos_first + nq - 1;
    const int nc = last_key / ACH + 1;
    const size_t rows_total = size_t(t) * heads;
    const __amdgpu_buffer_rsrc_t rm = coherent_rsrc(pm, rows_total * ASPLIT * 4);
    const __amdgpu_buffer_rsrc_t rl = coherent_rsrc(pl, rows_total * ASPLIT * 4);
    const __amdgpu_buffer_rsrc_t ro = coherent_rsrc(po, rows_total * ASPLIT * HD * 4);

    auto load_kv = [&](int c, float4* kx, float4* vx) {
        const int j0 = c * ACH, nk = min(ACH, last_key + 1 - j0);
#pragma unroll
        for (int u = 0; u < NP; u++) {
            const int p = tid + u * 256, j = p / H4, d = 4 * (p % H4);
            kx[u] = vx[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (p < ACH * H4 && j < nk) {
                kx[u] = *reinterpret_cast<const float4*>(kc + size_t(j0 + j) * kv + grp * HD + d);
                vx[u] = *reinterpret_cast<const float4*>(vc + size_t(j0 + j) * kv + grp * HD + d);
            }
        }
    };
    float4 kx[NP], vx[NP];
    if (s < nc) load_kv(s, kx, vx);
    for (int p = tid; p < ATQ * H4; p += 256) {
        const int i = p / H4, d = 4 * (p % H4);
        *reinterpret_cast<float4*>(Qs + i * QP + d) =
            i < nq ? *reinterpret_cast<const float4*>(q + size_t(i0 + i) * ldq + head * HD + d) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }

    // Running state of token `tok` (every lane of that token holds the same M and L).
    float M = -INFINITY, L = 0.0f;
    f32x4 O[DBW];
#pragma unroll
    for (int b = 0; b < DBW; b++) O[b] = f32x4{0, 0, 0, 0};

    for (int c = s; c < nc; c += ASPLIT) {
        const int j0 = c * ACH, nk = min(ACH, last_key + 1 - j0);
        __syncthreads();  // the previous chunk is done with Ks, Vs, Ps
#pragma unroll
        for (int u = 0; u < NP; u++) {
            const int p = tid + u * 256, j = p / H4, d = 4 * (p % H4);
            if (p < ACH * H4) {
                *reinterpret_cast<float4*>(Ks + j * KP + d) = kx[u];
                *reinterpret_cast<float4*>(Vs + j * VP + d) = vx[u];
            }
        }
        __syncthreads();
        if (c + ASPLIT < nc) load_kv(c + ASPLIT, kx, vx);  // in flight during this chunk

        // Scores [key 16 w + 4 g + i][token]: lane group g supplies dims g H4 + [0, H4).
        f32x4 sc = {0, 0, 0, 0};
#pragma unroll
        for (int d = 0; d < H4; d += 4) {
            const float4 k4 = *reinterpret_cast<const float4*>(Ks + (16 * w + tok) * KP + g * H4 + d);
            const float4 q4 = *reinterpret_cast<const float4*>(Qs + tok * QP + g * H4 + d);
            sc = mfma_f32(k4.x, q4.x, sc);
            sc = mfma_f32(k4.y, q4.y, sc);
            sc = mfma_f32(k4.z, q4.z, sc);
            sc = mfma_f32(k4.w, q4.w, sc);
        }
        // D of that product: lane (g, tok) holds keys 16 w + 4 g + i of token tok.
        float sv[4];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int j = 16 * w + 4 * g + i;
            sv[i] = (tok < nq && j < nk && j0 + j <= pos_first + tok) ? sc[i] * scale : -INFINITY;
            mx = fmaxf(mx, sv[i]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        if (g == 0) Rm[w * ATQ + tok] = mx;
        __syncthreads();
        const float mc = fmaxf(fmaxf(Rm[tok], Rm[ATQ + tok]), fmaxf(Rm[2 * ATQ + tok], Rm[3 * ATQ + tok]));
        const float Mn = fmaxf(M, mc);
        const float corr = M == -INFINITY ? 0.0f : expf(M - Mn);  // rescale of the running state
        float ls = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float e = sv[i] == -INFINITY ? 0.0f : expf(sv[i] - Mn);
            Ps[(16 * w + 4 * g + i) * ATQ + tok] = e;
            ls += e;
        }
        ls += __shfl_xor(ls, 16, 64);
        ls += __shfl_xor(ls, 32, 64);
        if (g == 0) Rl[w * ATQ + tok] = ls;
        __syncthreads();
        const float lc = ((Rl[tok] + Rl[ATQ + tok]) + Rl[2 * ATQ + tok]) + Rl[3 * ATQ + tok];
        L = __builtin_fmaf(L, corr, lc);
        M = Mn;
        // Output [dim][token]: lane group g supplies keys 4 u + g.
#pragma unroll
        for (int b = 0; b < DBW; b++) {
            const int db = w + 4 * b;
            if (db < DB) {
                f32x4 acc = {0, 0, 0, 0};
#pragma unroll
                for (int u = 0; u < 16; u++) {
                    const int key = 4 * u + g;
                    acc = mfma_f32(Vs[key * VP + 16 * db + tok], Ps[key * ATQ + tok], acc);
                }
#pragma unroll
                for (int i = 0; i < 4; i++) O[b][i] = __builtin_fmaf(O[b][i], corr, acc[i]);
            }
        }
    }
    // This workgroup's state: lane (g, tok) of wavefront w holds dims 16 (w + 4 b) + 4 g + [0, 4).
    // O is [dims][tokens] per lane: transpose the lane view. D of the output product: lane l
    // holds dims 16 db + 4 (l / 16) + i of token l % 16.
    if (tok < nq) {
        const size_t row = (size_t(i0 + tok) * heads + head) * ASPLIT + s;
        if (w == 0 && g == 0) {
            st_f32(M, rm, int(row * 4));
            st_f32(L, rl, int(row * 4));
        }
#pragma unroll
        for (int b = 0; b < DBW; b++) {
            const int db = w + 4 * b;
            if (db < DB) st_f32x4(O[b], ro, int((row * HD + 16 * db + 4 * g) * 4));
        }
    }

    // The last workgroup of (head, segment) merges the ASPLIT states in order.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        int* cn = cnt + size_t(seg) * heads + head;
        const int old = __hip_atomic_fetch_add(cn, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = old == ASPLIT - 1;
        if (last) __hip_atomic_store(cn, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        flag = last;
    }
    __syncthreads();
    if (!flag) return;
    constexpr int DPT = HD / 16;  // dims per thread: thread (row, sub) takes sub * DPT ..
    float* Os = sm;               // [ATQ][HD] output rows
    const int row = tid >> 4, sub = tid & 15;
    if (row < nq) {
        const size_t base = (size_t(i0 + row) * heads + head) * ASPLIT;
        float mv[ASPLIT], lv[ASPLIT], ov[ASPLIT][DPT];
#pragma unroll
        for (int k = 0; k < ASPLIT; k++) {
            mv[k] = ld_f32(rm, int((base + k) * 4));
            lv[k] = ld_f32(rl, int((base + k) * 4));
            if constexpr (DPT % 4 == 0) {
#pragma unroll
                for (int u = 0; u < DPT; u += 4) {
                    const f32x4 x = ld_f32x4(ro, int(((base + k) * HD + sub * DPT + u) * 4));
                    ov[k][u] = x[0];
                    ov[k][u + 1] = x[1];
                    ov[k][u + 2] = x[2];
                    ov[k][u + 3] = x[3];
                }
            } else {
#pragma unroll
                for (int u = 0; u < DPT; u++) ov[k][u] = ld_f32(ro, int(((base + k) * HD + sub * DPT + u) * 4));
            }
        }
        float Mx = -INFINITY;
#pragma unroll
        for (int k = 0; k < ASPLIT; k++) Mx = fmaxf(Mx, mv[k]);
        float Lt = 0.0f, o[DPT];
#pragma unroll
        for (int u = 0; u < DPT; u++) o[u] = 0.0f;
#pragma unroll
        for (int k = 0; k < ASPLIT; k++) {
            const float e = mv[k] == -INFINITY ? 0.0f : expf(mv[k] - Mx);
            Lt = __builtin_fmaf(lv[k], e, Lt);
#pragma unroll
            for (int u = 0; u < DPT; u++) o[u] = __builtin_fmaf(ov[k][u], e, o[u]);
        }
        const float inv = 1.0f / Lt;
#pragma unroll
        for (int u = 0; u < DPT; u++) Os[row * HD + sub * DPT + u] = o[u] * inv;
    }
    __syncthreads();
    uint8_t* tf = frags + size_t(tile) * frag_stride;
    for (int p = tid; p < nq * (HD / 8); p += 256) {
        const int i = p / (HD / 8), sl = p % (HD / 8), col = head * HD + 8 * sl;
        write_slot(tf, col / 32, tok0 + i + 16 * ((col % 32) / 8), Os + i * HD + 8 * sl);
    }
}

size_t attention_scratch_floats(int t, int heads, int hd, int) { return size_t(t) * heads * ASPLIT * (hd + 2); }

template <int HD>
static void launch_attn(const float* q, int ldq, int t, int heads, int kv_heads, const int* pos0, const AttnRows& rows,
                        const float* kc, const float* vc, float* scratch, int* cnt, uint8_t* frags, hipStream_t s) {
    float* pm = scratch;
    float* pl = pm + size_t(t) * heads * ASPLIT;
    float* po = pl + size_t(t) * heads * ASPLIT;
    using LY = AttnLds<HD>;
    const size_t lds = sizeof(float) * size_t(LY::END);
    const float scale = 1.0f / sqrtf(float(HD));
    const int nseg = rows.segs ? rows.n_segs : (t + ATQ - 1) / ATQ;
    hipLaunchKernelGGL(k_attn<HD>, dim3(ASPLIT, heads, nseg), dim3(256), lds, s, q, ldq, t, heads, kv_heads, pos0, rows,
                       scale, kc, vc, pm, pl, po, cnt, frags, frag_tile_bytes(heads * HD));
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
