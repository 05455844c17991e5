// Attention device code (included by kernels.hip and fused.hip). Only for .hip sources.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <type_traits>

#include "frag_dev.hpp"
#include "fused.hpp"
#include "kernels.hpp"

namespace ls {

// ---------------------------------------------------------------------------------------
// Causal GQA attention (src/model.rs:261-282), flash-decoding. The reference computes scores
// (q . k_j) * scale, a softmax (max, exp(x - max), sum, * 1/sum) and sum_j p_j v_j over every
// cached position.
//
// One launch: grid (ASPLIT, heads, row segments) of AWV-wavefront workgroups. A segment is a run
// of at most 16 consecutive rows of one sequence: every token tile of a single sequence, or, in a
// batch, a sequence's rows in pieces of 16 from its first row (a piece may straddle two tiles; each
// row's output goes to its own tile). A row's result depends only on its own query and keys. The keys are
// cut into 16-key blocks; block b belongs to wavefront b % (AWV ASPLIT) of the (head, segment)
// (workgroup (b % (AWV ASPLIT)) / AWV), which keeps a running (max, sum, output) per token over its
// blocks in order (online softmax) without any barrier: the scores ([keys][tokens]) and the
// weighted sum ([dims][tokens]) run on v_mfma_f32_16x16x4f32 straight from registers, each lane
// loading the K, V and q values it feeds. With AWV ASPLIT = 64 wavefronts per (head, segment) a
// wavefront owns at most a few blocks at these contexts, so one block's registers are loaded at a
// time: the second buffer would cost the occupancy that batched launches need. The AWV
// wavefronts' states merge in LDS in wavefront order, and the last of the ASPLIT workgroups to
// finish (an agent-scope counter) merges theirs in workgroup order and writes the output rows as
// fragments. Which blocks a wavefront takes depends only on key positions, so a token's result
// does not depend on how many tokens share the launch. The grid does not depend on the position
// (read from the device), so the launch can be replayed from a graph.
// ---------------------------------------------------------------------------------------
constexpr int AKB = 16;    // keys per block
constexpr int ATQ = 16;    // query tokens per tile
constexpr int AWV = 8;     // wavefronts per workgroup
constexpr int ASPLIT = ATTN_SPLIT;
typedef float attn_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t attn_u32x4 __attribute__((ext_vector_type(4)));

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
__device__ __forceinline__ void st_attn_f32x4(attn_f32x4 v, __amdgpu_buffer_rsrc_t r, int at) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(attn_u32x4, v), r, at, 0, CPOL_SC1);
}
__device__ __forceinline__ attn_f32x4 ld_attn_f32x4(__amdgpu_buffer_rsrc_t r, int at) {
    return __builtin_bit_cast(attn_f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, at, 0, CPOL_SC1));
}

__device__ __forceinline__ attn_f32x4 mfma_f32(float a, float b, attn_f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

// MFMA operand layout (16x16x4 f32): lane l = 16 g + c supplies A[m = c][k = g] and B[k = g][n = c]
// and receives D[m = 4 g + i][n = c], i < 4.
//
// Scores of block b, MFMA j < HD / 4: A = K[key 16 b + c][g HD/4 + j], B = q[token c][g HD/4 + j],
// so lane (g, c) holds HD/4 consecutive floats of key row c and of query row c, and receives
// the scores of keys 16 b + 4 g + i for token c. Weighted sum, output block db < DB = HD / 16,
// MFMA u < 4: the keys of its K dimension are 16 b + 4 g + u, so B = p[16 b + 4 g + u][c] is the
// lane's own score register u; its rows are dims DB m + db (m < 16), so A = V[16 b + 4 g + u]
// [DB c + db] (lane (g, c) loads DB consecutive floats per key) and lane (g, c) receives dims
// DB (4 g + i) + db of token c.
template <int HD>
struct AttnBlock {
    static constexpr int H4 = HD / 4, DB = HD / 16;
    float k[H4];
    float v[4 * DB];
};

template <int HD>
__device__ __forceinline__ void attn_load(AttnBlock<HD>& r, int b, int last_key, const float* __restrict__ kc,
                                          const float* __restrict__ vc, int kv, int col0, int g, int c) {
    constexpr int H4 = HD / 4, DB = HD / 16;
    const int key = AKB * b + c;
    if (key <= last_key) {
        const float* kp = kc + size_t(key) * kv + col0 + g * H4;
#pragma unroll
        for (int j = 0; j < H4; j += 4) {
            const float4 x = *reinterpret_cast<const float4*>(kp + j);
            r.k[j] = x.x;
            r.k[j + 1] = x.y;
            r.k[j + 2] = x.z;
            r.k[j + 3] = x.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < H4; j++) r.k[j] = 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int vk = AKB * b + 4 * g + u;
        const float* vp = vc + size_t(vk) * kv + col0 + DB * c;
        if constexpr (DB % 4 == 0) {
#pragma unroll
            for (int db = 0; db < DB; db += 4) {
                const float4 x = vk <= last_key ? *reinterpret_cast<const float4*>(vp + db) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                r.v[u * DB + db] = x.x;
                r.v[u * DB + db + 1] = x.y;
                r.v[u * DB + db + 2] = x.z;
                r.v[u * DB + db + 3] = x.w;
            }
        } else {
#pragma unroll
            for (int db = 0; db < DB; db++) r.v[u * DB + db] = vk <= last_key ? vp[db] : 0.0f;
        }
    }
}

// attn_load through the coherent path, for key rows written earlier in the same launch: rk and
// rv cover the caches from kc / vc.
template <int HD>
__device__ __forceinline__ void attn_load_coherent(AttnBlock<HD>& r, int b, int last_key, __amdgpu_buffer_rsrc_t rk,
                                                   __amdgpu_buffer_rsrc_t rv, int kv, int col0, int g, int c) {
    constexpr int H4 = HD / 4, DB = HD / 16;
    const int key = AKB * b + c;
#pragma unroll
    for (int j = 0; j < H4; j += 4) {
        const attn_f32x4 x = key <= last_key ? ld_attn_f32x4(rk, (key * kv + col0 + g * H4 + j) * 4) : attn_f32x4{0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 4; e++) r.k[j + e] = x[e];
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int vk = AKB * b + 4 * g + u;
        if constexpr (DB % 4 == 0) {
#pragma unroll
            for (int db = 0; db < DB; db += 4) {
                const attn_f32x4 x = vk <= last_key ? ld_attn_f32x4(rv, (vk * kv + col0 + DB * c + db) * 4) : attn_f32x4{0, 0, 0, 0};
#pragma unroll
                for (int e = 0; e < 4; e++) r.v[u * DB + db + e] = x[e];
            }
        } else {
#pragma unroll
            for (int db = 0; db < DB; db++) r.v[u * DB + db] = vk <= last_key ? ld_f32(rv, (vk * kv + col0 + DB * c + db) * 4) : 0.0f;
        }
    }
}

// The arguments of one attention launch (see attention() in kernels.hpp); pm, pl, po are the
// per-workgroup states in the scratch buffer.
struct AttnArgs {
    const float* q;
    int ldq, t, heads, kv_heads;
    const int* pos0p;
    AttnRows rows;
    float scale;
    const float* kc;
    const float* vc;
    float *pm, *pl, *po;
    int* cnt;
    uint8_t* frags;
    size_t frag_stride;
};

inline AttnArgs make_attn_args(const float* q, int ldq, int t, int heads, int kv_heads, int hd, const int* pos0, const AttnRows& rows,
                               const float* kc, const float* vc, float* scratch, int* cnt, uint8_t* frags) {
    AttnArgs a;
    a.q = q;
    a.ldq = ldq;
    a.t = t;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.pos0p = pos0;
    a.rows = rows;
    a.scale = 1.0f / sqrtf(float(hd));
    a.kc = kc;
    a.vc = vc;
    a.pm = scratch;
    a.pl = a.pm + size_t(t) * heads * ASPLIT;
    a.po = a.pl + size_t(t) * heads * ASPLIT;
    a.cnt = cnt;
    a.frags = frags;
    a.frag_stride = frag_tile_bytes(heads * hd);
    return a;
}

// Workgroup s of (head, segment seg) (256 threads). With OUT_FLOW the output fragments are
// written through the coherent path and the merging workgroup then signals fl (producer 0).
// With IN_FLOW (one sequence) q and the keys from the launch's first position on are written by
// earlier workgroups of the same launch: the workgroup loads its first block if it holds only
// older keys, waits on fin (counter `head`), then reads q and newer keys coherently.
// LDS of one attention workgroup: per-wavefront (max, sum) and outputs, then a flag.
template <int HD>
__host__ __device__ constexpr size_t attn_lds_bytes() { return size_t(2 * AWV * ATQ + AWV * ATQ * (HD + 4)) * 4 + 16; }

template <int HD, bool OUT_FLOW, bool IN_FLOW = false>
__device__ __forceinline__ void attn_body(const AttnArgs& A, int s, int head, int seg, const Flow& fl, uint8_t* smem,
                                          const Flow& fin = Flow{}) {
    const float* __restrict__ q = A.q;
    const int ldq = A.ldq, t = A.t, heads = A.heads, kv_heads = A.kv_heads;
    const AttnRows& rows = A.rows;
    const float scale = A.scale;
    const float* __restrict__ kc = A.kc;
    const float* __restrict__ vc = A.vc;
    float* pm = A.pm;
    float* pl = A.pl;
    float* po = A.po;
    uint8_t* __restrict__ frags = A.frags;
    const size_t frag_stride = A.frag_stride;
    constexpr int H4 = HD / 4, DB = HD / 16;
    // In the workgroup's LDS (attn_lds_bytes<HD>() from smem; a fused launch shares it with its
    // matrix roles, one role per workgroup).
    float(*sm_m)[ATQ] = reinterpret_cast<float(*)[ATQ]>(smem);
    float(*sm_l)[ATQ] = reinterpret_cast<float(*)[ATQ]>(smem + AWV * ATQ * 4);
    constexpr int HP = HD + 4;  // padded row of the wavefront outputs
    float* sm_o = reinterpret_cast<float*>(smem + 2 * AWV * ATQ * 4);  // wavefront outputs [wave][token][dim], then the output rows
    int& flag = *reinterpret_cast<int*>(smem + 2 * AWV * ATQ * 4 + AWV * ATQ * HP * 4);
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
    const int kv = kv_heads * HD, col0 = (head / (heads / kv_heads)) * HD;
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
        pos_first = *A.pos0p + i0;
    }
    const int tile = i0 / ATQ, tok0 = i0 % ATQ;  // fragment tile and token of the first row
    const int last_key = pos_first + nq - 1;
    const int nb = last_key / AKB + 1;
    const int first = s * AWV + w, stride = ASPLIT * AWV;
    // Splits whose first block is past the last key hold nothing: their state would be
    // (-inf, 0, 0), which the final merge adds exactly nothing from. In a launch of its own
    // (no flows) such a workgroup leaves at once and the merge counts only the live ones.
    constexpr bool SKIP = !OUT_FLOW && !IN_FLOW;
    const int live = SKIP ? min(ASPLIT, (nb + AWV - 1) / AWV) : ASPLIT;
    if (SKIP && s >= live) return;
    const size_t rows_total = size_t(t) * heads;
    const __amdgpu_buffer_rsrc_t rm = coherent_rsrc(pm, rows_total * ASPLIT * 4);
    const __amdgpu_buffer_rsrc_t rl = coherent_rsrc(pl, rows_total * ASPLIT * 4);
    const __amdgpu_buffer_rsrc_t ro = coherent_rsrc(po, rows_total * ASPLIT * HD * 4);

    AttnBlock<HD> ba;
    float qr[H4];
    // Blocks below nold hold only keys cached before this launch (every block without IN_FLOW).
    const int nold = IN_FLOW ? *A.pos0p / AKB : nb;
    const __amdgpu_buffer_rsrc_t rk = coherent_rsrc(kc, size_t(last_key + 1) * kv * 4);
    const __amdgpu_buffer_rsrc_t rv = coherent_rsrc(vc, size_t(last_key + 1) * kv * 4);
    auto load_block = [&](AttnBlock<HD>& r, int b) {
        if (IN_FLOW && b >= nold) attn_load_coherent<HD>(r, b, last_key, rk, rv, kv, col0, g, c);
        else attn_load<HD>(r, b, last_key, kc, vc, kv, col0, g, c);
    };
    if (first < nb && first < nold) load_block(ba, first);
    // In a fused launch (IN_FLOW) the wavefront's second block of cached keys is requested before
    // the wait too, so long contexts (two blocks per wavefront from 1024 keys) meet no load after
    // the input arrives (0.5B int4 after a 2048-token prompt: 0.879 -> 0.866 ms per verify step;
    // 3B int8 after 1024: 2.381 -> 2.361 ms).
    constexpr bool PF2 = IN_FLOW && HD <= 128;
    AttnBlock<HD> bb;
    const int second = first + stride;
    if constexpr (PF2)
        if (second < nb && second < nold) load_block(bb, second);
    if constexpr (IN_FLOW) {
        flow_wait(fin, head, s);
        if (first < nb && first >= nold) load_block(ba, first);
        const __amdgpu_buffer_rsrc_t rq = coherent_rsrc(q, size_t(t) * ldq * 4);
#pragma unroll
        for (int j = 0; j < H4; j += 4) {
            const attn_f32x4 x = c < nq ? ld_attn_f32x4(rq, ((i0 + c) * ldq + head * HD + g * H4 + j) * 4) : attn_f32x4{0, 0, 0, 0};
#pragma unroll
            for (int e = 0; e < 4; e++) qr[j + e] = x[e];
        }
    } else {
        const float* qp = q + size_t(i0 + c) * ldq + head * HD + g * H4;
#pragma unroll
        for (int j = 0; j < H4; j += 4) {
            const float4 x = c < nq ? *reinterpret_cast<const float4*>(qp + j) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            qr[j] = x.x;
            qr[j + 1] = x.y;
            qr[j + 2] = x.z;
            qr[j + 3] = x.w;
        }
    }

    // Running state of token c: M (the same in the four lanes of the token), this lane's share
    // of the sum (keys 16 b + 4 g + i), and output dims 16 db + 4 g + i.
    float M = -INFINITY, Lp = 0.0f;
    attn_f32x4 O[DB];
#pragma unroll
    for (int db = 0; db < DB; db++) O[db] = attn_f32x4{0, 0, 0, 0};
    auto block = [&](int b, const AttnBlock<HD>& r) {
        attn_f32x4 sc = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < H4; j++) sc = mfma_f32(r.k[j], qr[j], sc);
        float sv[4];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int key = AKB * b + 4 * g + i;
            sv[i] = (c < nq && key <= pos_first + c) ? sc[i] * scale : -INFINITY;
            mx = fmaxf(mx, sv[i]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float Mn = fmaxf(M, mx);
        const float corr = M == -INFINITY ? 0.0f : expf(M - Mn);  // rescale of the running state
        float p[4], ls = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            p[i] = sv[i] == -INFINITY ? 0.0f : expf(sv[i] - Mn);
            ls += p[i];
        }
        Lp = __builtin_fmaf(Lp, corr, ls);
        M = Mn;
#pragma unroll
        for (int db = 0; db < DB; db++) {
            attn_f32x4 acc = {0, 0, 0, 0};
#pragma unroll
            for (int u = 0; u < 4; u++) acc = mfma_f32(r.v[u * DB + db], p[u], acc);
#pragma unroll
            for (int i = 0; i < 4; i++) O[db][i] = __builtin_fmaf(O[db][i], corr, acc[i]);
        }
    };
    for (int b = first; b < nb; b += stride) {
        if constexpr (PF2) {
            if (b == second) {
                if (b >= nold) load_block(bb, b);
                block(b, bb);
                continue;
            }
        }
        if (b != first) load_block(ba, b);
        block(b, ba);
    }

    // The AWV wavefronts' states, merged in wavefront order into this workgroup's state.
    float L = Lp + __shfl_xor(Lp, 16, 64);
    L += __shfl_xor(L, 32, 64);
    if (g == 0) {
        sm_m[w][c] = M;
        sm_l[w][c] = L;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float* dst = &sm_o[(w * ATQ + c) * HP + DB * (4 * g + i)];  // dims DB (4 g + i) + [0, DB)
        if constexpr (DB % 4 == 0) {
#pragma unroll
            for (int db = 0; db < DB; db += 4)
                *reinterpret_cast<attn_f32x4*>(dst + db) = attn_f32x4{O[db][i], O[db + 1][i], O[db + 2][i], O[db + 3][i]};
        } else {
#pragma unroll
            for (int db = 0; db < DB; db++) dst[db] = O[db][i];
        }
    }
    __syncthreads();
    for (int e = tid; e < ATQ * (HD / 4); e += AWV * 64) {
        const int tk = e % ATQ, d = 4 * (e / ATQ);
        if (tk >= nq) continue;
        float mw[AWV], Mx = -INFINITY;
#pragma unroll
        for (int k = 0; k < AWV; k++) {
            mw[k] = sm_m[k][tk];
            Mx = fmaxf(Mx, mw[k]);
        }
        float Lw = 0.0f;
        attn_f32x4 ow = {0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < AWV; k++) {
            const float e2 = mw[k] == -INFINITY ? 0.0f : expf(mw[k] - Mx);
            Lw = __builtin_fmaf(sm_l[k][tk], e2, Lw);
            const attn_f32x4 x = *reinterpret_cast<const attn_f32x4*>(&sm_o[(k * ATQ + tk) * HP + d]);
#pragma unroll
            for (int i = 0; i < 4; i++) ow[i] = __builtin_fmaf(x[i], e2, ow[i]);
        }
        const size_t row = (size_t(i0 + tk) * heads + head) * ASPLIT + s;
        if (d == 0) {
            st_f32(Mx, rm, int(row * 4));
            st_f32(Lw, rl, int(row * 4));
        }
        st_attn_f32x4(ow, ro, int((row * HD + d) * 4));
    }

    // The last workgroup of (head, segment) merges the ASPLIT states in order.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        int* cn = A.cnt + size_t(seg) * heads + head;
        const int old = __hip_atomic_fetch_add(cn, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = old == live - 1;
        if (last) __hip_atomic_store(cn, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        flag = last;
    }
    __syncthreads();
    if (!flag) return;
    constexpr int DPT = HD / 16;  // dims per thread: thread (row, sub) takes sub * DPT ..
    float* Os = sm_o;             // [ATQ][HD] output rows
    const int row = tid >> 4, sub = tid & 15;
    if (row < nq) {
        const size_t base = (size_t(i0 + row) * heads + head) * ASPLIT;
        float mv[ASPLIT], lv[ASPLIT], ov[ASPLIT][DPT];
#pragma unroll
        for (int k = 0; k < ASPLIT; k++) {
            if (k >= live) {  // a split that held no keys: the state it would have stored
                mv[k] = -INFINITY;
                lv[k] = 0.0f;
#pragma unroll
                for (int u = 0; u < DPT; u++) ov[k][u] = 0.0f;
                continue;
            }
            mv[k] = ld_f32(rm, int((base + k) * 4));
            lv[k] = ld_f32(rl, int((base + k) * 4));
            if constexpr (DPT % 4 == 0) {
#pragma unroll
                for (int u = 0; u < DPT; u += 4) {
                    const attn_f32x4 x = ld_attn_f32x4(ro, int(((base + k) * HD + sub * DPT + u) * 4));
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
    // Row i0 + i goes to token (i0 + i) % 16 of tile (i0 + i) / 16 (a batch segment may straddle
    // two tiles; launches with in-launch consumers run whole tiles).
    uint8_t* tf = frags + size_t(tile) * frag_stride;
    const __amdgpu_buffer_rsrc_t rf = __builtin_amdgcn_make_buffer_rsrc(tf, 0, int(frag_stride), BUF_DWORD3);
    for (int p = tid; p < nq * (HD / 8); p += AWV * 64) {
        const int i = p / (HD / 8), sl = p % (HD / 8), col = head * HD + 8 * sl;
        if constexpr (OUT_FLOW) {
            write_slot_coherent(rf, 0, col / 32, tok0 + i + 16 * ((col % 32) / 8), Os + i * HD + 8 * sl);
        } else {
            const int r = i0 + i;
            write_slot(frags + size_t(r / ATQ) * frag_stride, col / 32, r % ATQ + 16 * ((col % 32) / 8), Os + i * HD + 8 * sl);
        }
    }
    if constexpr (OUT_FLOW) flow_signal(fl, 0);
}

// ---------------------------------------------------------------------------------------
// The same attention with the query heads of a KV group together (a batch's segments): workgroup
// (s, group, segment) takes split s of every head of the group. A wavefront loads its key block's
// K and V once (when it holds one block, as every wavefront does up to 1024 keys) and runs them
// against the group's (head, row) pairs, 16 pairs per MFMA query tile (a 9-row verify block of 7
// heads fills 4 tiles where a head at a time would take 7 of 9 live columns); each tile's states
// are merged over the wavefronts in LDS and stored, and the last of the ASPLIT workgroups of
// (group, segment) merges every pair. Per (head, row) this is attn_body's arithmetic in
// attn_body's order (the same blocks per wavefront, the same two merges; a query column's results
// depend only on its own q), so the bits do not change; the launch has heads / kv_heads times
// fewer workgroups and reads the cache that many times less.
// ---------------------------------------------------------------------------------------
// Pair tiles per pass of a grouped workgroup: the wavefronts' states of two tiles sit in LDS at
// once for head_dim <= 64 (one pair of barriers and one merge pass over all 512 threads for both),
// one tile above (two tiles' states and the staged q do not fit the LDS).
template <int HD>
__host__ __device__ constexpr int attn_grp_tiles() { return HD <= 64 ? 2 : 1; }
// LDS of one pair tile's wavefront states: (max, sum) [AWV][16], outputs [AWV x 16][HD + 4].
template <int HD>
__host__ __device__ constexpr size_t attn_grp_slot_bytes() { return size_t(2 * AWV * ATQ + AWV * ATQ * (HD + 4)) * 4; }
// LDS of a grouped workgroup: attn_grp_tiles slots, the q of up to AWV x 16 (head, row) pairs
// [pair][HD], then a flag.
template <int HD>
__host__ __device__ constexpr size_t attn_grp_lds_bytes() {
    return attn_grp_tiles<HD>() * attn_grp_slot_bytes<HD>() + size_t(AWV) * ATQ * HD * 4 + 16;
}

template <int HD>
__device__ __forceinline__ void attn_group_body(const AttnArgs& A, int s, int grp, int seg, uint8_t* smem) {
    const float* __restrict__ q = A.q;
    const int ldq = A.ldq, t = A.t, heads = A.heads, kv_heads = A.kv_heads, hpg = heads / kv_heads;
    const AttnRows& rows = A.rows;
    const float scale = A.scale;
    const float* __restrict__ kc = A.kc;
    const float* __restrict__ vc = A.vc;
    uint8_t* __restrict__ frags = A.frags;
    const size_t frag_stride = A.frag_stride;
    constexpr int H4 = HD / 4, DB = HD / 16, TP = attn_grp_tiles<HD>(), HP = HD + 4;
    constexpr size_t SLOT = attn_grp_slot_bytes<HD>();
    // Slot u: (max, sum) of each wavefront and query column, then the wavefronts' outputs.
    auto sm_m = [&](int u) { return reinterpret_cast<float(*)[ATQ]>(smem + u * SLOT); };
    auto sm_l = [&](int u) { return reinterpret_cast<float(*)[ATQ]>(smem + u * SLOT + AWV * ATQ * 4); };
    auto sm_o = [&](int u) { return reinterpret_cast<float*>(smem + u * SLOT + 2 * AWV * ATQ * 4); };
    float* sq = reinterpret_cast<float*>(smem + TP * SLOT);
    int& flag = *reinterpret_cast<int*>(smem + TP * SLOT + size_t(AWV) * ATQ * HD * 4);
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
    const int kv = kv_heads * HD, col0 = grp * HD;
    int i0, nq, pos_first;
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
        pos_first = *A.pos0p + i0;
    }
    const int last_key = pos_first + nq - 1;
    const int nb = last_key / AKB + 1;
    const int first = s * AWV + w, stride = ASPLIT * AWV;
    const int live = min(ASPLIT, (nb + AWV - 1) / AWV);  // splits that hold keys (as attn_body)
    if (s >= live) return;
    const bool one_block = first < nb && first + stride >= nb;  // this wavefront's only block: loaded once
    const size_t rows_total = size_t(t) * heads;
    const __amdgpu_buffer_rsrc_t rm = coherent_rsrc(A.pm, rows_total * ASPLIT * 4);
    const __amdgpu_buffer_rsrc_t rl = coherent_rsrc(A.pl, rows_total * ASPLIT * 4);
    const __amdgpu_buffer_rsrc_t ro = coherent_rsrc(A.po, rows_total * ASPLIT * HD * 4);

    AttnBlock<HD> ba;
    if (one_block) attn_load<HD>(ba, first, last_key, kc, vc, kv, col0, g, c);
    // The group's (head, row) pairs, pair hh nq + i = head grp hpg + hh at row i0 + i, fill the
    // 16 query columns of the MFMAs in tiles of 16 (9-row verify blocks of 7 heads: 4 tiles of
    // 16, not 7 of 9). Every pair's q into LDS at once (slots past the pairs: zeros): one round
    // trip to memory for all passes.
    const int npairs = hpg * nq, ptiles = (npairs + ATQ - 1) / ATQ;
    for (int e = tid; e < ptiles * ATQ * (HD / 4); e += AWV * 64) {
        const int pr = e / (HD / 4), d = 4 * (e % (HD / 4));
        float4 x = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (pr < npairs) x = *reinterpret_cast<const float4*>(q + size_t(i0 + pr % nq) * ldq + (grp * hpg + pr / nq) * HD + d);
        *reinterpret_cast<float4*>(sq + pr * HD + d) = x;
    }
    __syncthreads();
    // NT pair tiles from pt0: each wavefront's states of them over its blocks in order, then
    // their merge over the wavefronts in wavefront order (as attn_body), NT tiles per pair of
    // barriers. The tiles' chains are independent, so their MFMAs interleave.
    auto pair_tiles = [&](int pt0, auto nt) {
        constexpr int NT = decltype(nt)::value;
        float qr[NT][H4], M[NT], Lp[NT];
        int pos_c[NT];
        bool live_c[NT];
        attn_f32x4 O[NT][DB];
#pragma unroll
        for (int u = 0; u < NT; u++) {
            // Query column c: pair (pt0 + u) 16 + c, its row at position pos_first + row.
            const int pc = (pt0 + u) * ATQ + c;
            live_c[u] = pc < npairs;
            pos_c[u] = pos_first + pc % nq;
#pragma unroll
            for (int j = 0; j < H4; j += 4) {
                const float4 x = *reinterpret_cast<const float4*>(sq + pc * HD + g * H4 + j);
                qr[u][j] = x.x;
                qr[u][j + 1] = x.y;
                qr[u][j + 2] = x.z;
                qr[u][j + 3] = x.w;
            }
            M[u] = -INFINITY;
            Lp[u] = 0.0f;
#pragma unroll
            for (int db = 0; db < DB; db++) O[u][db] = attn_f32x4{0, 0, 0, 0};
        }
        auto block = [&](int b, const AttnBlock<HD>& r) {
#pragma unroll
            for (int u = 0; u < NT; u++) {
                attn_f32x4 sc = {0, 0, 0, 0};
#pragma unroll
                for (int j = 0; j < H4; j++) sc = mfma_f32(r.k[j], qr[u][j], sc);
                float sv[4];
                float mx = -INFINITY;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int key = AKB * b + 4 * g + i;
                    sv[i] = (live_c[u] && key <= pos_c[u]) ? sc[i] * scale : -INFINITY;
                    mx = fmaxf(mx, sv[i]);
                }
                mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
                mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                const float Mn = fmaxf(M[u], mx);
                const float corr = M[u] == -INFINITY ? 0.0f : expf(M[u] - Mn);
                float p[4], ls = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    p[i] = sv[i] == -INFINITY ? 0.0f : expf(sv[i] - Mn);
                    ls += p[i];
                }
                Lp[u] = __builtin_fmaf(Lp[u], corr, ls);
                M[u] = Mn;
#pragma unroll
                for (int db = 0; db < DB; db++) {
                    attn_f32x4 acc = {0, 0, 0, 0};
#pragma unroll
                    for (int k = 0; k < 4; k++) acc = mfma_f32(r.v[k * DB + db], p[k], acc);
#pragma unroll
                    for (int i = 0; i < 4; i++) O[u][db][i] = __builtin_fmaf(O[u][db][i], corr, acc[i]);
                }
            }
        };
        if (one_block) {
            block(first, ba);
        } else {
            for (int b = first; b < nb; b += stride) {
                AttnBlock<HD> r;
                attn_load<HD>(r, b, last_key, kc, vc, kv, col0, g, c);
                block(b, r);
            }
        }
#pragma unroll
        for (int u = 0; u < NT; u++) {
            float L = Lp[u] + __shfl_xor(Lp[u], 16, 64);
            L += __shfl_xor(L, 32, 64);
            if (g == 0) {
                sm_m(u)[w][c] = M[u];
                sm_l(u)[w][c] = L;
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float* dst = &sm_o(u)[(w * ATQ + c) * HP + DB * (4 * g + i)];
                if constexpr (DB % 4 == 0) {
#pragma unroll
                    for (int db = 0; db < DB; db += 4)
                        *reinterpret_cast<attn_f32x4*>(dst + db) = attn_f32x4{O[u][db][i], O[u][db + 1][i], O[u][db + 2][i], O[u][db + 3][i]};
                } else {
#pragma unroll
                    for (int db = 0; db < DB; db++) dst[db] = O[u][db][i];
                }
            }
        }
        __syncthreads();
        for (int e = tid; e < NT * ATQ * (HD / 4); e += AWV * 64) {
            const int u = e / (ATQ * (HD / 4)), f = e % (ATQ * (HD / 4));
            const int tk = f % ATQ, d = 4 * (f / ATQ), pr = (pt0 + u) * ATQ + tk;
            if (pr >= npairs) continue;
            float mw[AWV], Mx = -INFINITY;
#pragma unroll
            for (int k = 0; k < AWV; k++) {
                mw[k] = sm_m(u)[k][tk];
                Mx = fmaxf(Mx, mw[k]);
            }
            float Lw = 0.0f;
            attn_f32x4 ow = {0, 0, 0, 0};
#pragma unroll
            for (int k = 0; k < AWV; k++) {
                const float e2 = mw[k] == -INFINITY ? 0.0f : expf(mw[k] - Mx);
                Lw = __builtin_fmaf(sm_l(u)[k][tk], e2, Lw);
                const attn_f32x4 x = *reinterpret_cast<const attn_f32x4*>(&sm_o(u)[(k * ATQ + tk) * HP + d]);
#pragma unroll
                for (int i = 0; i < 4; i++) ow[i] = __builtin_fmaf(x[i], e2, ow[i]);
            }
            const size_t row = (size_t(i0 + pr % nq) * heads + grp * hpg + pr / nq) * ASPLIT + s;
            if (d == 0) {
                st_f32(Mx, rm, int(row * 4));
                st_f32(Lw, rl, int(row * 4));
            }
            st_attn_f32x4(ow, ro, int((row * HD + d) * 4));
        }
        __syncthreads();  // before the next pass reuses the LDS
    };
    int pt = 0;
    for (; pt + TP <= ptiles; pt += TP) pair_tiles(pt, std::integral_constant<int, TP>{});
    if constexpr (TP > 1)
        if (pt < ptiles) pair_tiles(pt, std::integral_constant<int, 1>{});

    // The last workgroup of (group, segment) merges the ASPLIT states of every pair in order.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        int* cn = A.cnt + size_t(seg) * kv_heads + grp;
        const int old = __hip_atomic_fetch_add(cn, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = old == live - 1;
        if (last) __hip_atomic_store(cn, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        flag = last;
    }
    __syncthreads();
    if (!flag) return;
    // (head, token) pairs over the 32 row slots of the workgroup, every head's rows into LDS
    // ([pair][HD]: at most heads_per_group x 16 rows), then the fragments.
    constexpr int DPT = HD / 16;
    float* Os = sm_o(0);
    const int sub = tid & 15;
    for (int pr = tid >> 4; pr < hpg * nq; pr += AWV * 64 / 16) {
        const int hh = pr / nq, row = pr % nq, head = grp * hpg + hh;
        const size_t base = (size_t(i0 + row) * heads + head) * ASPLIT;
        float mv[ASPLIT], lv[ASPLIT], ov[ASPLIT][DPT];
#pragma unroll
        for (int k = 0; k < ASPLIT; k++) {
            if (k >= live) {
                mv[k] = -INFINITY;
                lv[k] = 0.0f;
#pragma unroll
                for (int u = 0; u < DPT; u++) ov[k][u] = 0.0f;
                continue;
            }
            mv[k] = ld_f32(rm, int((base + k) * 4));
            lv[k] = ld_f32(rl, int((base + k) * 4));
            if constexpr (DPT % 4 == 0) {
#pragma unroll
                for (int u = 0; u < DPT; u += 4) {
                    const attn_f32x4 x = ld_attn_f32x4(ro, int(((base + k) * HD + sub * DPT + u) * 4));
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
        for (int u = 0; u < DPT; u++) Os[pr * HD + sub * DPT + u] = o[u] * inv;
    }
    __syncthreads();
    for (int p = tid; p < hpg * nq * (HD / 8); p += AWV * 64) {
        const int pr = p / (HD / 8), sl = p % (HD / 8), hh = pr / nq, i = pr % nq, col = (grp * hpg + hh) * HD + 8 * sl;
        const int r = i0 + i;  // token r % 16 of tile r / 16 (a segment may straddle two tiles)
        write_slot(frags + size_t(r / ATQ) * frag_stride, col / 32, r % ATQ + 16 * ((col % 32) / 8), Os + pr * HD + 8 * sl);
    }
}

}  // namespace ls
