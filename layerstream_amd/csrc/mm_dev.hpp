// Device helpers of the matrix kernels shared by fused.hip and pass.hip (the weight tile layout
// and activation fragments are described in fused.hpp). Only for .hip sources.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstddef>
#include <cstdint>

#include "frag_dev.hpp"
#include "fused.hpp"

namespace ls {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Sum of squares of 16 values v(0..15) (n of them, the rest zero) in the one order used
// everywhere: two sequential sums of eight, added.
template <class F>
__device__ __forceinline__ float ss16(F v, int n) {
    float s = 0.0f;
    for (int b = 0; b < 2; b++) {
        float sb = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int c = 8 * b + j;
            const float x = c < n ? v(c) : 0.0f;
            sb = __builtin_fmaf(x, x, sb);
        }
        s += sb;
    }
    return s;
}

// ---------------------------------------------------------------------------------------
// Main loop
// ---------------------------------------------------------------------------------------
// bf16 pair (a low, b high) of two floats that bf16 holds exactly: their high halves.
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
}

// A operand (8 bf16) of k-step q of a chunk slot.
template <int BITS>
__device__ __forceinline__ uint4 a_operand(const uint4& raw, int q) {
    if constexpr (BITS == 16) {
        return raw;
    } else if constexpr (BITS == 8) {
        const uint32_t d0 = q ? raw.z : raw.x, d1 = q ? raw.w : raw.y;
        float f[8];
#pragma unroll
        for (int b = 0; b < 4; b++) {
            f[b] = float(int32_t(d0 << (24 - 8 * b)) >> 24);
            f[4 + b] = float(int32_t(d1 << (24 - 8 * b)) >> 24);
        }
        return make_uint4(pack2(f[0], f[1]), pack2(f[2], f[3]), pack2(f[4], f[5]), pack2(f[6], f[7]));
    } else {
        const uint32_t d = q == 0 ? raw.x : (q == 1 ? raw.y : (q == 2 ? raw.z : raw.w));
        // Nibbles hold value + 8; ((n + 0x78) ^ 0x80) is the value as a signed byte, four bytes
        // at once (n + 0x78 <= 0x87, so no byte carries into the next). lo: values 0, 2, 4, 6;
        // hi: values 1, 3, 5, 7.
        const uint32_t lo = ((d & 0x0f0f0f0fu) + 0x78787878u) ^ 0x80808080u;
        const uint32_t hi = (((d >> 4) & 0x0f0f0f0fu) + 0x78787878u) ^ 0x80808080u;
        float f[8];
#pragma unroll
        for (int b = 0; b < 4; b++) {
            f[2 * b] = float(int32_t(lo << (24 - 8 * b)) >> 24);
            f[2 * b + 1] = float(int32_t(hi << (24 - 8 * b)) >> 24);
        }
        return make_uint4(pack2(f[0], f[1]), pack2(f[2], f[3]), pack2(f[4], f[5]), pack2(f[6], f[7]));
    }
}

__device__ __forceinline__ bf16x8 bf(const uint4& v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ f32x4 mfma3(const uint4& A, const uint4* B, f32x4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf(A), bf(B[0]), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf(A), bf(B[1]), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf(A), bf(B[2]), c, 0, 0, 0);
    return c;
}

__device__ __forceinline__ uint2 scales_raw(const uint16_t* __restrict__ sc, int strip, int n_groups, int g, int lane) {
    return *reinterpret_cast<const uint2*>(sc + (size_t(strip) * n_groups + g) * 16 + 4 * (lane >> 4));
}
__device__ __forceinline__ f32x4 scales_f32(uint2 v) {
    return f32x4{__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u), __uint_as_float(v.y << 16),
                 __uint_as_float(v.y & 0xffff0000u)};
}
__device__ __forceinline__ f32x4 scales4(const uint16_t* __restrict__ sc, int strip, int n_groups, int g, int lane) {
    return scales_f32(scales_raw(sc, strip, n_groups, g, lane));
}

// Chunks per wavefront: every wavefront covers 4 k-steps (128 columns).
template <int BITS>
struct Steps {
    static constexpr int Q = BITS == 16 ? 1 : (BITS == 8 ? 2 : 4);  // k-steps per chunk
    static constexpr int CPW = 4 / Q;                                // chunks per wavefront
};

// Weights are read once per pass: non-temporal loads keep them from displacing the activations.
template <int S>
__device__ __forceinline__ void load_chunk(const uint8_t* base, size_t sstride, int c, uint4* raw) {
#pragma unroll
    for (int r = 0; r < S; r++) {
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + r * sstride + size_t(c) * 1024));
        raw[r] = make_uint4(v[0], v[1], v[2], v[3]);
    }
}

// One chunk: Q k-steps x S strips x 3 MFMAs, with group scaling. B[q][term] are the fragments of
// the chunk's k-steps; [ks_begin, ks_end) is the wavefront's k-step range.
// Scale slots per chunk (k-steps that may close a group; groups of 16: two per k-step).
template <int BITS, bool G16>
constexpr int scale_slots() {
    return BITS == 16 ? 1 : (G16 ? 2 * Steps<BITS>::Q : Steps<BITS>::Q);
}

// The group scales chunk_mfma applies for chunk c, loaded ahead (with the weights): the same
// scales, so the products are unchanged, but their latency no longer follows the input's.
template <int BITS, bool G16, int S>
__device__ __forceinline__ void load_scales(const TMat& W, int s0, int c, int ks_end, uint2 (*scl)[S]) {
    const int lane = threadIdx.x & 63;
    constexpr int Q = Steps<BITS>::Q;
    const int G = W.group;
#pragma unroll
    for (int q = 0; q < Q; q++) {
        const int ks = c * Q + q;
        if constexpr (G16) {
#pragma unroll
            for (int r = 0; r < S; r++) {
                scl[2 * q][r] = scales_raw(W.scales, s0 + r, W.n_groups, 2 * ks, lane);
                scl[2 * q + 1][r] = scales_raw(W.scales, s0 + r, W.n_groups, 2 * ks + 1, lane);
            }
        } else {
            const bool last = ((ks + 1) * 32) % G == 0 || ks == ks_end - 1;
#pragma unroll
            for (int r = 0; r < S; r++) scl[q][r] = last ? scales_raw(W.scales, s0 + r, W.n_groups, ks * 32 / G, lane) : make_uint2(0, 0);
        }
    }
}

// With PRE the scales come from scl (load_scales for this chunk), else from memory here.
template <int BITS, bool G16, int S, bool PRE = false>
__device__ __forceinline__ void chunk_mfma(const TMat& W, int s0, int c, int ks_begin, int ks_end, const uint4 (*B)[3],
                                           const uint4* raw, f32x4* acc, f32x4* total, const uint2 (*scl)[S] = nullptr) {
    const int lane = threadIdx.x & 63;
    constexpr int Q = Steps<BITS>::Q;
    const int G = W.group;
#pragma unroll
    for (int q = 0; q < Q; q++) {
        const int ks = c * Q + q;
        if constexpr (BITS == 16) {
#pragma unroll
            for (int r = 0; r < S; r++) total[r] = mfma3(a_operand<BITS>(raw[r], q), B[q], total[r]);
        } else if constexpr (!G16) {
            const bool first = (ks * 32) % G == 0 || ks == ks_begin;
            const bool last = ((ks + 1) * 32) % G == 0 || ks == ks_end - 1;
#pragma unroll
            for (int r = 0; r < S; r++) acc[r] = mfma3(a_operand<BITS>(raw[r], q), B[q], first ? f32x4{0, 0, 0, 0} : acc[r]);
            if (last) {
                const int g = ks * 32 / G;
#pragma unroll
                for (int r = 0; r < S; r++) {
                    const f32x4 sc = PRE ? scales_f32(scl[q][r]) : scales4(W.scales, s0 + r, W.n_groups, g, lane);
#pragma unroll
                    for (int i = 0; i < 4; i++) total[r][i] = __builtin_fmaf(sc[i], acc[r][i], total[r][i]);
                }
            }
        } else {
            // Groups of 16: lanes 0-31 hold the k-step's first group, lanes 32-63 the second.
            const bool lo = lane < 32;
#pragma unroll
            for (int r = 0; r < S; r++) {
                const uint4 A = a_operand<BITS>(raw[r], q), Z = make_uint4(0, 0, 0, 0);
                const f32x4 a1 = mfma3(lo ? A : Z, B[q], f32x4{0, 0, 0, 0});
                const f32x4 a2 = mfma3(lo ? Z : A, B[q], f32x4{0, 0, 0, 0});
                const f32x4 s1 = PRE ? scales_f32(scl[2 * q][r]) : scales4(W.scales, s0 + r, W.n_groups, 2 * ks, lane);
                const f32x4 s2 = PRE ? scales_f32(scl[2 * q + 1][r]) : scales4(W.scales, s0 + r, W.n_groups, 2 * ks + 1, lane);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    total[r][i] = __builtin_fmaf(s1[i], a1[i], total[r][i]);
                    total[r][i] = __builtin_fmaf(s2[i], a2[i], total[r][i]);
                }
            }
        }
    }
}

enum { EPI_QKV = 0, EPI_RESID = 1, EPI_SILU = 2, EPI_HEAD = 3 };

// 1 / rms per token of a tile from the producer's sum-of-squares partials, by one wavefront:
// lane (part, token) adds slots part, part + 4, ... in order (loads issued 16 at a time), then a
// fixed shuffle tree over the four parts (src/kernels.rs:217-228 up to the summation order).
// The first 16 loads are issued by rms_issue (at workgroup entry, beside the weight loads) and
// consumed by rms_finish (after the matrix work), so their latency hides behind the weights'.
struct RmsLoads {
    float x[16];
};
// With COH the partials were written earlier in the same launch and are read through the
// coherent path.
template <bool COH = false>
__device__ __forceinline__ float ss_load(const MMArgs& a, int tile, int sl, int tok) {
    if constexpr (COH) {
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.ss) + size_t(tile) * a.ss_slots * FTOK, 0,
                                                                          a.ss_slots * FTOK * 4, BUF_DWORD3);
        return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (sl * FTOK + tok) * 4, 0, CPOL_SC1));
    } else {
        return a.ss[(size_t(tile) * a.ss_slots + sl) * FTOK + tok];
    }
}
template <bool COH = false>
__device__ __forceinline__ void rms_issue(const MMArgs& a, int tile, RmsLoads& r) {
    const int lane = threadIdx.x & 63, tok = lane & 15, part = lane >> 4;
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const int sl = part + 4 * k;
        r.x[k] = sl < a.ss_slots ? ss_load<COH>(a, tile, sl, tok) : 0.0f;
    }
}
template <bool COH = false>
__device__ __forceinline__ void rms_finish(const MMArgs& a, int tile, int cols, const RmsLoads& r, float* inv) {
    const int lane = threadIdx.x & 63, tok = lane & 15, part = lane >> 4;
    float v = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; k++) v += r.x[k];
    for (int k0 = 16; part + 4 * k0 < a.ss_slots; k0 += 16) {
        float x[16];
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int sl = part + 4 * (k0 + k);
            x[k] = sl < a.ss_slots ? ss_load<COH>(a, tile, sl, tok) : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < 16; k++) v += x[k];
    }
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    if (lane < FTOK) inv[lane] = 1.0f / sqrtf(v / float(cols) + a.eps);
}
__device__ __forceinline__ void inv_rms(const MMArgs& a, int tile, int cols, float* inv) {
    RmsLoads r;
    rms_issue(a, tile, r);
    rms_finish(a, tile, cols, r, inv);
}

__device__ __forceinline__ bool beats(float va, int ia, float vb, int ib) {
    const bool an = isnan(va), bn = isnan(vb);
    if (an != bn) return !an;
    if (an) return ia < ib;
    if (va != vb) return va > vb;
    return ia < ib;
}

// q|k rows are stored with each head's RoPE pairs adjacent: tile row 2j holds dimension j and
// tile row 2j + 1 dimension j + hd / 2. Reference row of a tile row of the q|k|v matrix:
__device__ __forceinline__ int qkv_ref_row(int row, int hd, int qk_rows) {
    if (row >= qk_rows) return row;
    const int r = row % hd;
    return row - r + ((r & 1) ? hd / 2 + (r >> 1) : (r >> 1));
}

constexpr int MAX_SPLIT = 16;
constexpr int MAX_KW = 16;  // wavefronts along K of one row group (mm_max_waves)
constexpr int ROPE_HALF_MAX = 128;

}  // namespace ls
