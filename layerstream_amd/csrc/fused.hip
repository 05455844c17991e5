// Fused MFMA kernels of the verify step for gfx950 (CDNA4, wave64, v_mfma_f32_16x16x32_bf16).
//
// One launch handles one tile of up to 16 tokens. A workgroup owns 64 * RG weight rows and splits
// the padded K range into KSPLIT contiguous pieces, one wavefront each; a wavefront streams four
// 16-row strips of its piece, one 1 KiB load per strip and chunk, converts the int8 / int4 / bf16
// weights to bf16 in registers and issues three MFMAs per strip and k-step (one per input term).
// Group scales multiply each group's accumulator. The pieces are summed in a fixed order in LDS and
// an epilogue consumes the [rows][tokens] tile. Every output element's arithmetic depends only on
// the matrix shape, never on the number of tokens in the launch: a verify pass over k+1 tokens
// gives the same bits as k+1 single-token passes (src/spec.rs:8-11).
#include "fused.hpp"

#include <cmath>
#include <stdexcept>
#include <string>

namespace ls {

#define FCHECK(x)                                                                                         \
    do {                                                                                                  \
        hipError_t e_ = (x);                                                                              \
        if (e_ != hipSuccess) throw std::runtime_error(std::string("HIP: ") + hipGetErrorString(e_)); \
    } while (0)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------------------
// Layout
// ---------------------------------------------------------------------------------------

TMat tile_shape(int bits, int group, int rows, int cols, int row_align) {
    TMat m;
    m.bits = bits;
    m.group = bits == 16 ? 0 : group;
    m.rows = rows;
    m.cols = cols;
    m.n_strips = (rows + row_align - 1) / row_align * (row_align / 16);
    m.n_chunks = tile_kpad(cols) / tile_chunk_cols(bits);
    m.n_groups = bits == 16 ? 0 : tile_kpad(cols) / group + (tile_kpad(cols) % group ? 1 : 0);
    return m;
}

size_t tile_data_bytes(const TMat& m) { return size_t(m.n_strips) * m.n_chunks * 64 * 16; }
size_t tile_scale_bytes(const TMat& m) { return m.bits == 16 ? 0 : size_t(m.n_strips) * m.n_groups * 16 * 2; }

TMat tile_bind(const TMat& shape, uint8_t* data, uint16_t* scales) {
    TMat m = shape;
    m.data = data;
    m.scales = shape.bits == 16 ? nullptr : scales;
    return m;
}

void tile_clear(const TMat& m, hipStream_t s) {
    FCHECK(hipMemsetAsync(const_cast<uint8_t*>(m.data), m.bits == 4 ? 0x88 : 0, tile_data_bytes(m), s));
    if (m.bits != 16) FCHECK(hipMemsetAsync(const_cast<uint16_t*>(m.scales), 0, tile_scale_bytes(m), s));
}

// Value stored for (row, col) of a reference row: bf16 bits, the int8 byte, or the int4 nibble.
__device__ __forceinline__ uint32_t raw_elem(const uint8_t* row, int bits, int group, int c) {
    if (bits == 16) return uint32_t(row[2 * c]) | uint32_t(row[2 * c + 1]) << 8;
    if (bits == 8) return row[c];
    const int half = group / 2, g = c / group, wj = c % group;
    const uint8_t b = row[g * half + (wj % half)];
    return wj < half ? (b & 15u) : (b >> 4);
}

// One thread per (row, chunk): the 64 bytes of its four lane slots.
__global__ void k_tile_repack(const uint8_t* __restrict__ raw, int rows, TMat m, int row_off, int block, int stride) {
    const int r = blockIdx.x;
    if (r >= rows) return;
    const int bits = m.bits, K = m.cols;
    const int db = bits == 16 ? 2 * K : K * bits / 8;
    const int ng_real = bits == 16 ? 0 : K / m.group;
    const uint8_t* row = raw + size_t(r) * (db + 2 * ng_real);
    const int dr = row_off + (r / block) * stride + r % block, strip = dr / 16, rl = dr % 16;
    const int cc = tile_chunk_cols(bits), Q = cc / 32;
    uint8_t* data = const_cast<uint8_t*>(m.data);
    for (int c = threadIdx.x; c < m.n_chunks; c += blockDim.x) {
        for (int lg = 0; lg < 4; lg++) {
            uint8_t out[16];
            for (int i = 0; i < 16; i++) out[i] = bits == 4 ? 0x88 : 0;
            for (int q = 0; q < Q; q++)
                for (int j = 0; j < 8; j++) {
                    const int col = c * cc + 32 * q + 8 * lg + j;
                    if (col >= K) continue;
                    const uint32_t v = raw_elem(row, bits, m.group, col);
                    if (bits == 16) {
                        out[2 * j] = uint8_t(v);
                        out[2 * j + 1] = uint8_t(v >> 8);
                    } else if (bits == 8) {
                        out[8 * q + j] = uint8_t(v);
                    } else {
                        uint8_t& o = out[4 * q + j / 2];
                        o = (j & 1) ? uint8_t((o & 0x0f) | (v << 4)) : uint8_t((o & 0xf0) | v);
                    }
                }
            uint8_t* dst = data + ((size_t(strip) * m.n_chunks + c) * 64 + rl + 16 * lg) * 16;
            for (int i = 0; i < 16; i++) dst[i] = out[i];
        }
    }
    if (bits != 16) {
        uint16_t* sc = const_cast<uint16_t*>(m.scales);
        for (int g = threadIdx.x; g < ng_real; g += blockDim.x)
            sc[(size_t(strip) * m.n_groups + g) * 16 + rl] = uint16_t(row[db + 2 * g] | (row[db + 2 * g + 1] << 8));
    }
}

void tile_repack(const uint8_t* raw, int rows, const TMat& dst, int row_off, int block, int stride, hipStream_t s) {
    if (rows <= 0) return;
    hipLaunchKernelGGL(k_tile_repack, dim3(rows), dim3(64), 0, s, raw, rows, dst, row_off, block, stride);
    FCHECK(hipGetLastError());
}

__global__ void k_tile_embed(TMat E, const uint32_t* __restrict__ tokens, float* __restrict__ x) {
    const int i = blockIdx.x;
    const int r = int(tokens[i]), strip = r / 16, rl = r % 16;
    const int cc = tile_chunk_cols(E.bits);
    for (int col = threadIdx.x; col < E.cols; col += blockDim.x) {
        const int c = col / cc, q = (col % cc) / 32, lg = (col % 32) / 8, j = col % 8;
        const uint8_t* slot = E.data + ((size_t(strip) * E.n_chunks + c) * 64 + rl + 16 * lg) * 16;
        float v;
        if (E.bits == 16) {
            v = __uint_as_float(uint32_t(slot[2 * j] | (slot[2 * j + 1] << 8)) << 16);
        } else {
            float qv;
            if (E.bits == 8) {
                qv = float(int32_t(int8_t(slot[8 * q + j])));
            } else {
                const uint8_t b = slot[4 * q + j / 2];
                qv = float(int32_t((j & 1) ? (b >> 4) : (b & 15)) - 8);
            }
            const uint16_t sb = E.scales[(size_t(strip) * E.n_groups + col / E.group) * 16 + rl];
            v = qv * __uint_as_float(uint32_t(sb) << 16);
        }
        x[size_t(i) * E.cols + col] = v;
    }
}

void tile_embed(const TMat& E, const uint32_t* tokens, int t, float* x, hipStream_t s) {
    hipLaunchKernelGGL(k_tile_embed, dim3(t), dim3(256), 0, s, E, tokens, x);
    FCHECK(hipGetLastError());
}

// ---------------------------------------------------------------------------------------
// B fragments: f32 value -> three bf16 terms (truncations) whose sum is the value exactly.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ void split3(float v, uint32_t& h, uint32_t& m, uint32_t& l) {
    const uint32_t vb = __float_as_uint(v);
    const float hv = __uint_as_float(vb & 0xffff0000u);
    const float r1 = v - hv;
    const uint32_t r1b = __float_as_uint(r1);
    const float mv = __uint_as_float(r1b & 0xffff0000u);
    const float r2 = r1 - mv;
    h = vb >> 16;
    m = r1b >> 16;
    l = __float_as_uint(r2) >> 16;
}

// Fragment slot p = (k-step, lane): token lane % 16, columns 32 ks + 8 (lane / 16) + j.
__device__ __forceinline__ void build_frag_slot(int p, const float* __restrict__ x, int ldx, int i0, int nt, int K,
                                                const float* __restrict__ w, const float* inv, uint8_t* dst) {
    const int ks = p >> 6, lane = p & 63, tok = lane & 15;
    const int col0 = 32 * ks + 8 * (lane >> 4);
    uint32_t H[4], M[4], L[4];
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        float v0 = 0.0f, v1 = 0.0f;
        if (tok < nt) {
            const float* xr = x + size_t(i0 + tok) * ldx;
            const float iv = inv ? inv[tok] : 1.0f;
            if (col0 + j < K) v0 = w ? __fmul_rn(__fmul_rn(xr[col0 + j], iv), w[col0 + j]) : xr[col0 + j];
            if (col0 + j + 1 < K) v1 = w ? __fmul_rn(__fmul_rn(xr[col0 + j + 1], iv), w[col0 + j + 1]) : xr[col0 + j + 1];
        }
        uint32_t h0, m0, l0, h1, m1, l1;
        split3(v0, h0, m0, l0);
        split3(v1, h1, m1, l1);
        H[j / 2] = h0 | (h1 << 16);
        M[j / 2] = m0 | (m1 << 16);
        L[j / 2] = l0 | (l1 << 16);
    }
    uint4* o = reinterpret_cast<uint4*>(dst + (size_t(ks) * 3 * 64 + lane) * 16);
    o[0] = make_uint4(H[0], H[1], H[2], H[3]);
    o[64] = make_uint4(M[0], M[1], M[2], M[3]);
    o[128] = make_uint4(L[0], L[1], L[2], L[3]);
}

// Per-token 1 / sqrt(mean(x^2) + eps) (src/kernels.rs:217-228): token i is always reduced by one
// wavefront with lane-strided partial sums and a fixed shuffle tree.
__device__ void norm_invs(const float* __restrict__ x, int ldx, int i0, int nt, int K, float eps, float* inv, int nwaves) {
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int tok = wv; tok < nt; tok += nwaves) {
        const float* xr = x + size_t(i0 + tok) * ldx;
        float ss = 0.0f;
        for (int c = lane; c < K; c += 64) ss = __builtin_fmaf(xr[c], xr[c], ss);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
        if (lane == 0) inv[tok] = 1.0f / sqrtf(ss / float(K) + eps);
    }
}

__global__ __launch_bounds__(256) void k_frag_build(const float* __restrict__ x, int ldx, int i0, int nt, int K,
                                                    const float* __restrict__ w, float eps, uint8_t* __restrict__ frags) {
    __shared__ float inv[FTOK];
    if (w) norm_invs(x, ldx, i0, nt, K, eps, inv, 4);
    __syncthreads();
    const int n = tile_kpad(K) / 32 * 64;
    for (int p = blockIdx.x * 256 + threadIdx.x; p < n; p += gridDim.x * 256) build_frag_slot(p, x, ldx, i0, nt, K, w, w ? inv : nullptr, frags);
}

void frag_build(const float* x, int ldx, int i0, int nt, int cols, const float* w, float eps, uint8_t* frags, hipStream_t s) {
    const int n = tile_kpad(cols) / 32 * 64;
    hipLaunchKernelGGL(k_frag_build, dim3((n + 255) / 256), dim3(256), 0, s, x, ldx, i0, nt, cols, w, eps, frags);
    FCHECK(hipGetLastError());
}

// ---------------------------------------------------------------------------------------
// Main loop
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    return (__float_as_uint(a) >> 16) | (__float_as_uint(b) & 0xffff0000u);
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
        float f[8];
#pragma unroll
        for (int j = 0; j < 8; j++) f[j] = float(int32_t((d >> (4 * j)) & 15u) - 8);
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

__device__ __forceinline__ f32x4 scales4(const uint16_t* __restrict__ sc, int strip, int n_groups, int g, int lane) {
    const uint2 v = *reinterpret_cast<const uint2*>(sc + (size_t(strip) * n_groups + g) * 16 + 4 * (lane >> 4));
    return f32x4{__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u), __uint_as_float(v.y << 16),
                 __uint_as_float(v.y & 0xffff0000u)};
}

// A wavefront's share of the matrix: four strips s0..s0+3 over chunks [c0, c1). Weight loads
// run PF chunks ahead of the MFMAs: the first PF chunks are requested before the caller's
// prologue, so HBM latency overlaps the input normalisation.
constexpr int PF = 2;

struct WaveLoads {
    uint4 buf[PF][4];
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Weights are read once per pass: non-temporal loads keep them from displacing the activations.
__device__ __forceinline__ void load_chunk(const uint8_t* base, size_t sstride, int c, uint4* raw) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + r * sstride + size_t(c) * 1024));
        raw[r] = make_uint4(v[0], v[1], v[2], v[3]);
    }
}

__device__ __forceinline__ void wave_prefetch(const TMat& W, int s0, int c0, int c1, WaveLoads& L) {
    const int lane = threadIdx.x & 63;
    const uint8_t* base = W.data + (size_t(s0) * W.n_chunks * 64 + lane) * 16;
    const size_t sstride = size_t(W.n_chunks) * 64 * 16;
#pragma unroll
    for (int p = 0; p < PF; p++)
        if (c0 + p < c1) load_chunk(base, sstride, c0 + p, L.buf[p]);
}

// One chunk: Q k-steps x 4 strips x 3 MFMAs, with group scaling.
template <int BITS, bool G16>
__device__ __forceinline__ void chunk_mfma(const TMat& W, int s0, int c, int ks_begin, int ks_end, const uint4* fr,
                                           const uint4* raw, f32x4* acc, f32x4* total) {
    const int lane = threadIdx.x & 63;
    constexpr int Q = BITS == 16 ? 1 : (BITS == 8 ? 2 : 4);
    const int G = W.group;
#pragma unroll(BITS == 4 ? 1 : Q)
    for (int q = 0; q < Q; q++) {
        const int ks = c * Q + q;
        uint4 B[3];
        B[0] = fr[(ks * 3 + 0) * 64 + lane];
        B[1] = fr[(ks * 3 + 1) * 64 + lane];
        B[2] = fr[(ks * 3 + 2) * 64 + lane];
        if constexpr (BITS == 16) {
#pragma unroll
            for (int r = 0; r < 4; r++) total[r] = mfma3(a_operand<BITS>(raw[r], q), B, total[r]);
        } else if constexpr (!G16) {
            const bool first = (ks * 32) % G == 0 || ks == ks_begin;
            const bool last = ((ks + 1) * 32) % G == 0 || ks == ks_end - 1;
#pragma unroll
            for (int r = 0; r < 4; r++) acc[r] = mfma3(a_operand<BITS>(raw[r], q), B, first ? f32x4{0, 0, 0, 0} : acc[r]);
            if (last) {
                const int g = ks * 32 / G;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const f32x4 sc = scales4(W.scales, s0 + r, W.n_groups, g, lane);
#pragma unroll
                    for (int i = 0; i < 4; i++) total[r][i] = __builtin_fmaf(sc[i], acc[r][i], total[r][i]);
                }
            }
        } else {
            // Groups of 16: lanes 0-31 hold the k-step's first group, lanes 32-63 the second.
            const bool lo = lane < 32;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint4 A = a_operand<BITS>(raw[r], q), Z = make_uint4(0, 0, 0, 0);
                const f32x4 a1 = mfma3(lo ? A : Z, B, f32x4{0, 0, 0, 0});
                const f32x4 a2 = mfma3(lo ? Z : A, B, f32x4{0, 0, 0, 0});
                const f32x4 s1 = scales4(W.scales, s0 + r, W.n_groups, 2 * ks, lane);
                const f32x4 s2 = scales4(W.scales, s0 + r, W.n_groups, 2 * ks + 1, lane);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    total[r][i] = __builtin_fmaf(s1[i], a1[i], total[r][i]);
                    total[r][i] = __builtin_fmaf(s2[i], a2[i], total[r][i]);
                }
            }
        }
    }
}

template <int BITS, bool G16>
__device__ __forceinline__ void wave_tiles(const TMat& W, int s0, int c0, int c1, const uint4* fr, WaveLoads& L, f32x4* total) {
    const int lane = threadIdx.x & 63;
    constexpr int Q = BITS == 16 ? 1 : (BITS == 8 ? 2 : 4);
    const int ks_begin = c0 * Q, ks_end = c1 * Q;
    const uint8_t* base = W.data + (size_t(s0) * W.n_chunks * 64 + lane) * 16;
    const size_t sstride = size_t(W.n_chunks) * 64 * 16;
    f32x4 acc[4];
#pragma unroll
    for (int r = 0; r < 4; r++) total[r] = acc[r] = f32x4{0, 0, 0, 0};
    for (int c = c0; c < c1; c += PF) {
#pragma unroll
        for (int p = 0; p < PF; p++) {
            if (c + p < c1) {
                chunk_mfma<BITS, G16>(W, s0, c + p, ks_begin, ks_end, fr, L.buf[p], acc, total);
                if (c + p + PF < c1) load_chunk(base, sstride, c + p + PF, L.buf[p]);
            }
        }
    }
}

enum { EPI_QKV = 0, EPI_RESID = 1, EPI_SILU = 2, EPI_HEAD = 3 };

struct FusedCfg {
    int rg;          // 64-row groups per workgroup
    int ksplit;      // wavefronts per row group
    int frag_lds;    // 1: build B fragments in LDS from x (prologue); 0: read a.frags from global
    int frag_bytes;  // LDS bytes of the fragments
};

// Dynamic LDS: [fragments | reduction] then [tile: rows x 16 floats] then [16 inverse norms].
template <int BITS, int EPI, bool G16>
__global__ __launch_bounds__(1024) void k_fused(FusedArgs a, FusedCfg cfg) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int nw = cfg.rg * cfg.ksplit;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int rows_wg = 64 * cfg.rg;
    const size_t red_bytes = size_t(nw) * 4 * 64 * 16;
    const size_t region = cfg.frag_bytes > int(red_bytes) ? size_t(cfg.frag_bytes) : red_bytes;
    float* tile = reinterpret_cast<float*>(smem + region);
    float* inv = tile + rows_wg * FTOK;
    const TMat& W = a.W;

    // This wavefront's rows and k range; its first weight chunks are requested right away.
    const int rgi = wv / cfg.ksplit, kp = wv % cfg.ksplit;
    const int s0 = (blockIdx.x * cfg.rg + rgi) * 4;
    const int c0 = kp * W.n_chunks / cfg.ksplit, c1 = (kp + 1) * W.n_chunks / cfg.ksplit;
    WaveLoads loads;
    wave_prefetch(W, s0, c0, c1, loads);

    // Prologue: B fragments of the token tile.
    const uint4* fr;
    if (cfg.frag_lds) {
        if (a.norm) norm_invs(a.x, a.ldx, a.i0, a.nt, W.cols, a.eps, inv, nw);
        __syncthreads();
        const int n = W.n_chunks * tile_chunk_cols(BITS) / 32 * 64;
        for (int p = threadIdx.x; p < n; p += nw * 64)
            build_frag_slot(p, a.x, a.ldx, a.i0, a.nt, W.cols, a.norm, a.norm ? inv : nullptr, smem);
        __syncthreads();
        fr = reinterpret_cast<const uint4*>(smem);
    } else {
        fr = reinterpret_cast<const uint4*>(a.frags);
    }

    f32x4 total[4];
    wave_tiles<BITS, G16>(W, s0, c0, c1, fr, loads, total);

    // Fixed-order sum of the pieces: red[wave][strip][lane] (float4), then the tile.
    __syncthreads();
    f32x4* red = reinterpret_cast<f32x4*>(smem);
#pragma unroll
    for (int r = 0; r < 4; r++) red[(wv * 4 + r) * 64 + lane] = total[r];
    __syncthreads();
    for (int e = threadIdx.x; e < cfg.rg * 4 * 64; e += nw * 64) {
        const int rg = e / 256, r = (e / 64) % 4, ln = e % 64;
        f32x4 sum = red[((rg * cfg.ksplit) * 4 + r) * 64 + ln];
        for (int k = 1; k < cfg.ksplit; k++) {
            const f32x4 v = red[(((rg * cfg.ksplit) + k) * 4 + r) * 64 + ln];
#pragma unroll
            for (int i = 0; i < 4; i++) sum[i] += v[i];
        }
#pragma unroll
        for (int i = 0; i < 4; i++) tile[(64 * rg + 16 * r + 4 * (ln >> 4) + i) * FTOK + (ln & 15)] = sum[i];
    }
    __syncthreads();

    // Epilogues over tile[row_local][token].
    const int row0 = blockIdx.x * rows_wg;
    if constexpr (EPI == EPI_QKV) {
        // rows: [0, h) q heads, [h, h + kv) k heads, [h + kv, h + 2 kv) v heads
        const int hd = a.hd, half = hd / 2, h = a.heads * hd, kv = a.kv_heads * hd;
        const int pos0 = *a.pos0;
        for (int e = threadIdx.x; e < rows_wg * FTOK; e += nw * 64) {
            const int rl = e / FTOK, tok = e % FTOK, row = row0 + rl;
            if (tok >= a.nt || row >= W.rows) continue;
            tile[rl * FTOK + tok] += a.bias[row];
        }
        __syncthreads();
        for (int e = threadIdx.x; e < rows_wg * FTOK; e += nw * 64) {
            const int rl = e / FTOK, tok = e % FTOK, row = row0 + rl;
            if (tok >= a.nt || row >= W.rows) continue;
            const int i = a.i0 + tok, pos = pos0 + i;
            float v = tile[rl * FTOK + tok];
            if (row < h + kv) {  // RoPE, rotate half (src/kernels.rs:242-252)
                const int d = row % hd, j = d % half;
                const float c = a.rope_cos[size_t(pos) * half + j], sn = a.rope_sin[size_t(pos) * half + j];
                if (d < half) {
                    const float b = tile[(rl + half) * FTOK + tok];
                    v = __fsub_rn(__fmul_rn(v, c), __fmul_rn(b, sn));
                } else {
                    const float aa = tile[(rl - half) * FTOK + tok];
                    v = __fadd_rn(__fmul_rn(v, c), __fmul_rn(aa, sn));
                }
            }
            if (row < h) a.out[size_t(i) * a.ldo + row] = v;
            else if (row < h + kv) a.kcache[size_t(pos) * kv + (row - h)] = v;
            else a.vcache[size_t(pos) * kv + (row - h - kv)] = v;
        }
    } else if constexpr (EPI == EPI_RESID) {
        for (int e = threadIdx.x; e < rows_wg * FTOK; e += nw * 64) {
            const int rl = e / FTOK, tok = e % FTOK, row = row0 + rl;
            if (tok >= a.nt || row >= W.rows) continue;
            float* o = a.out + size_t(a.i0 + tok) * a.ldo + row;
            *o = *o + tile[rl * FTOK + tok];
        }
    } else if constexpr (EPI == EPI_SILU) {
        // rows: [64 gate rows | 64 up rows] for act columns 64 * blockIdx.x + [0, 64)
        for (int p = threadIdx.x; p < 2 * 64; p += nw * 64) {
            const int ksl = p / 64, ln = p % 64, tok = ln & 15;
            const int colb = 32 * ksl + 8 * (ln >> 4);
            const int col0 = 64 * blockIdx.x + colb;
            uint32_t H[4], M[4], L[4];
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                float v[2];
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    v[u] = 0.0f;
                    if (tok < a.nt) {
                        const float g = tile[(colb + j + u) * FTOK + tok], up = tile[(64 + colb + j + u) * FTOK + tok];
                        v[u] = __fmul_rn(g / (1.0f + expf(-g)), up);
                    }
                }
                uint32_t h0, m0, l0, h1, m1, l1;
                split3(v[0], h0, m0, l0);
                split3(v[1], h1, m1, l1);
                H[j / 2] = h0 | (h1 << 16);
                M[j / 2] = m0 | (m1 << 16);
                L[j / 2] = l0 | (l1 << 16);
            }
            const int ks = col0 / 32;
            uint4* o = reinterpret_cast<uint4*>(a.frag_out + (size_t(ks) * 3 * 64 + ln) * 16);
            o[0] = make_uint4(H[0], H[1], H[2], H[3]);
            o[64] = make_uint4(M[0], M[1], M[2], M[3]);
            o[128] = make_uint4(L[0], L[1], L[2], L[3]);
        }
    } else {
        // Output head: optional logits, per-token best (value, index) of this block.
        if (a.out) {
            for (int e = threadIdx.x; e < rows_wg * FTOK; e += nw * 64) {
                const int rl = e / FTOK, tok = e % FTOK, row = row0 + rl;
                if (tok < a.nt && row < W.rows) a.out[size_t(a.i0 + tok) * a.ldo + row] = tile[rl * FTOK + tok];
            }
        }
        float* bv = inv + FTOK;               // [16 tokens][16 parts]
        int* bi = reinterpret_cast<int*>(bv + FTOK * 16);
        for (int e = threadIdx.x; e < FTOK * 16; e += nw * 64) {
            const int tok = e % FTOK, part = e / FTOK;
            float v = NAN;
            int ix = 0x7fffffff;
            for (int rl = part; rl < rows_wg; rl += 16) {
                const int row = row0 + rl;
                if (row >= W.rows) break;
                const float x = tile[rl * FTOK + tok];
                const bool xn = isnan(x), vn = isnan(v);
                const bool take = (xn != vn) ? !xn : (xn ? row < ix : (x != v ? x > v : row < ix));
                if (take) {
                    v = x;
                    ix = a.row_base + row;
                }
            }
            bv[tok * 16 + part] = v;
            bi[tok * 16 + part] = ix;
        }
        __syncthreads();
        if (threadIdx.x < FTOK) {
            const int tok = threadIdx.x;
            float v = bv[tok * 16];
            int ix = bi[tok * 16];
            for (int p = 1; p < 16; p++) {
                const float x = bv[tok * 16 + p];
                const int xi = bi[tok * 16 + p];
                const bool xn = isnan(x), vn = isnan(v);
                const bool take = (xn != vn) ? !xn : (xn ? xi < ix : (x != v ? x > v : xi < ix));
                if (take) {
                    v = x;
                    ix = xi;
                }
            }
            a.arg_val[blockIdx.x * FTOK + tok] = v;
            a.arg_idx[blockIdx.x * FTOK + tok] = ix;
            if (blockIdx.x == 0 && a.row0) a.row0[tok] = tile[tok];
        }
    }
}

static size_t lds_bytes(const FusedCfg& c, int rows_wg) {
    const size_t red = size_t(c.rg) * c.ksplit * 4 * 64 * 16;
    const size_t region = size_t(c.frag_bytes) > red ? size_t(c.frag_bytes) : red;
    return region + size_t(rows_wg) * FTOK * 4 + FTOK * 4 + FTOK * 16 * 8;
}

template <int EPI>
static void launch(const FusedArgs& a, FusedCfg cfg, int nblocks, hipStream_t s) {
    const int rows_wg = 64 * cfg.rg;
    const size_t lds = lds_bytes(cfg, rows_wg);
    const dim3 grid(nblocks), block(64 * cfg.rg * cfg.ksplit);
    const bool g16 = a.W.bits != 16 && a.W.group == 16;
    switch (a.W.bits) {
        case 16: hipLaunchKernelGGL((k_fused<16, EPI, false>), grid, block, lds, s, a, cfg); break;
        case 8:
            if (g16) hipLaunchKernelGGL((k_fused<8, EPI, true>), grid, block, lds, s, a, cfg);
            else hipLaunchKernelGGL((k_fused<8, EPI, false>), grid, block, lds, s, a, cfg);
            break;
        default:
            if (g16) hipLaunchKernelGGL((k_fused<4, EPI, true>), grid, block, lds, s, a, cfg);
            else hipLaunchKernelGGL((k_fused<4, EPI, false>), grid, block, lds, s, a, cfg);
            break;
    }
    FCHECK(hipGetLastError());
}

constexpr int FRAG_LDS_MAX = 96 * 1024;

static FusedCfg make_cfg(const FusedArgs& a, int rg, int ksplit) {
    FusedCfg c;
    c.rg = rg;
    c.ksplit = ksplit < 1 ? 1 : (ksplit > a.W.n_chunks ? a.W.n_chunks : ksplit);
    while (c.rg * c.ksplit > 16) c.ksplit--;
    const int fb = tile_kpad(a.W.cols) / 32 * 3 * 1024;
    c.frag_lds = a.frags == nullptr ? 1 : 0;
    if (c.frag_lds && fb > FRAG_LDS_MAX) throw std::runtime_error("fused kernel: input too wide for LDS fragments");
    c.frag_bytes = c.frag_lds ? fb : 0;
    return c;
}

void fused_qkv(const FusedArgs& a, hipStream_t s) {
    const int rg = a.hd > 64 ? a.hd / 64 : 1;
    FusedCfg c = make_cfg(a, rg, 16 / rg);
    launch<EPI_QKV>(a, c, (a.W.rows + 64 * rg - 1) / (64 * rg), s);
}

void fused_residual(const FusedArgs& a, int ksplit, hipStream_t s) {
    FusedCfg c = make_cfg(a, 1, ksplit);
    launch<EPI_RESID>(a, c, (a.W.rows + 63) / 64, s);
}

void fused_gate_up(const FusedArgs& a, hipStream_t s) {
    FusedCfg c = make_cfg(a, 2, 8);
    launch<EPI_SILU>(a, c, a.W.rows / 128, s);
}

constexpr int HEAD_RG = 4;
int fused_head_blocks(const TMat& E) { return (E.rows + 64 * HEAD_RG - 1) / (64 * HEAD_RG); }

void fused_head(const FusedArgs& a, hipStream_t s) {
    FusedCfg c = make_cfg(a, HEAD_RG, 2);
    launch<EPI_HEAD>(a, c, fused_head_blocks(a.W), s);
}

__device__ __forceinline__ bool beats2(float va, int ia, float vb, int ib) {
    const bool an = isnan(va), bn = isnan(vb);
    if (an != bn) return !an;
    if (an) return ia < ib;
    if (va != vb) return va > vb;
    return ia < ib;
}

// One wavefront per token: lane-strided scan of the block partials, then a shuffle tree.
__global__ void k_head_final(const float* __restrict__ pv, const int* __restrict__ pi, int nblocks,
                             const float* __restrict__ row0, int i0, uint32_t* __restrict__ amax) {
    const int tok = blockIdx.x, lane = threadIdx.x;
    float v = NAN;
    int ix = 0x7fffffff;
    for (int b = lane; b < nblocks; b += 64) {
        const float x = pv[b * FTOK + tok];
        const int xi = pi[b * FTOK + tok];
        if (beats2(x, xi, v, ix)) {
            v = x;
            ix = xi;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o, 64);
        const int oi = __shfl_xor(ix, o, 64);
        if (beats2(ov, oi, v, ix)) {
            v = ov;
            ix = oi;
        }
    }
    if (lane == 0) amax[i0 + tok] = isnan(row0[tok]) ? 0u : uint32_t(ix);
}

void head_argmax_final(const float* pv, const int* pi, int nblocks, const float* row0, int i0, int nt, uint32_t* amax,
                       hipStream_t s) {
    hipLaunchKernelGGL(k_head_final, dim3(nt), dim3(64), 0, s, pv, pi, nblocks, row0, i0, amax);
    FCHECK(hipGetLastError());
}

}  // namespace ls
