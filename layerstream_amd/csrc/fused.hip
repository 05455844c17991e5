// Fused MFMA kernels of the verify step for gfx950 (CDNA4, wave64, v_mfma_f32_16x16x32_bf16).
//
// A launch covers every 16-token tile of its tokens (grid.y). A workgroup owns rg groups of 64
// weight rows and one K range; each of its wavefronts streams four 16-row strips over 128 columns
// of that range (4 k-steps), issuing every weight and input-fragment load of its share at once,
// then converts the int8 / int4 / bf16 weights to bf16 in registers and issues three MFMAs per
// strip and k-step (one per input term). Group scales multiply each group's accumulator. The
// wavefronts of a row group are summed in a fixed order in LDS; when the K range is split over
// several workgroups, each stores its piece and the last one of the row block to arrive (an
// atomic counter) adds the pieces in split order and runs the epilogue. Every output element's
// arithmetic depends only on the matrix shape, never on the number of tokens in the launch: a
// verify pass over k+1 tokens gives the same bits as k+1 single-token passes (src/spec.rs:8-11).
#include "fused.hpp"
#include "attn_dev.hpp"
#include "frag_dev.hpp"
#include "mm_dev.hpp"

#include <hip/hip_ext.h>

#include <algorithm>
#include <cmath>
#include <stdexcept>
#include <string>
#include <type_traits>

namespace ls {

#define FCHECK(x)                                                                                         \
    do {                                                                                                  \
        hipError_t e_ = (x);                                                                              \
        if (e_ != hipSuccess) throw std::runtime_error(std::string("HIP: ") + hipGetErrorString(e_)); \
    } while (0)


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

// One wavefront per source row: the row (reference layout: data, then the bf16 group scales) is
// staged in LDS with coalesced loads; then each lane assembles whole 16-byte lane slots of the
// tile layout (chunk c, lane group lg: columns 32 q + 8 lg + [0, 8) of every k-step q of the
// chunk) and stores each with one 16-byte store; the scales go to [strip][group][16 rows].
// Padding columns get zero weights (int4: nibble 8).
template <int BITS>
__global__ __launch_bounds__(256) void k_tile_repack(const uint8_t* __restrict__ raw, int rows, TMat m, int row_off, int block,
                                                     int stride, int pair_hd, int rpw, int lds_row) {
    extern __shared__ __align__(16) float lds_f[];
    uint8_t* lds = reinterpret_cast<uint8_t*>(lds_f);
    constexpr int CC = BITS == 16 ? 32 : (BITS == 8 ? 64 : 128), Q = CC / 32;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = blockIdx.x * rpw + w;
    const int K = m.cols;
    const int db = BITS == 16 ? 2 * K : K * BITS / 8;
    const int ng_real = BITS == 16 ? 0 : K / m.group;
    const int rb = db + 2 * ng_real;
    uint8_t* L = lds + size_t(w) * lds_row;
    if (r < rows) {
        const uint8_t* row = raw + size_t(r) * rb;
        if (((reinterpret_cast<uintptr_t>(row) | uintptr_t(rb)) & 3) == 0) {
            const uint32_t* r4 = reinterpret_cast<const uint32_t*>(row);
            uint32_t* l4 = reinterpret_cast<uint32_t*>(L);
            for (int i = lane; i < rb / 4; i += 64) l4[i] = r4[i];
        } else {
            for (int i = lane; i < rb; i += 64) L[i] = row[i];
        }
    }
    __syncthreads();
    if (r >= rows) return;
    int lr = r;
    if (pair_hd > 0) {
        const int d = r % pair_hd, half = pair_hd / 2;
        lr = r - d + (d < half ? 2 * d : 2 * (d - half) + 1);
    }
    const int dr = row_off + (lr / block) * stride + lr % block, strip = dr / 16, rl = dr % 16;
    uint8_t* data = const_cast<uint8_t*>(m.data);
    for (int p = lane; p < m.n_chunks * 4; p += 64) {
        const int c = p >> 2, lg = p & 3;
        uint8_t out[16];
#pragma unroll
        for (int i = 0; i < 16; i++) out[i] = BITS == 4 ? 0x88 : 0;
#pragma unroll
        for (int q = 0; q < Q; q++)
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int col = c * CC + 32 * q + 8 * lg + j;
                if (col >= K) continue;
                const uint32_t v = raw_elem(L, BITS, m.group, col);
                if constexpr (BITS == 16) {
                    out[2 * j] = uint8_t(v);
                    out[2 * j + 1] = uint8_t(v >> 8);
                } else if constexpr (BITS == 8) {
                    out[8 * q + j] = uint8_t(v);
                } else {
                    uint8_t& o = out[4 * q + j / 2];
                    o = (j & 1) ? uint8_t((o & 0x0f) | (v << 4)) : uint8_t((o & 0xf0) | v);
                }
            }
        uint4 o4;
        __builtin_memcpy(&o4, out, 16);
        *reinterpret_cast<uint4*>(data + ((size_t(strip) * m.n_chunks + c) * 64 + rl + 16 * lg) * 16) = o4;
    }
    if (BITS != 16) {
        uint16_t* sc = const_cast<uint16_t*>(m.scales);
        for (int g = lane; g < ng_real; g += 64)
            sc[(size_t(strip) * m.n_groups + g) * 16 + rl] = uint16_t(L[db + 2 * g] | (L[db + 2 * g + 1] << 8));
    }
}

constexpr size_t REPACK_LDS = 64 * 1024;  // LDS of one repack workgroup (up to 4 rows)

void tile_repack(const uint8_t* raw, int rows, const TMat& dst, int row_off, int block, int stride, hipStream_t s,
                 int pair_hd) {
    if (rows <= 0) return;
    if (pair_hd > 0 && (pair_hd % 2 || rows % pair_hd)) throw std::runtime_error("RoPE pairing needs whole even heads");
    const int K = dst.cols;
    const size_t rb = dst.bits == 16 ? 2 * size_t(K) : size_t(K) * dst.bits / 8 + 2 * size_t(K / dst.group);
    const size_t lds_row = (rb + 15) / 16 * 16;
    if (lds_row > REPACK_LDS) throw std::runtime_error("row too long for the repack kernel");
    const int rpw = int(std::min<size_t>(4, REPACK_LDS / lds_row));
    const dim3 grid((rows + rpw - 1) / rpw), blk(64 * rpw);
    const size_t lds = size_t(rpw) * lds_row;
    switch (dst.bits) {
        case 16: hipLaunchKernelGGL(k_tile_repack<16>, grid, blk, lds, s, raw, rows, dst, row_off, block, stride, pair_hd, rpw, int(lds_row)); break;
        case 8: hipLaunchKernelGGL(k_tile_repack<8>, grid, blk, lds, s, raw, rows, dst, row_off, block, stride, pair_hd, rpw, int(lds_row)); break;
        default: hipLaunchKernelGGL(k_tile_repack<4>, grid, blk, lds, s, raw, rows, dst, row_off, block, stride, pair_hd, rpw, int(lds_row)); break;
    }
    FCHECK(hipGetLastError());
}

// Row i of x -> fragment slots of token i (x * w when w is set) and per-16-column sums of
// squares. The row (cols values, a multiple of 8) is staged in LDS; one workgroup per token.
__device__ void row_frags(const float* xr, int i, int cols, const float* __restrict__ w, uint8_t* frags, float* ss,
                          float* lds) {
    if (xr != lds)
        for (int c = threadIdx.x; c < cols; c += blockDim.x) lds[c] = xr[c];
    __syncthreads();
    const int tile = i / FTOK, tok = i % FTOK;
    uint8_t* tf = frags + size_t(tile) * frag_tile_bytes(cols);
    for (int sl = threadIdx.x; sl < cols / 8; sl += blockDim.x) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = w ? __fmul_rn(lds[8 * sl + j], w[8 * sl + j]) : lds[8 * sl + j];
        write_slot(tf, sl / 4, tok + 16 * (sl % 4), v);
    }
    if (!ss) return;
    const int slots = ss_slots(cols);
    for (int g = threadIdx.x; g < slots; g += blockDim.x) {
        const int n = min(16, cols - 16 * g);
        ss[(size_t(tile) * slots + g) * FTOK + tok] = ss16([&](int c) { return lds[16 * g + c]; }, n);
    }
}

__global__ __launch_bounds__(256) void k_tile_embed(TMat E, const uint32_t* __restrict__ tokens, float* __restrict__ x,
                                                    const float* __restrict__ w, uint8_t* frags, float* ss, StageMirror sm) {
    extern __shared__ float lds[];
    const int i = blockIdx.x;
    // Host words are read at system scope (past the GPU caches, which may hold an earlier call's).
    const int r = sm.host ? __hip_atomic_load(sm.host + sm.tok_off + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) : int(tokens[i]);
    if (sm.host && i == 0)
        for (int k = threadIdx.x; k < sm.words; k += blockDim.x)
            sm.dev[k] = __hip_atomic_load(sm.host + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    if (sm.epoch && i == 0 && threadIdx.x == 0) sm.epoch[0] += 1;
    const int strip = r / 16, rl = r % 16;
    const int cc = tile_chunk_cols(E.bits);
    float* xr = x + size_t(i) * E.cols;
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
        xr[col] = v;
        lds[col] = v;
    }
    if (frags) row_frags(lds, i, E.cols, w, frags, ss, lds);
}

void tile_embed(const TMat& E, const uint32_t* tokens, int n, float* x, const float* w, uint8_t* frags, float* ss,
                hipStream_t s, const StageMirror& mirror) {
    if (E.cols % 8) throw std::runtime_error("embedding width must be a multiple of 8");
    if (mirror.host && (!mirror.dev || mirror.tok_off < 0 || mirror.tok_off + n > mirror.words))
        throw std::runtime_error("staging mirror does not hold the tokens");
    hipLaunchKernelGGL(k_tile_embed, dim3(n), dim3(256), size_t(E.cols) * 4, s, E, tokens, x, w, frags, ss, mirror);
    FCHECK(hipGetLastError());
}

__global__ __launch_bounds__(256) void k_x_frags(const float* __restrict__ x, int cols, const float* __restrict__ w,
                                                 uint8_t* frags, float* ss) {
    extern __shared__ float lds[];
    row_frags(x + size_t(blockIdx.x) * cols, blockIdx.x, cols, w, frags, ss, lds);
}

void x_frags(const float* x, int n, int cols, const float* w, uint8_t* frags, float* ss, hipStream_t s) {
    if (cols % 8) throw std::runtime_error("row width must be a multiple of 8");
    hipLaunchKernelGGL(k_x_frags, dim3(n), dim3(256), size_t(cols) * 4, s, x, cols, w, frags, ss);
    FCHECK(hipGetLastError());
}


// Dynamic LDS: [wavefront sums (kw > 1)] [tile: 16 S rg rows x 16 floats] [16 inverse rms]
// [flag] [argmax scratch 2 x 256] [epilogue operands staged by the prologue: residual rows
// 16 S rg x 16, per-row vector 16 S rg, RoPE cos and sin 2 x 16 x half, per-token position and
// cache row 2 x 16].
// One matrix workgroup (row block bx / nsplit, K range bx % nsplit, token tile `tile`). With
// IN_FLOW the input (fragments, and the sum-of-squares partials of a normalised input) comes
// from earlier workgroups of the same launch: it is read through the coherent path after
// waiting on fin. With OUT_FLOW the outputs are written through the coherent path and the
// workgroup then signals fout; for the residual epilogue the residual rows themselves were
// written in the same launch, so they too are read coherently after the wait.
template <int BITS, int EPI, bool G16, int S, bool IN_FLOW = false, bool OUT_FLOW = false, bool PRE = false, int WD = 1>
__device__ __forceinline__ void mm_body(const MMArgs& a, const MMPlan& p, const MMScratch& sc, const Flow& fin, const Flow& fout, int bx,
                                        int tile, uint8_t* smem) {
    constexpr int Q = Steps<BITS>::Q, CPW = Steps<BITS>::CPW * WD;  // WD: the plan's wide
    const int nw = p.rg * p.kw, nthr = nw * 64;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int rb = bx / p.nsplit, sp = bx % p.nsplit;
    const int rows_wg = 16 * S * p.rg, row0 = rb * rows_wg;
    const int nt = min(FTOK, a.n - tile * FTOK);
    const TMat& W = a.W;
    const int rgi = wv / p.kw, kw = wv % p.kw;
    const int s0 = (rb * p.rg + rgi) * S;
    const int c0 = (sp * p.kw + kw) * CPW;
    const int nch = min(CPW, W.n_chunks - c0);  // chunks of this wavefront (none when <= 0)

    const size_t red_bytes = p.kw > 1 ? size_t(nw) * S * 64 * 16 : 0;
    float* tl = reinterpret_cast<float*>(smem + red_bytes);
    float* inv = tl + rows_wg * FTOK;
    int* flag = reinterpret_cast<int*>(inv + FTOK);
    float* bv = reinterpret_cast<float*>(flag + 4);
    int* bi = reinterpret_cast<int*>(bv + FTOK * 16);
    float* xs = reinterpret_cast<float*>(bi + FTOK * 16);
    float* vec = xs + rows_wg * FTOK;
    float* rcos = vec + rows_wg;
    float* rsin = rcos + FTOK * (EPI == EPI_QKV ? a.hd / 2 : 0);
    int* tpos = reinterpret_cast<int*>(rsin + FTOK * (EPI == EPI_QKV ? a.hd / 2 : 0));  // [position][cache row] per token
    const int ibase = tile * FTOK;  // launch token index of token 0 of the tile

    // Every load of the wavefront's share (weights, their group scales, and the input when it
    // was written before the launch) is issued before any arithmetic.
    uint4 raw[CPW][S];
    uint4 B[CPW * Q][3];
    // With PRE the group scales are loaded here too (a consumer of in-launch data would otherwise
    // load them only after its wait); launches that are short of registers leave them to the
    // matrix loop, which the compiler schedules ahead by itself when no wait sits in between.
    uint2 scl[PRE ? CPW : 1][PRE ? scale_slots<BITS, G16>() : 1][S];
    {
        const uint8_t* wb = W.data + (size_t(s0) * W.n_chunks * 64 + lane) * 16;
        const size_t sst = size_t(W.n_chunks) * 1024;
        const uint4* fb = reinterpret_cast<const uint4*>(a.frags + size_t(tile) * a.frag_stride) + lane;
#pragma unroll
        for (int c = 0; c < CPW; c++) {
            if (c < nch) {
                load_chunk<S>(wb, sst, c0 + c, raw[c]);
                if constexpr (PRE && BITS != 16) load_scales<BITS, G16, S>(W, s0, c0 + c, (c0 + nch) * Q, scl[c]);
                if constexpr (!IN_FLOW) {
#pragma unroll
                    for (int q = 0; q < Q; q++) {
                        const int ks = (c0 + c) * Q + q;
#pragma unroll
                        for (int t = 0; t < 3; t++) B[c * Q + q][t] = fb[(ks * 3 + t) * 64];
                    }
                }
            }
        }
    }
    // Sum-of-squares partials for 1 / rms (wavefront 0), in flight with the weights.
    RmsLoads rms;
    const bool do_rms = a.ss && wv == 0;
    if (do_rms && !IN_FLOW) rms_issue(a, tile, rms);
    // Residual rows written in this launch (coherent residual epilogue): XR per thread, loaded
    // after the wait.
    constexpr bool XCOH = EPI == EPI_RESID && OUT_FLOW;
    static_assert(!XCOH || IN_FLOW, "a residual epilogue with in-launch consumers also has an in-launch input");
    constexpr int XR = 4;  // the host checks 16 S rg x 16 <= XR x 64 rg kw (S <= kw)
    float xr[XR];
    // Epilogue operands, staged in LDS while the weights are in flight.
    if constexpr (EPI == EPI_RESID) {
        for (int e0 = threadIdx.x; !XCOH && e0 < rows_wg * FTOK; e0 += 4 * nthr) {
            float xv[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int e = e0 + u * nthr, rl = e / FTOK, tok = e % FTOK, row = row0 + rl;
                xv[u] = (e < rows_wg * FTOK && tok < nt && row < W.rows) ? a.out[size_t(ibase + tok) * a.ldo + row] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (e0 + u * nthr < rows_wg * FTOK) xs[e0 + u * nthr] = xv[u];
        }
        if (a.onorm)
            for (int r = threadIdx.x; r < rows_wg; r += nthr) vec[r] = row0 + r < W.rows ? a.onorm[row0 + r] : 0.0f;
    } else if constexpr (EPI == EPI_QKV) {
        const int qk = (a.heads + a.kv_heads) * a.hd;
        for (int r = threadIdx.x; r < rows_wg; r += nthr)
            vec[r] = row0 + r < W.rows ? a.bias[qkv_ref_row(row0 + r, a.hd, qk)] : 0.0f;
        const int half = a.hd / 2;
        const int pos0 = a.row_pos ? 0 : *a.pos0;
        for (int tok = threadIdx.x; tok < nt; tok += nthr) {
            const int i = ibase + tok, pos = a.row_pos ? a.row_pos[i] : pos0 + i;
            tpos[tok] = pos;
            tpos[FTOK + tok] = a.row_seq ? int(a.row_seq[i] * a.seq_stride) + pos : pos;
        }
        for (int e = threadIdx.x; e < nt * half; e += nthr) {
            const int tok = e / half, j = e % half, i = ibase + tok;
            const size_t at = size_t(a.row_pos ? a.row_pos[i] : pos0 + i) * half + j;
            rcos[tok * half + j] = a.rope_cos[at];
            rsin[tok * half + j] = a.rope_sin[at];
        }
    }
    if constexpr (IN_FLOW) {
        // The weights are in flight; touch this workgroup's share of the prefetch range (1 KiB
        // per wavefront load, into LDS that the reduction overwrites later), wait for the input,
        // then read it coherently.
        if (a.pf) {
            const size_t nwg = size_t(p.nrb) * p.nsplit, per = (a.pf_bytes / nwg + 1023) / 1024 * 1024;
            const size_t beg = size_t(bx) * per, end = min(a.pf_bytes, beg + per);
            auto* lds = (__attribute__((address_space(3))) void*)(smem + size_t(wv) * 1024);
            for (size_t off = beg + size_t(wv) * 1024; off < end; off += size_t(nw) * 1024)
                if (off + size_t(lane) * 16 + 16 <= end) __builtin_amdgcn_global_load_lds(a.pf + off + lane * 16, lds, 16, 0, 0);
        }
        flow_wait(fin, sp, rb);
        if (do_rms) rms_issue<true>(a, tile, rms);
        if constexpr (XCOH) {
            const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(a.out, 0, a.n * a.ldo * 4, BUF_DWORD3);
#pragma unroll
            for (int u = 0; u < XR; u++) {
                const int e = threadIdx.x + u * nthr, rl = e / FTOK, tok = e % FTOK, row = row0 + rl;
                xr[u] = (e < rows_wg * FTOK && tok < nt && row < W.rows)
                            ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rx, ((ibase + tok) * a.ldo + row) * 4, 0, CPOL_SC1))
                            : 0.0f;
            }
        }
        const __amdgpu_buffer_rsrc_t rf =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.frags) + size_t(tile) * a.frag_stride, 0, int(a.frag_stride), BUF_DWORD3);
#pragma unroll
        for (int c = 0; c < CPW; c++) {
            if (c < nch) {
#pragma unroll
                for (int q = 0; q < Q; q++) {
                    const int ks = (c0 + c) * Q + q;
#pragma unroll
                    for (int t = 0; t < 3; t++) {
                        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rf, ((ks * 3 + t) * 64 + lane) * 16, 0, CPOL_SC1);
                        B[c * Q + q][t] = make_uint4(v[0], v[1], v[2], v[3]);
                    }
                }
            }
        }
    }

    if (OUT_FLOW && a.tlw && threadIdx.x == 0) {
        __builtin_amdgcn_s_waitcnt(0);
        a.tlw[3] = __builtin_amdgcn_s_memrealtime();
    }
    f32x4 total[S], acc[S];
#pragma unroll
    for (int r = 0; r < S; r++) total[r] = acc[r] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < CPW; c++)
        if (c < nch) chunk_mfma<BITS, G16, S, PRE>(W, s0, c0 + c, c0 * Q, (c0 + nch) * Q, &B[c * Q], raw[c], acc, total, scl[PRE ? c : 0]);
    if (OUT_FLOW && a.tlw && threadIdx.x == 0) a.tlw[4] = __builtin_amdgcn_s_memrealtime();
    // Row-group tile: the kw wavefront sums added in wavefront order. Lane l of strip r holds
    // rows 16 r + 4 (l / 16) + i of token l % 16. Wavefront 0 works out 1 / rms (read after the
    // barriers below) while the other wavefronts finish their products.
    if (p.kw > 1) {
        f32x4* red = reinterpret_cast<f32x4*>(smem);
#pragma unroll
        for (int r = 0; r < S; r++) red[(wv * S + r) * 64 + lane] = total[r];
        if (do_rms) rms_finish<IN_FLOW>(a, tile, W.cols, rms, inv);
        __syncthreads();
        for (int e = threadIdx.x; e < p.rg * S * 64; e += nthr) {
            const int g = e / (S * 64), r = (e / 64) % S, ln = e % 64;
            // All kw reads in flight at once, then the sums in wavefront order.
            f32x4 v[MAX_KW];
#pragma unroll
            for (int k = 0; k < MAX_KW; k++)
                if (k < p.kw) v[k] = red[((g * p.kw + k) * S + r) * 64 + ln];
            f32x4 sum = v[0];
#pragma unroll
            for (int k = 1; k < MAX_KW; k++)
                if (k < p.kw)
#pragma unroll
                    for (int i = 0; i < 4; i++) sum[i] += v[k][i];
#pragma unroll
            for (int i = 0; i < 4; i++) tl[(16 * (S * g + r) + 4 * (ln >> 4) + i) * FTOK + (ln & 15)] = sum[i];
        }
    } else {
        if (do_rms) rms_finish<IN_FLOW>(a, tile, W.cols, rms, inv);
#pragma unroll
        for (int r = 0; r < S; r++)
#pragma unroll
            for (int i = 0; i < 4; i++) tl[(16 * (S * rgi + r) + 4 * (lane >> 4) + i) * FTOK + (lane & 15)] = total[r][i];
    }
    __syncthreads();
    if (OUT_FLOW && a.tlw && threadIdx.x == 0) a.tlw[5] = __builtin_amdgcn_s_memrealtime();

    // Split K: store this piece; the last workgroup of the row block adds all pieces in split
    // order. Pieces move with 128-bit sc1 buffer accesses and the counter with an agent-scope
    // atomic, all coherent across the L2s of the XCDs; the stores are complete (s_waitcnt)
    // before the counter moves.
    if (p.nsplit > 1) {
        const int elems = rows_wg * FTOK, e4n = elems / 4;
        float* base = sc.part + (size_t(tile) * p.nrb + rb) * p.nsplit * elems;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(base, 0, p.nsplit * elems * 4, BUF_DWORD3);
        const f32x4* tl4 = reinterpret_cast<const f32x4*>(tl);
        for (int e4 = threadIdx.x; e4 < e4n; e4 += nthr)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, tl4[e4]), rs, (sp * elems + 4 * e4) * 4, 0, CPOL_SC1);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0) {
            int* cn = sc.cnt + size_t(tile) * p.nrb + rb;
            const int old = __hip_atomic_fetch_add(cn, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int last = old == p.nsplit - 1;
            if (last) __hip_atomic_store(cn, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            flag[0] = last;
        }
        __syncthreads();
        if (!flag[0]) return;
        f32x4* tw = reinterpret_cast<f32x4*>(tl);
        for (int e4 = threadIdx.x; e4 < e4n; e4 += nthr) {
            f32x4 v[MAX_SPLIT];
#pragma unroll
            for (int k = 0; k < MAX_SPLIT; k++)
                if (k < p.nsplit)
                    v[k] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (k * elems + 4 * e4) * 4, 0, CPOL_SC1));
            f32x4 sum = v[0];
#pragma unroll
            for (int k = 1; k < MAX_SPLIT; k++)
                if (k < p.nsplit)
#pragma unroll
                    for (int i = 0; i < 4; i++) sum[i] += v[k][i];
            tw[e4] = sum;
        }
        __syncthreads();
    }

    if constexpr (EPI == EPI_QKV) {
        // Tile rows: q heads, k heads (RoPE pairs adjacent), v heads (src/kernels.rs:242-252).
        // With OUT_FLOW the rows go through the coherent path for this launch's attention.
        const int hd = a.hd, half = hd / 2, h = a.heads * hd, kvd = a.kv_heads * hd;
        const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(a.out, 0, a.n * a.ldo * 4, BUF_DWORD3);
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(a.kcache, 0, 0x7ffffffc, BUF_DWORD3);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(a.vcache, 0, 0x7ffffffc, BUF_DWORD3);
        for (int e = threadIdx.x; e < rows_wg * FTOK; e += nthr) {
            const int rl = e / FTOK, tok = e % FTOK, row = row0 + rl;
            if (tok >= nt || row >= W.rows) continue;
            const int i = ibase + tok, crow = tpos[FTOK + tok];  // cache row
            const float iv = a.ss ? inv[tok] : 1.0f;
            float v = __fadd_rn(a.ss ? __fmul_rn(tl[e], iv) : tl[e], vec[rl]);
            int ref = row;
            if (row < h + kvd) {
                const int r = row % hd, j = r >> 1, pr = rl ^ 1;
                const float pv = __fadd_rn(a.ss ? __fmul_rn(tl[pr * FTOK + tok], iv) : tl[pr * FTOK + tok], vec[pr]);
                const float c = rcos[tok * half + j], sn = rsin[tok * half + j];
                if ((r & 1) == 0) {
                    v = __fsub_rn(__fmul_rn(v, c), __fmul_rn(pv, sn));  // dimension j: x_j c - x_{j+half} s
                    ref = row - r + j;
                } else {
                    v = __fadd_rn(__fmul_rn(v, c), __fmul_rn(pv, sn));  // dimension j + half: x c + x_j s
                    ref = row - r + half + j;
                }
            }
            if constexpr (OUT_FLOW) {
                if (ref < h) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), rq, (i * a.ldo + ref) * 4, 0, CPOL_SC1);
                else if (ref < h + kvd) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), rk, (crow * kvd + ref - h) * 4, 0, CPOL_SC1);
                else __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), rv, (crow * kvd + ref - h - kvd) * 4, 0, CPOL_SC1);
            } else {
                if (ref < h) a.out[size_t(i) * a.ldo + ref] = v;
                else if (ref < h + kvd) a.kcache[size_t(crow) * kvd + (ref - h)] = v;
                else a.vcache[size_t(crow) * kvd + (ref - h - kvd)] = v;
            }
        }
        if (OUT_FLOW && a.tlw && threadIdx.x == 0) a.tlw[6] = __builtin_amdgcn_s_memrealtime();
        if constexpr (OUT_FLOW) qkv_signal(fout, rb * S, a.heads, a.kv_heads, a.hd);
    } else if constexpr (EPI == EPI_RESID) {
        if constexpr (XCOH) {
            // Residual rows, fragments and partials all go through the coherent path. The new
            // rows stay in xr until after the barrier below: a barrier waits for the wavefront's
            // outstanding stores, so every store of this epilogue is issued after it.
#pragma unroll
            for (int u = 0; u < XR; u++) {
                const int e = threadIdx.x + u * nthr, rl = e / FTOK, tok = e % FTOK, row = row0 + rl;
                if (e < rows_wg * FTOK) {
                    const float xn = tok < nt && row < W.rows ? __fadd_rn(xr[u], tl[e]) : 0.0f;
                    xr[u] = xn;
                    tl[e] = xn;
                }
            }
        } else {
            for (int e = threadIdx.x; e < rows_wg * FTOK; e += nthr) {
                const int rl = e / FTOK, tok = e % FTOK, row = row0 + rl;
                float xn = 0.0f;
                if (tok < nt && row < W.rows) {
                    xn = __fadd_rn(xs[e], tl[e]);
                    a.out[size_t(ibase + tok) * a.ldo + row] = xn;
                }
                tl[e] = xn;
            }
        }
        __syncthreads();
        if (a.ofrags) {
            uint8_t* tf = a.ofrags + size_t(tile) * a.ofrag_stride;
            const __amdgpu_buffer_rsrc_t rof = __builtin_amdgcn_make_buffer_rsrc(tf, 0, int(a.ofrag_stride), BUF_DWORD3);
            for (int q = threadIdx.x; q < (rows_wg / 8) * FTOK; q += nthr) {
                const int cg = q / FTOK, tok = q % FTOK, col = row0 + 8 * cg;
                float v[8];
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float x = tl[(8 * cg + j) * FTOK + tok];
                    v[j] = a.onorm ? __fmul_rn(x, vec[8 * cg + j]) : x;
                }
                if constexpr (XCOH) write_slot_coherent(rof, 0, col / 32, tok + 16 * ((col % 32) / 8), v);
                else write_slot(tf, col / 32, tok + 16 * ((col % 32) / 8), v);
            }
        }
        if (a.oss) {
            const __amdgpu_buffer_rsrc_t ros =
                __builtin_amdgcn_make_buffer_rsrc(a.oss + size_t(tile) * a.oss_slots * FTOK, 0, a.oss_slots * FTOK * 4, BUF_DWORD3);
            for (int q = threadIdx.x; q < (rows_wg / 16) * FTOK; q += nthr) {
                const int g = q / FTOK, tok = q % FTOK, slot = row0 / 16 + g;
                if (slot >= a.oss_slots) continue;
                const float v = ss16([&](int c) { return tl[(16 * g + c) * FTOK + tok]; }, 16);
                if constexpr (XCOH) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), ros, (slot * FTOK + tok) * 4, 0, CPOL_SC1);
                else a.oss[(size_t(tile) * a.oss_slots + slot) * FTOK + tok] = v;
            }
        }
        if constexpr (XCOH) {
            const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(a.out, 0, a.n * a.ldo * 4, BUF_DWORD3);
#pragma unroll
            for (int u = 0; u < XR; u++) {
                const int e = threadIdx.x + u * nthr, rl = e / FTOK, tok = e % FTOK, row = row0 + rl;
                if (e < rows_wg * FTOK && tok < nt && row < W.rows)
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(xr[u]), rx, ((ibase + tok) * a.ldo + row) * 4, 0, CPOL_SC1);
            }
            if (OUT_FLOW && a.tlw && threadIdx.x == 0) a.tlw[6] = __builtin_amdgcn_s_memrealtime();
            flow_signal(fout, rb);
        }
    } else if constexpr (EPI == EPI_SILU) {
        // rows: [h gate rows | h up rows] for act columns h rb + [0, h), h = rows_wg / 2. Each
        // thread forms one SiLU(g) * u value in place of its gate value, then the fragments.
        const int hw = rows_wg / 2;
        uint8_t* tf = a.ofrags + size_t(tile) * a.ofrag_stride;
        const __amdgpu_buffer_rsrc_t rof = __builtin_amdgcn_make_buffer_rsrc(tf, 0, int(a.ofrag_stride), BUF_DWORD3);
        for (int e = threadIdx.x; e < hw * FTOK; e += nthr) {
            const int tok = e % FTOK;
            float v = 0.0f;
            if (tok < nt) {
                float g = tl[e], up = tl[hw * FTOK + e];
                if (a.ss) {
                    g = __fmul_rn(g, inv[tok]);
                    up = __fmul_rn(up, inv[tok]);
                }
                v = __fmul_rn(g / (1.0f + expf(-g)), up);
            }
            tl[e] = v;
        }
        __syncthreads();
        for (int q = threadIdx.x; q < (hw / 8) * FTOK; q += nthr) {
            const int cg = q / FTOK, tok = q % FTOK, col = hw * rb + 8 * cg;
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = tl[(8 * cg + j) * FTOK + tok];
            if constexpr (OUT_FLOW) write_slot_coherent(rof, 0, col / 32, tok + 16 * ((col % 32) / 8), v);
            else write_slot(tf, col / 32, tok + 16 * ((col % 32) / 8), v);
        }
        if (OUT_FLOW && a.tlw && threadIdx.x == 0) a.tlw[6] = __builtin_amdgcn_s_memrealtime();
        if constexpr (OUT_FLOW) flow_signal(fout, rb);
    } else {
        // Output head: logits, optional store, per-token best (value, index) of this block.
        for (int e = threadIdx.x; e < rows_wg * FTOK; e += nthr) {
            const int rl = e / FTOK, tok = e % FTOK, row = row0 + rl;
            if (tok >= nt || row >= W.rows) continue;
            const float v = a.ss ? __fmul_rn(tl[e], inv[tok]) : tl[e];
            tl[e] = v;
            if (a.out) a.out[size_t(ibase + tok) * a.ldo + a.row_base + row] = v;
        }
        __syncthreads();
        for (int e = threadIdx.x; e < FTOK * 16; e += nthr) {
            const int tok = e % FTOK, part = e / FTOK;
            float v = NAN;
            int ix = 0x7fffffff;
            for (int rl = part; rl < rows_wg; rl += 16) {
                const int row = row0 + rl;
                if (row >= W.rows) break;
                const float x = tl[rl * FTOK + tok];
                if (beats(x, a.row_base + row, v, ix)) {
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
            for (int q = 1; q < 16; q++) {
                const float x = bv[tok * 16 + q];
                const int xi = bi[tok * 16 + q];
                if (beats(x, xi, v, ix)) {
                    v = x;
                    ix = xi;
                }
            }
            const size_t at = (size_t(tile) * a.arg_stride + a.arg_off + rb) * FTOK + tok;
            a.arg_val[at] = v;
            a.arg_idx[at] = ix;
            if (rb == 0 && a.row0) a.row0[ibase + tok] = tl[tok];
        }
    }
}

// Workgroup -> (row block and split, token tile) of a launch over several tiles. Workgroups go
// to the 8 XCDs in turn (dispatch index L to XCD L % 8); each XCD gets a contiguous run of
// (row block, tile) pairs, row block major, so the tiles of one row block run side by side on
// one XCD and all but the first read its weights from that XCD's L2. Any order gives the same
// bits: only which workgroup computes a piece changes.
__device__ __forceinline__ void xcd_tile_map(int& bx, int& tile) {
    const int tiles = gridDim.y, G = gridDim.x * tiles;
    const int L = blockIdx.x + blockIdx.y * gridDim.x;
    const int x = L % 8, k = L / 8, base = G / 8, rem = G % 8;
    const int P = x * base + min(x, rem) + k;
    bx = P / tiles;
    tile = P % tiles;
}

// The same for a launch with a K split: each XCD gets a contiguous run of (split, tile, row block)
// triples, row block innermost, so the row blocks that read one split of one tile's input
// fragments run side by side on one XCD (the fragments, 96 B per input column and token tile, are
// what a down launch over 9 tiles mostly fetched: 47 MB per launch for 4.4 MB of weights), and a
// run covers several tiles of a split, whose weights the L2 then serves again.
__device__ __forceinline__ void xcd_split_map(int& bx, int& tile, int nsplit) {
    const int tiles = gridDim.y, G = gridDim.x * tiles, nrb = gridDim.x / nsplit;
    const int L = blockIdx.x + blockIdx.y * gridDim.x;
    const int x = L % 8, k = L / 8, base = G / 8, rem = G % 8;
    const int P = x * base + min(x, rem) + k;
    const int rb = P % nrb, rest = P / nrb;
    tile = rest % tiles;
    bx = rb * nsplit + rest / tiles;
}

template <int BITS, int EPI, bool G16, int S, int WD = 1>
__global__ __launch_bounds__((WD > 1 ? 8 : mm_max_waves(BITS, G16 ? 16 : 32, S)) * 64) void k_mm(MMArgs a, MMPlan p, MMScratch sc) {
    extern __shared__ __align__(16) uint8_t smem[];
    int bx = blockIdx.x, tile = blockIdx.y;
    if (gridDim.y > 1) {
        if (p.nsplit > 1) xcd_split_map(bx, tile, p.nsplit);
        else xcd_tile_map(bx, tile);
    }
    mm_body<BITS, EPI, G16, S, false, false, false, WD>(a, p, sc, Flow{}, Flow{}, bx, tile, smem);
}

// ---------------------------------------------------------------------------------------
// Pipelined gate|up over one token tile
// ---------------------------------------------------------------------------------------
// For a gate|up matrix with more strip pairs than the device has CUs (the 3B shape: 688): one
// workgroup per CU walks a contiguous, balanced range of items (a gate strip and its up strip),
// each of its 8 wavefronts covering 2 of the plan's K shares. A wavefront's input fragments are
// loaded once and stay in its registers; the weights and group scales of the next two items are
// in flight while the current one is reduced across the shares and its epilogue runs. Inside the
// loop the wavefronts issue loads only, the same ones every iteration (loads complete in order,
// so each wait covers just the item it needs; pending stores would make every wait a full one),
// and the SiLU fragments are staged in LDS and stored after the loop. Each value is summed as k_mm
// sums it under the same plan (share totals in share order), so both give the same bits.
// Measured on the 3B shape (45 MB): 15.4 us against 17.8 us for k_mm.

constexpr int PIPE_WAVES = 8, PIPE_SPW = 2, PIPE_NBUF = 2;
constexpr size_t PIPE_MAX_BYTES = size_t(1) << 30;  // weights and scales of a pipelined matrix, at most

// Weights and group scales of one item for one wavefront: the gate and up strips over the chunks
// of its PIPE_SPW shares. Groups of GK k-steps lie inside one chunk (GK divides Q): a scale is read
// only for a group's last k-step.
template <int BITS, int GK>
struct PipeW {
    static constexpr int Q = Steps<BITS>::Q, CPW = Steps<BITS>::CPW, SLOTS = BITS == 16 ? 1 : Q / GK;
    uint4 raw[PIPE_SPW][CPW][2];
    uint2 scl[PIPE_SPW][CPW][SLOTS][2];
};

// Buffer loads: an item past the workgroup's range names strips past the matrix, whose offsets
// lie beyond the resource; the hardware range check answers them with zeros and no memory
// access, so every iteration issues the same loads whether or not its item exists (offsets stay
// below 2^31: checked on the host).
template <int BITS, int GK>
__device__ __forceinline__ void pipe_load(const TMat& W, __amdgpu_buffer_rsrc_t rw, __amdgpu_buffer_rsrc_t rsc, const int* st, int cbase,
                                          PipeW<BITS, GK>& w) {
    using P = PipeW<BITS, GK>;
    const int lane = threadIdx.x & 63;
    const uint32_t sst = uint32_t(W.n_chunks) * 1024;
#pragma unroll
    for (int u = 0; u < PIPE_SPW; u++)
#pragma unroll
        for (int c = 0; c < P::CPW; c++) {
            const int cc = min(cbase + u * P::CPW + c, W.n_chunks - 1);
#pragma unroll
            for (int r = 0; r < 2; r++) {
                const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rw, uint32_t(st[r]) * sst + uint32_t(cc) * 1024 + lane * 16, 0, CPOL_NT);
                w.raw[u][c][r] = make_uint4(v[0], v[1], v[2], v[3]);
            }
            if constexpr (BITS != 16) {
#pragma unroll
                for (int g = 0; g < P::SLOTS; g++)
#pragma unroll
                    for (int r = 0; r < 2; r++) {
                        const uint32_t off = ((uint32_t(st[r]) * W.n_groups + cc * P::Q / GK + g) * 16 + 4 * (lane >> 4)) * 2;
                        const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rsc, off, 0, 0);
                        w.scl[u][c][g][r] = make_uint2(v[0], v[1]);
                    }
            }
        }
}

// One chunk of one share: chunk_mfma's arithmetic for groups that end inside the chunk.
template <int BITS, int GK>
__device__ __forceinline__ void pipe_chunk(const uint4 (*B)[3], const PipeW<BITS, GK>& w, int u, int c, f32x4* acc, f32x4* total) {
    constexpr int Q = Steps<BITS>::Q;
#pragma unroll
    for (int q = 0; q < Q; q++) {
        if constexpr (BITS == 16) {
#pragma unroll
            for (int r = 0; r < 2; r++) total[r] = mfma3(a_operand<BITS>(w.raw[u][c][r], q), B[q], total[r]);
        } else {
            const bool first = q % GK == 0, last = (q + 1) % GK == 0;
#pragma unroll
            for (int r = 0; r < 2; r++) acc[r] = mfma3(a_operand<BITS>(w.raw[u][c][r], q), B[q], first ? f32x4{0, 0, 0, 0} : acc[r]);
            if (last) {
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    const f32x4 sc = scales_f32(w.scl[u][c][q / GK][r]);
#pragma unroll
                    for (int i = 0; i < 4; i++) total[r][i] = __builtin_fmaf(sc[i], acc[r][i], total[r][i]);
                }
            }
        }
    }
}

// LDS of the pipelined gate|up: share totals, the item's 32 x FTOK tile, 1 / rms and the staged
// fragments (3 x 16 bytes per (column group, token)) of up to `most` items.
__host__ __device__ constexpr size_t pipe_lds_bytes(int kw, int most) {
    return size_t(kw) * 2 * 64 * 16 + (32 * FTOK + FTOK) * 4 + size_t(most) * 2 * FTOK * 48;
}

template <int BITS, int GK>
__global__ __launch_bounds__(PIPE_WAVES * 64) void k_gu_pipe(MMArgs a, MMPlan p, int most) {
    constexpr int Q = Steps<BITS>::Q, CPW = Steps<BITS>::CPW, NBUF = PIPE_NBUF, SPW = PIPE_SPW;
    using PW = PipeW<BITS, GK>;
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int nthr = PIPE_WAVES * 64;
    const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const TMat& W = a.W;
    const int nt = min(FTOK, a.n), kw = p.kw;
    const int items = p.nrb * GU_STRIPS;
    const int i0 = int(int64_t(blockIdx.x) * items / gridDim.x), i1 = int(int64_t(blockIdx.x + 1) * items / gridDim.x);
    const int cbase = wv * SPW * CPW;  // first chunk of this wavefront's shares

    f32x4* red = reinterpret_cast<f32x4*>(smem);                             // [kw][2 strips][64 lanes]
    float* tl = reinterpret_cast<float*>(smem + size_t(kw) * 2 * 64 * 16);  // [32 rows][FTOK]
    float* inv = tl + 32 * FTOK;                                             // [FTOK]
    uint4* stage = reinterpret_cast<uint4*>(inv + FTOK);                     // [most][2][FTOK][3]

    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(W.data), 0,
                                                                       int(size_t(W.n_strips) * W.n_chunks * 1024), BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t rsc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(W.scales), 0,
                                                                        BITS == 16 ? 0 : int(size_t(W.n_strips) * W.n_groups * 32), BUF_DWORD3);
    // Item j of the range: the gate strip and its up strip of row block it / GU_STRIPS; past the
    // range's end, item `items`, whose strips lie past the matrix.
    auto load = [&](int j, PW& w) {
        const int it = i0 + j < i1 ? i0 + j : items;
        int st[2];
        st[0] = (it / GU_STRIPS) * 2 * GU_STRIPS + it % GU_STRIPS;
        st[1] = st[0] + GU_STRIPS;
        pipe_load<BITS, GK>(W, rw, rsc, st, cbase, w);
    };

    // Issue order: norm partials, fragments, the first item's weights, then (once wavefront 0 has
    // its partials) the second's.
    RmsLoads rms;
    const bool do_rms = a.ss && wv == 0;
    if (do_rms) rms_issue(a, 0, rms);
    uint4 B[SPW][CPW * Q][3];
    {
        const uint4* fb = reinterpret_cast<const uint4*>(a.frags) + lane;
        const int ks_last = W.n_chunks * Q - 1;
#pragma unroll
        for (int u = 0; u < SPW; u++)
#pragma unroll
            for (int c = 0; c < CPW; c++)
#pragma unroll
                for (int q = 0; q < Q; q++) {
                    const int ks = min((cbase + u * CPW + c) * Q + q, ks_last);
#pragma unroll
                    for (int t = 0; t < 3; t++) B[u][c * Q + q][t] = fb[(ks * 3 + t) * 64];
                }
    }
    PW w0, w1;
    load(0, w0);
    if (do_rms) rms_finish(a, 0, W.cols, rms, inv);
    load(1, w1);

    // Every workgroup runs `most` items, those past its range on zeros (no memory access). With
    // PF the item NBUF ahead is requested once this one's MFMAs have their operands.
    auto run = [&](int j, PW& w, auto pf) {
        const bool ok = i0 + j < i1;
        f32x4 acc[SPW][2], total[SPW][2];
#pragma unroll
        for (int u = 0; u < SPW; u++)
#pragma unroll
            for (int r = 0; r < 2; r++) acc[u][r] = total[u][r] = f32x4{0, 0, 0, 0};
#pragma unroll
        for (int u = 0; u < SPW; u++) {
            const int nch = min(CPW, W.n_chunks - (cbase + u * CPW));
#pragma unroll
            for (int c = 0; c < CPW; c++)
                if (c < nch) pipe_chunk<BITS, GK>(&B[u][c * Q], w, u, c, acc[u], total[u]);
        }
        if constexpr (decltype(pf)::value) load(j + NBUF, w);
#pragma unroll
        for (int u = 0; u < SPW; u++)
#pragma unroll
            for (int r = 0; r < 2; r++) red[((wv * SPW + u) * 2 + r) * 64 + lane] = total[u][r];
        __syncthreads();
        // The kw share totals of each value, added in share order (one value per thread).
        {
            const int r = tid / 256, ln = (tid / 4) % 64, i = tid % 4;
            const float* rf = reinterpret_cast<const float*>(red);
            float v[MAX_KW];
#pragma unroll
            for (int jj = 0; jj < MAX_KW; jj++) v[jj] = jj < kw ? rf[((jj * 2 + r) * 64 + ln) * 4 + i] : 0.0f;
            float sum = v[0];
#pragma unroll
            for (int jj = 1; jj < MAX_KW; jj++)
                if (jj < kw) sum += v[jj];
            tl[(16 * r + 4 * (ln >> 4) + i) * FTOK + (ln & 15)] = sum;
        }
        __syncthreads();
        // tl rows 0-15: the gate strip, 16-31: its up strip. Thread (row, token): SiLU(g) * u, its
        // three bf16 terms staged at element row % 8 of fragment slot (row / 8, token).
        if (ok && tid < 16 * FTOK) {
            const int rl = tid / FTOK, tok = tid % FTOK;
            float g = tl[rl * FTOK + tok], up = tl[(16 + rl) * FTOK + tok], o = 0.0f;
            if (tok < nt) {
                if (a.ss) {
                    g = __fmul_rn(g, inv[tok]);
                    up = __fmul_rn(up, inv[tok]);
                }
                o = __fmul_rn(g / (1.0f + expf(-g)), up);
            }
            uint32_t h, m, l;
            split3(o, h, m, l);
            uint16_t* d = reinterpret_cast<uint16_t*>(stage + (size_t(j) * 2 * FTOK + (rl / 8) * FTOK + tok) * 3) + rl % 8;
            d[0] = uint16_t(h);
            d[8] = uint16_t(m);
            d[16] = uint16_t(l);
        }
    };
    using PF = std::integral_constant<bool, true>;
    using NOPF = std::integral_constant<bool, false>;
    int j = 0;
    for (; j + NBUF <= most; j += NBUF) {
        run(j, w0, PF{});
        run(j + 1, w1, PF{});
    }
    if (j < most) run(j, w0, NOPF{});  // one item left, already in flight
    __syncthreads();
    // The staged fragments: (item, column group, token) -> fragment slot of act columns
    // 16 GU_STRIPS rb + 16 (item % GU_STRIPS) + 8 group + [0, 8).
    for (int e = tid; e < (i1 - i0) * 2 * FTOK; e += nthr) {
        const int it = i0 + e / (2 * FTOK), cg = (e / FTOK) % 2, tok = e % FTOK;
        const int col = (it / GU_STRIPS) * 16 * GU_STRIPS + 16 * (it % GU_STRIPS) + 8 * cg;
        uint4* o = reinterpret_cast<uint4*>(a.ofrags + (size_t(col / 32) * 3 * 64 + tok + 16 * ((col % 32) / 8)) * 16);
        const uint4* d = stage + size_t(e) * 3;
        o[0] = d[0];
        o[64] = d[1];
        o[128] = d[2];
    }
}

// gate|up and down in one launch (one token tile): workgroups [0, n_gu) run gate|up and count
// themselves done once their SiLU fragments are stored; the down workgroups after them load
// their weights, wait for the gate|up row blocks that produce their K range, then read the
// fragments. Every gate|up workgroup has a lower index than every down workgroup, so it is
// dispatched first and a waiting down workgroup never holds back one it waits for.
template <int BITS, bool G16>
__global__ __launch_bounds__(1024) void k_gu_down(MMArgs gu, MMPlan pgu, MMArgs dn, MMPlan pdn, MMScratch sc, Flow fl) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int ngu = pgu.nrb * pgu.nsplit;
    if (int(blockIdx.x) < ngu) {
        if (int(threadIdx.x) >= 64 * pgu.rg * pgu.kw) return;
        mm_body<BITS, EPI_SILU, G16, gu_wave_strips(BITS, G16 ? 16 : 32), false, true>(gu, pgu, sc, Flow{}, fl, blockIdx.x, 0, smem);
    } else {
        if (int(threadIdx.x) >= 64 * pdn.rg * pdn.kw) return;
        mm_body<BITS, EPI_RESID, G16, DOWN_STRIPS, true, false>(dn, pdn, sc, fl, Flow{}, blockIdx.x - ngu, 0, smem);
    }
}

// Attention and the o projection in one launch (one token tile): workgroups [0, ASPLIT heads)
// run attention, and the one that merges a head's states writes its output fragments through
// the coherent path and counts the head done; the o workgroups after them load their weights,
// wait for every head, then read the fragments coherently. Every attention workgroup has a lower
// index than every o workgroup, so it is dispatched first, and it never waits.
template <int HD, int BITS, bool G16>
__global__ __launch_bounds__(512) void k_attn_o(AttnArgs aa, MMArgs o, MMPlan po, MMScratch sc, Flow fl) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int na = ASPLIT * aa.heads;
    if (int(blockIdx.x) < na) {
        if (int(threadIdx.x) >= AWV * 64) return;
        attn_body<HD, true>(aa, int(blockIdx.x) % ASPLIT, int(blockIdx.x) / ASPLIT, 0, fl, smem);
    } else {
        if (int(threadIdx.x) >= 64 * po.rg * po.kw) return;
        mm_body<BITS, EPI_RESID, G16, 1, true, false>(o, po, sc, fl, Flow{}, int(blockIdx.x) - na, 0, smem);
    }
}

// q|k|v, attention and o in one launch (one token tile): workgroups [0, nq) are the q|k|v strips
// (producers of the per-head counters), then ASPLIT per head run attention (consumers of their
// head's counter, producers of the o counter), then the o workgroups. Every workgroup waits only
// for workgroups with lower indices, which are dispatched before it.
template <int HD, int BITS, bool G16>
__global__ __launch_bounds__(512) void k_qkv_attn_o(MMArgs qa, MMPlan pq, AttnArgs aa, MMArgs o, MMPlan po, MMScratch sc, Flow fq,
                                                    Flow fo) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int nq = pq.nrb * pq.nsplit, na = ASPLIT * aa.heads, bid = blockIdx.x;
    if (bid < nq) {
        if (int(threadIdx.x) >= 64 * pq.rg * pq.kw) return;
        mm_body<BITS, EPI_QKV, G16, 1, false, true>(qa, pq, sc, Flow{}, fq, bid, 0, smem);
    } else if (bid < nq + na) {
        if (int(threadIdx.x) >= AWV * 64) return;
        attn_body<HD, true, true>(aa, (bid - nq) % ASPLIT, (bid - nq) / ASPLIT, 0, fo, smem, fq);
    } else {
        if (int(threadIdx.x) >= 64 * po.rg * po.kw) return;
        mm_body<BITS, EPI_RESID, G16, 1, true, false>(o, po, sc, fo, Flow{}, bid - nq - na, 0, smem);
    }
}

// Every layer of a one-tile pass in one launch. The workgroups of layer l follow those of layer
// l - 1, and inside a layer come q|k|v (one per strip), attention (ASPLIT per head), o, gate|up
// and down (K splits of a row block side by side), so every workgroup waits only for workgroups
// with lower indices. Those are dispatched before it: whatever the number of workgroups resident
// at once, the lowest unfinished one always has its inputs, and the launch cannot deadlock.
// Workgroups of later stages and layers are dispatched while earlier ones still wait or work,
// issue their weight loads at once, and only then wait for their input. Counters (per layer,
// FLOW_LAYER_STRIDE apart): q|k|v -> attention one per head, attention -> o, o -> gate|up,
// gate|up -> down one per down K split, down -> the next layer's q|k|v.
// QS, OS, DS: strips per wavefront of q|k|v, o and down (WD and the strips: the plans' wide and s).
// TL: the per-workgroup timeline (LayerFlows::tl) is recorded.
template <int HD, int BITS, bool G16, int WD = 1, int QS = 1, int OS = 1, int DS = DOWN_STRIPS, bool TL = false>
__global__ __launch_bounds__(512) void k_layers(const LayerPtrs* __restrict__ lp, size_t seq_off, MMArgs qa, MMPlan pq, AttnArgs aa,
                                                MMArgs oa, MMPlan po, MMArgs ga, MMPlan pg, MMArgs da, MMPlan pd, MMScratch sc,
                                                LayerFlows lf) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int nq = pq.nrb, na = ASPLIT * aa.heads, no = po.nrb, ng = pg.nrb, nd = pd.nrb * pd.nsplit;
    const int per_layer = nq + na + no + ng + nd;
    const int l = int(blockIdx.x) / per_layer;
    int r = int(blockIdx.x) % per_layer;
    const LayerPtrs& P = lp[l];
    const int base = FLOW_COUNTERS + FLOW_LAYER_STRIDE * l;
    const bool last = l + 1 == lf.layers;
    unsigned long long* tl = TL ? lf.tl + size_t(blockIdx.x) * 8 : nullptr;
    if (tl && threadIdx.x == 0) {
        tl[0] = __builtin_amdgcn_s_memrealtime();
        tl[1] = tl[3] = tl[4] = tl[5] = tl[6] = 0;  // stamps this workgroup may not reach (or not wait for)
        const int rr = int(blockIdx.x) % per_layer;
        tl[7] = (unsigned long long)(l) << 8 | (rr < nq ? 0 : rr < nq + na ? 1 : rr < nq + na + no ? 2 : rr < nq + na + no + ng ? 3 : 4);
    }
    if (r < nq) {
        if (int(threadIdx.x) >= 64 * pq.kw) return;
        MMArgs a = qa;
        a.W = P.qkv;
        a.tlw = tl;
        a.bias = P.b_qkv;
        a.kcache = P.kc + seq_off;
        a.vcache = P.vc + seq_off;
        Flow fin;  // the previous layer's down row blocks (layer 0: written before the launch)
        if (l > 0) {
            fin.ctl = lf.ctl;
            fin.producers = fin.per = pd.nrb;
            fin.base = base - FLOW_LAYER_STRIDE + FL_D;
            fin.mirrors = lf.m_d;
            fin.stamp = tl ? tl + 1 : nullptr;
        }
        Flow fout;
        fout.ctl = lf.ctl;
        fout.producers = nq;
        fout.want = 3 * (HD / 16) / QS;
        fout.base = base + FL_Q;
        if (l > 0 && r == 0) {
            // Every workgroup of the previous layer's gate|up and down has finished waiting (the
            // down row blocks this workgroup waited for merged every K split).
            fout.zero0 = base - FLOW_LAYER_STRIDE + FL_O;
            fout.nzero0 = lf.m_o;
            fout.zero1 = base - FLOW_LAYER_STRIDE + FL_G;
            fout.nzero1 = (pg.nrb + lf.gu_per - 1) / lf.gu_per * lf.m_g;
        }
        mm_body<BITS, EPI_QKV, G16, QS, true, true, true, WD>(a, pq, sc, fin, fout, r, 0, smem);
        if (tl && threadIdx.x == 0) tl[2] = __builtin_amdgcn_s_memrealtime();
        return;
    }
    r -= nq;
    if (r < na) {
        if (int(threadIdx.x) >= AWV * 64) return;
        AttnArgs A = aa;
        A.kc = P.kc + seq_off;
        A.vc = P.vc + seq_off;
        Flow fin;
        fin.ctl = lf.ctl;
        fin.producers = nq;
        fin.want = 3 * (HD / 16) / QS;
        fin.base = base + FL_Q;
        fin.stamp = tl ? tl + 1 : nullptr;
        Flow fout;
        fout.ctl = lf.ctl;
        fout.producers = fout.per = aa.heads;
        fout.base = base + FL_A;
        fout.mirrors = lf.m_a;
        attn_body<HD, true, true>(A, r % ASPLIT, r / ASPLIT, 0, fout, smem, fin);
        if (tl && threadIdx.x == 0) tl[2] = __builtin_amdgcn_s_memrealtime();
        return;
    }
    r -= na;
    // Counters of these flows go back to zero in the next layer's first q|k|v workgroup; after the
    // last layer there is none, so there the consumers count themselves.
    Flow fo;  // o -> gate|up
    fo.ctl = lf.ctl;
    fo.producers = fo.per = no;
    fo.consumers = last ? ng : 0;
    fo.base = base + FL_O;
    fo.mirrors = lf.m_o;
    Flow fg;  // gate|up -> down, one counter per down K split
    fg.ctl = lf.ctl;
    fg.producers = ng;
    fg.per = lf.gu_per;
    fg.consumers = last ? pd.nrb : 0;
    fg.base = base + FL_G;
    fg.mirrors = lf.m_g;
    if (r < no) {
        if (int(threadIdx.x) >= 64 * po.rg * po.kw) return;
        MMArgs a = oa;
        a.W = P.o;
        a.tlw = tl;
        a.onorm = P.post_norm;
        Flow fin;
        fin.ctl = lf.ctl;
        fin.producers = fin.per = aa.heads;
        fin.base = base + FL_A;
        fin.mirrors = lf.m_a;
        fin.stamp = tl ? tl + 1 : nullptr;
        if (r == 0) {
            // Every attention workgroup of this layer, and so every q|k|v workgroup, has finished
            // waiting (all heads merged).
            fo.zero0 = base + FL_Q;
            fo.nzero0 = aa.heads;
            if (l > 0) {
                fo.zero1 = base - FLOW_LAYER_STRIDE + FL_D;
                fo.nzero1 = lf.m_d;
            }
        }
        mm_body<BITS, EPI_RESID, G16, OS, true, true, true, WD>(a, po, sc, fin, fo, r, 0, smem);
        if (tl && threadIdx.x == 0) tl[2] = __builtin_amdgcn_s_memrealtime();
        return;
    }
    r -= no;
    if (r < ng) {
        if (int(threadIdx.x) >= 64 * pg.rg * pg.kw) return;
        MMArgs a = ga;
        a.W = P.gu;
        a.tlw = tl;
        if (r == 0) {
            // Every o workgroup of this layer has finished waiting.
            fg.zero0 = base + FL_A;
            fg.nzero0 = lf.m_a;
        }
        fo.stamp = tl ? tl + 1 : nullptr;
        mm_body<BITS, EPI_SILU, G16, gu_wave_strips(BITS, G16 ? 16 : 32), true, true, true, WD>(a, pg, sc, fo, fg, r, 0, smem);
        if (tl && threadIdx.x == 0) tl[2] = __builtin_amdgcn_s_memrealtime();
        return;
    }
    r -= ng;
    if (int(threadIdx.x) >= 64 * pd.rg * pd.kw) return;
    MMArgs a = da;
    a.W = P.down;
    a.tlw = tl;
    a.onorm = P.next_norm;
    Flow fout;  // the next layer's q|k|v; after the last layer the head reads x in a later launch
    if (!last) {
        fout.ctl = lf.ctl;
        fout.producers = fout.per = pd.nrb;
        fout.base = base + FL_D;  // back to zero in the next layer's first o workgroup
        fout.mirrors = lf.m_d;
    }
    fg.stamp = tl ? tl + 1 : nullptr;
    mm_body<BITS, EPI_RESID, G16, DS, true, true, true, WD>(a, pd, sc, fg, fout, r, 0, smem);
    if (tl && threadIdx.x == 0) tl[2] = __builtin_amdgcn_s_memrealtime();
}

// The head's last workgroup to finish: partials were stored at agent scope and waited on before
// the count moved, so the last one reads them all (agent-scope loads, past its own L2) and does
// what k_head_final does for a verify block: per token the best partial (src/spec.rs:41-49; a
// NaN logit of row 0 makes the argmax 0), then greedy acceptance (src/spec.rs:119-127). The
// result also goes straight to pinned host memory, which saves the copy back.
template <int WAVES>
__device__ __forceinline__ void head_final_last(const MMArgs& a, int* lds) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const int total = int(gridDim.x * gridDim.y);
        const int old = __hip_atomic_fetch_add(a.fin_cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = old == total - 1;
        if (last) __hip_atomic_store(a.fin_cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        lds[0] = last;
    }
    __syncthreads();
    if (!lds[0]) return;
    uint32_t* am = reinterpret_cast<uint32_t*>(lds + 1);  // [a.n]
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nb = int(gridDim.x);
    for (int i = w; i < a.n; i += WAVES) {
        const size_t base = size_t(i / FTOK) * a.arg_stride * FTOK + i % FTOK;
        float v = NAN;
        int ix = 0x7fffffff;
        // Four partials per lane in flight at once (one workgroup per CU: 256 blocks in one round).
        for (int b0 = lane; b0 < nb; b0 += 4 * 64) {
            float xv[4];
            int xi[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int b = b0 + 64 * u;
                const size_t at = base + size_t(b < nb ? b : 0) * FTOK;
                xv[u] = __hip_atomic_load(a.arg_val + at, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                xi[u] = __hip_atomic_load(a.arg_idx + at, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (b0 + 64 * u < nb && beats(xv[u], xi[u], v, ix)) {
                    v = xv[u];
                    ix = xi[u];
                }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(v, o, 64);
            const int oi = __shfl_xor(ix, o, 64);
            if (beats(ov, oi, v, ix)) {
                v = ov;
                ix = oi;
            }
        }
        if (lane == 0) {
            const float r0 = __hip_atomic_load(a.row0 + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            am[i] = isnan(r0) ? 0u : uint32_t(ix);
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < a.n; i += blockDim.x) a.fin_amax[i] = am[i];
    if (threadIdx.x == 0) {
        int m = 0;
        while (m < a.n - 1 && am[m] == a.fin_block[m + 1]) m++;
        const uint32_t next = am[m];
        const int err = __hip_atomic_load(a.fin_ctl + FLOW_ERR, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        a.fin_ctl[FLOW_ACC] = m;
        a.fin_ctl[FLOW_ACC + 1] = int(next);
        __hip_atomic_store(a.fin_host + FLOW_ERR, uint32_t(err), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(a.fin_host + FLOW_ACC, uint32_t(m), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(a.fin_host + FLOW_ACC + 1, next, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        // Complete before the wave ends (no fence: one would write back this XCD's whole L2).
        __builtin_amdgcn_s_waitcnt(0);
    }
}

// Output head, persistent: each workgroup copies the tile's fragments (every k-step) to LDS
// once; its wavefronts then stream 64-row groups of the table over the whole K range, PF chunks
// ahead, and reduce each group to logits and a per-token (value, index) argmax partial inside
// the wavefront (lane l holds rows 16 r + 4 (l / 16) + i of token l % 16).
// Chunks in flight per wavefront (int4 chunks carry four k-steps of fragments each).
template <int BITS, bool G16>
constexpr int head_pf() { return BITS == 4 ? (G16 ? 1 : 2) : 3; }
// Wavefronts per workgroup: 10 give 2560 on 256 CUs, so a 151936-row table (2374 groups of 64)
// takes at most one group per wavefront; the groups-of-16 variants keep 8 for registers. A launch
// over several token tiles (MT) runs 12 (198 workgroups, one group per wavefront): measured on the
// 0.5B table over 9 tiles, 231 us against 279 us with 10 (one tile: 36-37 us either way).
template <bool G16, bool MT = false>
constexpr int head_waves() { return G16 ? 8 : (MT ? 12 : 10); }
constexpr int HEAD_WAVES_MAX = 12;
constexpr int HEAD_BMAX = 16;  // fragment slots (16 B) copied to LDS per thread
constexpr int HEAD_FIN_MAX = 128;  // tokens of a head launch that does its own final reduction

// CMP (one token tile of nt tokens): LDS holds only the live tokens' fragment slots, [k-step][term]
// [column group][nt], for tables whose full fragments (16 token columns) exceed the LDS; the slots
// are copied through registers, a few per thread at a time.
template <int BITS, bool G16, bool CMP = false, bool MT = false>
__global__ __launch_bounds__((64 * head_waves<G16, MT>())) void k_head(MMArgs a, int n_groups) {
    constexpr int HEAD_WAVES = head_waves<G16, MT>();
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int Q = Steps<BITS>::Q, HEAD_PF = head_pf<BITS, G16>();
    const TMat& W = a.W;
    int bx = blockIdx.x, tile = blockIdx.y;
    if (gridDim.y > 1) xcd_tile_map(bx, tile);  // a block's tiles side by side on one XCD
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nt = min(FTOK, a.n - tile * FTOK), ibase = tile * FTOK;
    const int nks = W.n_chunks * Q;
    uint4* bl = reinterpret_cast<uint4*>(smem);
    const int row_slots = CMP ? 4 * nt : 64;  // LDS slots per (k-step, term)
    float* inv = reinterpret_cast<float*>(smem + size_t(nks) * 3 * row_slots * 16);

    // This wavefront's groups: g = first + k * stride. Its first weight chunks go out at once.
    const int stride = gridDim.x * HEAD_WAVES, first = bx * HEAD_WAVES + wv;
    const int my_groups = first < n_groups ? (n_groups - first + stride - 1) / stride : 0;
    const int NC = W.n_chunks, F = my_groups * NC;
    const size_t sst = size_t(NC) * 1024;
    auto wbase = [&](int f) { return W.data + (size_t(4 * (first + (f / NC) * stride)) * NC * 64 + lane) * 16; };
    // The tile's fragments (at most HEAD_BMAX slots per thread) go straight to LDS, requested
    // before the weight chunks; staged through registers they would spill. The wait for them
    // also covers the first HEAD_PF chunks, which the first MFMAs need anyway.
    const uint4* fb = reinterpret_cast<const uint4*>(a.frags + size_t(tile) * a.frag_stride);
    const int nb = nks * 3 * 64, nthr = 64 * HEAD_WAVES;
    uint4 raw[HEAD_PF][4];
    if constexpr (!CMP) {
        // A wavefront moves 64 slots of 16 bytes per load.
        for (int u = 0; u < HEAD_BMAX; u++) {
            const int w0 = wv * 64 + u * nthr;  // this wavefront's first slot; nb is a multiple of 64
            if (w0 >= nb) break;
            __builtin_amdgcn_global_load_lds(fb + w0 + lane, (__attribute__((address_space(3))) void*)(bl + w0), 16, 0, 0);
        }
#pragma unroll
        for (int p = 0; p < HEAD_PF; p++)
            if (p < F) load_chunk<4>(wbase(p), sst, p % NC, raw[p]);
    } else {
        // The first weight chunks go out first; then the live slots, four loads per thread in
        // flight: LDS slot e = (row * 4 + group) * nt + token holds fragment slot row * 64 +
        // 16 group + token.
#pragma unroll
        for (int p = 0; p < HEAD_PF; p++)
            if (p < F) load_chunk<4>(wbase(p), sst, p % NC, raw[p]);
        const int tot = nks * 3 * 4 * nt;
        for (int e0 = threadIdx.x; e0 < tot; e0 += 4 * nthr) {
            uint4 v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int e = e0 + u * nthr, row = e / (4 * nt), rem = e % (4 * nt);
                if (e < tot) v[u] = fb[row * 64 + 16 * (rem / nt) + rem % nt];
            }
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (e0 + u * nthr < tot) bl[e0 + u * nthr] = v[u];
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    if (wv == 0) {
        if (a.ss) inv_rms(a, tile, W.cols, inv);
        else if (lane < FTOK) inv[lane] = 1.0f;
    }
    __syncthreads();

    f32x4 total[4], acc[4];
#pragma unroll
    for (int r = 0; r < 4; r++) total[r] = acc[r] = f32x4{0, 0, 0, 0};
    float wbv = NAN;  // this wavefront's best (value, row) for token lane % 16 so far
    int wbi = 0x7fffffff;
    for (int f0 = 0; f0 < F; f0 += HEAD_PF) {
#pragma unroll
        for (int p = 0; p < HEAD_PF; p++) {
            const int f = f0 + p;
            if (f >= F) break;
            const int c = f % NC;
            const int g = first + (f / NC) * stride;
            uint4 B[Q][3];
#pragma unroll
            for (int q = 0; q < Q; q++)
#pragma unroll
                for (int t = 0; t < 3; t++) {
                    if constexpr (CMP)
                        B[q][t] = (lane & 15) < nt ? bl[(((c * Q + q) * 3 + t) * 4 + (lane >> 4)) * nt + (lane & 15)] : make_uint4(0, 0, 0, 0);
                    else
                        B[q][t] = bl[((c * Q + q) * 3 + t) * 64 + lane];
                }
            chunk_mfma<BITS, G16, 4>(W, 4 * g, c, 0, nks, B, raw[p], acc, total);
            if (f + HEAD_PF < F) load_chunk<4>(wbase(f + HEAD_PF), sst, (f + HEAD_PF) % NC, raw[p]);
            if (c == NC - 1) {
                // Group done: logits, optional store, argmax over its 64 rows per token.
                const int tok = lane & 15;
                const float iv = inv[tok];
                float bvv = NAN;
                int bix = 0x7fffffff;
#pragma unroll
                for (int r = 0; r < 4; r++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int row = 64 * g + 16 * r + 4 * (lane >> 4) + i;
                        const float v = __fmul_rn(total[r][i], iv);
                        if (row < W.rows) {
                            if (a.out && tok < nt) a.out[size_t(ibase + tok) * a.ldo + a.row_base + row] = v;
                            if (beats(v, a.row_base + row, bvv, bix)) {
                                bvv = v;
                                bix = a.row_base + row;
                            }
                        }
                        if (row == 0 && a.row0) {
                            if (a.fin_cnt) __hip_atomic_store(a.row0 + ibase + tok, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            else a.row0[ibase + tok] = v;
                        }
                    }
#pragma unroll
                for (int o = 16; o < 64; o <<= 1) {
                    const float ov = __shfl_xor(bvv, o, 64);
                    const int oi = __shfl_xor(bix, o, 64);
                    if (beats(ov, oi, bvv, bix)) {
                        bvv = ov;
                        bix = oi;
                    }
                }
                if (beats(bvv, bix, wbv, wbi)) {
                    wbv = bvv;
                    wbi = bix;
                }
#pragma unroll
                for (int r = 0; r < 4; r++) total[r] = f32x4{0, 0, 0, 0};
            }
        }
    }
    // One partial per workgroup: the best of its wavefronts, per token.
    float* wv_v = reinterpret_cast<float*>(inv + FTOK);
    int* wv_i = reinterpret_cast<int*>(wv_v + HEAD_WAVES * FTOK);
    if (lane < FTOK) {
        wv_v[wv * FTOK + lane] = wbv;
        wv_i[wv * FTOK + lane] = wbi;
    }
    __syncthreads();
    if (threadIdx.x < FTOK) {
        const int tok = threadIdx.x;
        float v = wv_v[tok];
        int ix = wv_i[tok];
        for (int w = 1; w < HEAD_WAVES; w++)
            if (beats(wv_v[w * FTOK + tok], wv_i[w * FTOK + tok], v, ix)) {
                v = wv_v[w * FTOK + tok];
                ix = wv_i[w * FTOK + tok];
            }
        const size_t at = (size_t(tile) * a.arg_stride + a.arg_off + bx) * FTOK + tok;
        if (a.fin_cnt) {
            __hip_atomic_store(a.arg_val + at, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(a.arg_idx + at, ix, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            a.arg_val[at] = v;
            a.arg_idx[at] = ix;
        }
    }
    if (a.fin_cnt) head_final_last<HEAD_WAVES>(a, reinterpret_cast<int*>(wv_i + HEAD_WAVES * FTOK));
}

int device_cu_count() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        FCHECK(hipGetDevice(&dev));
        FCHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    }
    return cus;
}

constexpr size_t HEAD_LDS_MAX = 150 * 1024;

MMPlan mm_plan(const TMat& W, int rg, int kw, int n_tokens, int strips, int wide) {
    MMPlan p;
    if (strips != 1 && strips != 2 && strips != 4) throw std::runtime_error("1, 2 or 4 strips per wavefront");
    if (wide != 1 && wide != 2) throw std::runtime_error("a wavefront's share of K is 128 or 256 columns");
    if (wide == 2 && W.bits != 16 && W.group == 16) throw std::runtime_error("256-column shares need groups of 32 or more");
    p.s = strips;
    p.rg = rg;
    p.kw = kw < 1 ? 1 : kw;
    p.wide = wide;
    // 256-column shares double the registers that hold weights and fragments: 8 wavefronts at most.
    const int max_waves = wide > 1 ? 8 : mm_max_waves(W.bits, W.group, strips);
    const int cpw = wide * 4 / (W.bits == 16 ? 1 : (W.bits == 8 ? 2 : 4));
    const int waves_k = (W.n_chunks + cpw - 1) / cpw;  // wavefront shares along K
    if (p.kw > waves_k) p.kw = waves_k;
    if (p.rg > max_waves) throw std::runtime_error("too many row groups for one workgroup");
    if (p.rg * p.kw > max_waves) p.kw = max_waves / p.rg;
    if (p.kw > MAX_KW) throw std::runtime_error("more wavefronts along K than the row-group reduction adds");
    p.nsplit = (waves_k + p.kw - 1) / p.kw;
    while (p.nsplit > MAX_SPLIT && p.rg * (p.kw + 1) <= max_waves) {
        p.kw++;
        p.nsplit = (waves_k + p.kw - 1) / p.kw;
    }
    if (p.nsplit > MAX_SPLIT) throw std::runtime_error("matrix too wide for the split-K limit");
    if (W.n_strips % (strips * rg)) throw std::runtime_error("matrix rows do not fill whole row blocks");
    p.nrb = W.n_strips / (strips * rg);
    p.tiles = (n_tokens + FTOK - 1) / FTOK;
    return p;
}

MMPlan gu_plan(const TMat& W, int kw, int n_tokens, int wide) {
    const int gs = gu_wave_strips(W.bits, W.group);
    return mm_plan(W, 2 * GU_STRIPS / gs, kw, n_tokens, gs, wide);
}

size_t mm_part_floats(const MMPlan& p) {
    return p.nsplit > 1 ? size_t(p.tiles) * p.nrb * p.nsplit * 16 * p.s * p.rg * FTOK : 0;
}
size_t mm_counters(const MMPlan& p) { return p.nsplit > 1 ? size_t(p.tiles) * p.nrb : 0; }

// LDS of a matrix workgroup (the layout at the top of mm_body); hd: head_dim of a q|k|v matrix
// (its RoPE tables), 0 for the others.
static size_t lds_bytes(const MMPlan& p, int hd = 0) {
    const size_t red = p.kw > 1 ? size_t(p.rg) * p.kw * p.s * 64 * 16 : 0;
    const size_t rows = size_t(16 * p.s * p.rg);
    return red + rows * FTOK * 4 + FTOK * 4 + 16 + FTOK * 16 * 8 + (rows * FTOK + rows + 2 * FTOK * size_t(hd / 2) + 2 * FTOK) * 4;
}

static thread_local hipEvent_t t_start = nullptr, t_stop = nullptr;

void mm_time_next_launch(hipEvent_t start, hipEvent_t stop) {
    t_start = start;
    t_stop = stop;
}

// hipLaunchKernelGGL, or the timed launch when events are pending.
template <class K, class... Args>
static void go(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t s, Args... args) {
    if (t_start) {
        hipExtLaunchKernelGGL(kernel, grid, block, uint32_t(lds), s, t_start, t_stop, 0u, args...);
        t_start = t_stop = nullptr;
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, s, args...);
    }
}

template <int EPI, int S>
static void launch(const MMArgs& a, const MMPlan& p, const MMScratch& sc, hipStream_t s) {
    if (p.s != S) throw std::runtime_error("matrix plan does not match the kernel's strips per wavefront");
    if (p.nsplit > 1 && (!sc.part || !sc.cnt)) throw std::runtime_error("split matrix launch without scratch");
    const dim3 grid(p.nrb * p.nsplit, p.tiles), block(64 * p.rg * p.kw);
    const size_t lds = lds_bytes(p, EPI == EPI_QKV ? a.hd : 0);
    const bool g16 = a.W.bits != 16 && a.W.group == 16;
    if (p.wide != 1) {
        if (p.wide != 2 || g16) throw std::runtime_error("256-column shares need groups of 32 or more");
        switch (a.W.bits) {
            case 16: go(k_mm<16, EPI, false, S, 2>, grid, block, lds, s, a, p, sc); break;
            case 8: go(k_mm<8, EPI, false, S, 2>, grid, block, lds, s, a, p, sc); break;
            default: go(k_mm<4, EPI, false, S, 2>, grid, block, lds, s, a, p, sc); break;
        }
        FCHECK(hipGetLastError());
        return;
    }
    switch (a.W.bits) {
        case 16: go(k_mm<16, EPI, false, S>, grid, block, lds, s, a, p, sc); break;
        case 8:
            if (g16) go(k_mm<8, EPI, true, S>, grid, block, lds, s, a, p, sc);
            else go(k_mm<8, EPI, false, S>, grid, block, lds, s, a, p, sc);
            break;
        default:
            if (g16) go(k_mm<4, EPI, true, S>, grid, block, lds, s, a, p, sc);
            else go(k_mm<4, EPI, false, S>, grid, block, lds, s, a, p, sc);
            break;
    }
    FCHECK(hipGetLastError());
}

void mm_qkv(const MMArgs& a, const MMPlan& p, const MMScratch& sc, hipStream_t s) {
    if (a.hd % 2 || a.hd / 2 > ROPE_HALF_MAX) throw std::runtime_error("head_dim must be even and at most 256");
    if ((a.heads + a.kv_heads) * a.hd % 16) throw std::runtime_error("q|k rows must fill whole strips");
    if (p.s == 4) launch<EPI_QKV, 4>(a, p, sc, s);  // 64-row blocks (the epilogue is per row)
    else launch<EPI_QKV, 1>(a, p, sc, s);
}
void mm_residual(const MMArgs& a, const MMPlan& p, const MMScratch& sc, hipStream_t s) {
    switch (p.s) {
        case 1: launch<EPI_RESID, 1>(a, p, sc, s); break;
        case 2: launch<EPI_RESID, 2>(a, p, sc, s); break;
        default: launch<EPI_RESID, 4>(a, p, sc, s); break;
    }
}
void mm_gate_up(const MMArgs& a, const MMPlan& p, const MMScratch& sc, hipStream_t s) {
    const int gs = gu_wave_strips(a.W.bits, a.W.group);
    if (p.s != gs || p.s * p.rg != 2 * GU_STRIPS) throw std::runtime_error("gate|up plan does not hold a gate block and its up block");
    if (gs == 2 * GU_STRIPS) launch<EPI_SILU, 2 * GU_STRIPS>(a, p, sc, s);
    else launch<EPI_SILU, GU_STRIPS>(a, p, sc, s);
}

// k-steps per scale group when every group lies inside one chunk (the pipelined launches' case).
static bool pipe_group_steps(const TMat& W, int& gk) {
    if (W.bits == 16) {
        gk = 1;
        return true;
    }
    const int q = W.bits == 8 ? 2 : 4;
    if (W.group < 32 || W.group % 32) return false;
    gk = W.group / 32;
    return q % gk == 0;
}

bool mm_gate_up_pipe_fits(const MMArgs& a, const MMPlan& p) {
    int gk = 0;
    // 8 wavefronts of 2 shares each, one tile, no K split; byte offsets (past-the-end items
    // included) below 2^31.
    if (p.wide != 1 || p.tiles != 1 || p.rg != 1 || p.kw != PIPE_WAVES * PIPE_SPW || p.nsplit != 1 || p.s != 2 * GU_STRIPS) return false;
    if (!pipe_group_steps(a.W, gk)) return false;
    return tile_data_bytes(a.W) <= PIPE_MAX_BYTES && tile_scale_bytes(a.W) <= PIPE_MAX_BYTES;
}

void mm_gate_up_pipe(const MMArgs& a, const MMPlan& p, hipStream_t s) {
    int gk = 0;
    if (!mm_gate_up_pipe_fits(a, p) || !pipe_group_steps(a.W, gk)) throw std::runtime_error("gate|up plan does not fit the pipelined launch");
    const int items = p.nrb * GU_STRIPS, wgs = std::min(items, device_cu_count());
    const int most = (items + wgs - 1) / wgs;
    const size_t lds = pipe_lds_bytes(p.kw, most);
    if (lds > 160 * 1024) throw std::runtime_error("gate|up too large for the pipelined launch");
    const dim3 grid(wgs), block(64 * PIPE_WAVES);
    switch (a.W.bits) {
        case 16: go(k_gu_pipe<16, 1>, grid, block, lds, s, a, p, most); break;
        case 8:
            if (gk == 1) go(k_gu_pipe<8, 1>, grid, block, lds, s, a, p, most);
            else go(k_gu_pipe<8, 2>, grid, block, lds, s, a, p, most);
            break;
        default:
            if (gk == 1) go(k_gu_pipe<4, 1>, grid, block, lds, s, a, p, most);
            else if (gk == 2) go(k_gu_pipe<4, 2>, grid, block, lds, s, a, p, most);
            else go(k_gu_pipe<4, 4>, grid, block, lds, s, a, p, most);
            break;
    }
    FCHECK(hipGetLastError());
}

void mm_gate_up_down(const MMArgs& gu, const MMPlan& pgu, const MMArgs& dn, const MMPlan& pdn, const MMScratch& sc,
                     int* ctl, hipStream_t s) {
    if (pgu.s != gu_wave_strips(gu.W.bits, gu.W.group) || pgu.s * pgu.rg != 2 * GU_STRIPS || pdn.s != DOWN_STRIPS)
        throw std::runtime_error("gate|up/down plans do not match");
    if (pgu.tiles != 1 || pdn.tiles != 1) throw std::runtime_error("the fused gate|up/down launch takes one token tile");
    if (pgu.nsplit != 1) throw std::runtime_error("the fused gate|up/down launch needs gate|up without a K split");
    if (pgu.wide != 1 || pdn.wide != 1) throw std::runtime_error("the fused gate|up/down launch takes 128-column K shares");
    if (pdn.nsplit > 1 && (!sc.part || !sc.cnt)) throw std::runtime_error("split matrix launch without scratch");
    // A down K split covers 128 kw columns (4 k-steps of 32 per wavefront); a gate|up row block
    // produces 16 GU_STRIPS of them.
    const int split_cols = 128 * pdn.kw, act_cols = 16 * GU_STRIPS;
    Flow fl;
    fl.ctl = ctl;
    fl.producers = pgu.nrb;
    fl.per = split_cols / act_cols;
    fl.consumers = pdn.nrb;
    fl.mirrors = std::min(FLOW_GU_MIRRORS, pdn.nrb);
    if (split_cols % act_cols || (fl.producers + fl.per - 1) / fl.per != pdn.nsplit || pdn.nsplit * fl.mirrors > FLOW_ATTN_O)
        throw std::runtime_error("gate|up row blocks do not map onto the down K splits");
    const int n = pgu.nrb * pgu.nsplit + pdn.nrb * pdn.nsplit;
    const size_t lds = std::max(lds_bytes(pgu), lds_bytes(pdn));
    const dim3 grid(n), block(64 * std::max(pgu.rg * pgu.kw, pdn.rg * pdn.kw));
    const bool g16 = gu.W.bits != 16 && gu.W.group == 16;
    switch (gu.W.bits) {
        case 16: go(k_gu_down<16, false>, grid, block, lds, s, gu, pgu, dn, pdn, sc, fl); break;
        case 8:
            if (g16) go(k_gu_down<8, true>, grid, block, lds, s, gu, pgu, dn, pdn, sc, fl);
            else go(k_gu_down<8, false>, grid, block, lds, s, gu, pgu, dn, pdn, sc, fl);
            break;
        default:
            if (g16) go(k_gu_down<4, true>, grid, block, lds, s, gu, pgu, dn, pdn, sc, fl);
            else go(k_gu_down<4, false>, grid, block, lds, s, gu, pgu, dn, pdn, sc, fl);
            break;
    }
    FCHECK(hipGetLastError());
}

int attention_o_workgroups(int heads, const MMPlan& po) { return ASPLIT * heads + po.nrb * po.nsplit; }

template <int HD>
static void launch_attn_o(const AttnArgs& aa, const MMArgs& o, const MMPlan& po, const MMScratch& sc, const Flow& fl, hipStream_t s) {
    const dim3 grid(attention_o_workgroups(aa.heads, po)), block(std::max(AWV * 64, 64 * po.rg * po.kw));
    const size_t lds = std::max(lds_bytes(po), attn_lds_bytes<HD>());
    const bool g16 = o.W.bits != 16 && o.W.group == 16;
    switch (o.W.bits) {
        case 16: go(k_attn_o<HD, 16, false>, grid, block, lds, s, aa, o, po, sc, fl); break;
        case 8:
            if (g16) go(k_attn_o<HD, 8, true>, grid, block, lds, s, aa, o, po, sc, fl);
            else go(k_attn_o<HD, 8, false>, grid, block, lds, s, aa, o, po, sc, fl);
            break;
        default:
            if (g16) go(k_attn_o<HD, 4, true>, grid, block, lds, s, aa, o, po, sc, fl);
            else go(k_attn_o<HD, 4, false>, grid, block, lds, s, aa, o, po, sc, fl);
            break;
    }
    FCHECK(hipGetLastError());
}

void attention_o(const float* q, int ldq, int t, int heads, int kv_heads, int hd, const int* pos0, const float* kc, const float* vc,
                 float* scratch, int* cnt, uint8_t* frags, const MMArgs& o, const MMPlan& po, const MMScratch& sc, int* ctl,
                 hipStream_t s) {
    if (t > FTOK || po.tiles != 1) throw std::runtime_error("the fused attention/o launch takes one token tile");
    if (po.s != 1 || po.nsplit != 1) throw std::runtime_error("the fused attention/o launch needs o without a K split");
    if (po.wide != 1) throw std::runtime_error("the fused attention/o launch takes 128-column K shares");
    if (64 * po.rg * po.kw > 512) throw std::runtime_error("o workgroups too large for the fused attention/o launch");
    const AttnArgs aa = make_attn_args(q, ldq, t, heads, kv_heads, hd, pos0, AttnRows{}, kc, vc, scratch, cnt, frags);
    Flow fl;
    fl.ctl = ctl;
    fl.producers = heads;
    fl.per = heads;
    fl.consumers = po.nrb * po.nsplit;
    fl.base = FLOW_ATTN_O;
    fl.mirrors = std::min(FLOW_AO_MIRRORS, fl.consumers);
    switch (hd) {
        case 16: launch_attn_o<16>(aa, o, po, sc, fl, s); break;
        case 32: launch_attn_o<32>(aa, o, po, sc, fl, s); break;
        case 64: launch_attn_o<64>(aa, o, po, sc, fl, s); break;
        case 128: launch_attn_o<128>(aa, o, po, sc, fl, s); break;
        default: throw std::runtime_error("head_dim must be 16, 32, 64 or 128");
    }
}

int qkv_attention_o_workgroups(int heads, const MMPlan& pq, const MMPlan& po) {
    return pq.nrb * pq.nsplit + ASPLIT * heads + po.nrb * po.nsplit;
}

template <int HD>
static void launch_qkv_attn_o(const MMArgs& qa, const MMPlan& pq, const AttnArgs& aa, const MMArgs& o, const MMPlan& po, const MMScratch& sc,
                              const Flow& fq, const Flow& fo, hipStream_t s) {
    const dim3 grid(qkv_attention_o_workgroups(aa.heads, pq, po)), block(std::max({AWV * 64, 64 * po.rg * po.kw, 64 * pq.rg * pq.kw}));
    const size_t lds = std::max({lds_bytes(pq, qa.hd), lds_bytes(po), attn_lds_bytes<HD>()});
    const bool g16 = o.W.bits != 16 && o.W.group == 16;
    switch (o.W.bits) {
        case 16: go(k_qkv_attn_o<HD, 16, false>, grid, block, lds, s, qa, pq, aa, o, po, sc, fq, fo); break;
        case 8:
            if (g16) go(k_qkv_attn_o<HD, 8, true>, grid, block, lds, s, qa, pq, aa, o, po, sc, fq, fo);
            else go(k_qkv_attn_o<HD, 8, false>, grid, block, lds, s, qa, pq, aa, o, po, sc, fq, fo);
            break;
        default:
            if (g16) go(k_qkv_attn_o<HD, 4, true>, grid, block, lds, s, qa, pq, aa, o, po, sc, fq, fo);
            else go(k_qkv_attn_o<HD, 4, false>, grid, block, lds, s, qa, pq, aa, o, po, sc, fq, fo);
            break;
    }
    FCHECK(hipGetLastError());
}

void qkv_attention_o(const MMArgs& qa, const MMPlan& pq, float* scratch, int* cnt, uint8_t* frags, const MMArgs& o, const MMPlan& po,
                     const MMScratch& sc, int* ctl, hipStream_t s) {
    const int heads = qa.heads, kvh = qa.kv_heads, hd = qa.hd, t = qa.n;
    if (t < 1 || t > FTOK || pq.tiles != 1 || po.tiles != 1) throw std::runtime_error("the fused q|k|v/attention/o launch takes one token tile");
    if (pq.s != 1 || pq.rg != 1 || pq.nsplit != 1) throw std::runtime_error("the fused launch needs q|k|v as one workgroup per strip");
    if (po.s != 1 || po.nsplit != 1) throw std::runtime_error("the fused launch needs o without a K split");
    if (pq.wide != 1 || po.wide != 1) throw std::runtime_error("the fused launch takes 128-column K shares");
    if (64 * po.rg * po.kw > 512 || 64 * pq.kw > 512) throw std::runtime_error("workgroups too large for the fused launch");
    if (heads > FLOW_ATTN_O || hd % 16 || heads % kvh) throw std::runtime_error("heads do not fit the fused launch's counters");
    if (hd / 2 > ROPE_HALF_MAX || (heads + kvh) * hd % 16) throw std::runtime_error("head_dim must be even and at most 256");
    const AttnArgs aa = make_attn_args(qa.out, qa.ldo, t, heads, kvh, hd, qa.pos0, AttnRows{}, qa.kcache, qa.vcache, scratch, cnt, frags);
    // q|k|v -> attention: counter h (h < heads) counts the q strips of head h and the k and v
    // strips of its group.
    Flow fq;
    fq.ctl = ctl;
    fq.producers = pq.nrb;
    fq.want = 3 * (hd / 16);
    fq.consumers = ASPLIT;
    fq.base = 0;
    Flow fo;
    fo.ctl = ctl;
    fo.producers = heads;
    fo.per = heads;
    fo.consumers = po.nrb * po.nsplit;
    fo.base = FLOW_ATTN_O;
    fo.mirrors = std::min(FLOW_AO_MIRRORS, fo.consumers);
    switch (hd) {
        case 16: launch_qkv_attn_o<16>(qa, pq, aa, o, po, sc, fq, fo, s); break;
        case 32: launch_qkv_attn_o<32>(qa, pq, aa, o, po, sc, fq, fo, s); break;
        case 64: launch_qkv_attn_o<64>(qa, pq, aa, o, po, sc, fq, fo, s); break;
        case 128: launch_qkv_attn_o<128>(qa, pq, aa, o, po, sc, fq, fo, s); break;
        default: throw std::runtime_error("head_dim must be 16, 32, 64 or 128");
    }
}

int layer_stack_workgroups(int heads, const MMPlan& pq, const MMPlan& po, const MMPlan& pg, const MMPlan& pd) {
    return pq.nrb + ASPLIT * heads + po.nrb + pg.nrb + pd.nrb * pd.nsplit;
}

const char* layer_stack_unfit(int t, int heads, int kv_heads, int hd, const MMPlan& pq, const MMPlan& po, const MMPlan& pg,
                              const MMPlan& pd) {
    if (t < 1 || t > FTOK || pq.tiles != 1 || po.tiles != 1 || pg.tiles != 1 || pd.tiles != 1) return "the layer stack takes one token tile";
    // Strips per wavefront: 1 (q|k|v), 1 (o), DOWN_STRIPS (down) with 128-column K shares; 1, 1, 4
    // with 256-column shares.
    const int want_qs = 1, want_ds = pq.wide == 2 ? 4 : DOWN_STRIPS;
    if (pq.s != want_qs || pq.rg != 1 || pq.nsplit != 1) return "the layer stack needs q|k|v as one row group per workgroup, without a K split";
    if ((hd / 16) % pq.s) return "q|k|v row blocks must not straddle heads";
    if (po.s != want_qs || po.nsplit != 1) return "the layer stack needs o without a K split";
    if (pg.nsplit != 1 || pg.s * pg.rg != 2 * GU_STRIPS) return "the layer stack needs gate|up row blocks without a K split";
    if (pd.s != want_ds) return "the layer stack needs the down plan's strips per wavefront";
    if (pd.nsplit * FLOW_GU_MIRRORS > FLOW_LAYER_STRIDE - FL_G) return "too many down K splits for the layer counters";
    if (pq.wide != pd.wide || po.wide != pd.wide || pg.wide != pd.wide) return "the layer's plans differ in their K shares";
    if (pd.wide != 1 && hd != 128) return "256-column K shares run in the layer stack for head_dim 128 only";
    const int split_cols = 128 * pd.wide * pd.kw, act_cols = 16 * GU_STRIPS;
    if (split_cols % act_cols || (pg.nrb + split_cols / act_cols - 1) / (split_cols / act_cols) != pd.nsplit)
        return "gate|up row blocks do not map onto the down K splits";
    if (std::max({64 * pq.kw, AWV * 64, 64 * po.rg * po.kw, 64 * pg.rg * pg.kw, 64 * pd.rg * pd.kw}) > 512)
        return "workgroups too large for the layer stack";
    if (po.s > po.kw || pd.s > pd.kw) return "residual rows do not fit the per-thread registers";
    if (heads > FL_A - FL_Q || hd % 16 || heads % kv_heads) return "heads do not fit the layer counters";
    if (hd != 16 && hd != 32 && hd != 64 && hd != 128) return "head_dim must be 16, 32, 64 or 128";
    if (hd / 2 > ROPE_HALF_MAX || (heads + kv_heads) * hd % 16) return "head_dim must be even and at most 256";
    return nullptr;
}

template <int HD>
static void launch_layers(const LayerPtrs* lp, int layers, size_t seq_off, const MMArgs& qa, const MMPlan& pq, const AttnArgs& aa,
                          const MMArgs& oa, const MMPlan& po, const MMArgs& ga, const MMPlan& pg, const MMArgs& da, const MMPlan& pd,
                          const MMScratch& sc, const LayerFlows& lf, hipStream_t s) {
    const dim3 grid(layers * layer_stack_workgroups(aa.heads, pq, po, pg, pd)), block(512);
    // One workgroup per CU (the launch asks for more than half its LDS): a pass is bound by
    // handoff latency, and twice the resident workgroups poll twice as much (0.5B int8: 0.89 ms
    // per step at one, 0.97 at two; int4: 1.01 and 1.18).
    const size_t lds = std::max({lds_bytes(pq, qa.hd), lds_bytes(po), lds_bytes(pg), lds_bytes(pd), attn_lds_bytes<HD>(),
                                 size_t(96) << 10});
    const bool g16 = qa.W.bits != 16 && qa.W.group == 16;
    if constexpr (HD == 128) {
        if (pq.wide == 2) {
            if (g16) throw std::runtime_error("256-column shares need groups of 32 or more");
            if (lf.tl) {
                if (qa.W.bits != 8 || HD != 128) throw std::runtime_error("the layer-stack timeline is built for int8 weights");
                go(k_layers<HD, 8, false, 2, 1, 1, 4, true>, grid, block, lds, s, lp, seq_off, qa, pq, aa, oa, po, ga, pg, da, pd, sc, lf);
                FCHECK(hipGetLastError());
                return;
            }
            switch (qa.W.bits) {
                case 16: go(k_layers<HD, 16, false, 2, 1, 1, 4>, grid, block, lds, s, lp, seq_off, qa, pq, aa, oa, po, ga, pg, da, pd, sc, lf); break;
                case 8: go(k_layers<HD, 8, false, 2, 1, 1, 4>, grid, block, lds, s, lp, seq_off, qa, pq, aa, oa, po, ga, pg, da, pd, sc, lf); break;
                default: go(k_layers<HD, 4, false, 2, 1, 1, 4>, grid, block, lds, s, lp, seq_off, qa, pq, aa, oa, po, ga, pg, da, pd, sc, lf); break;
            }
            FCHECK(hipGetLastError());
            return;
        }
    }
    if (pq.wide != 1) throw std::runtime_error("256-column K shares run in the layer stack for head_dim 128 only");
    if (lf.tl) {
        if constexpr (HD == 64) {
            if (qa.W.bits != 8 || g16) throw std::runtime_error("the layer-stack timeline is built for int8 weights in groups of 32 or more");
            go(k_layers<HD, 8, false, 1, 1, 1, DOWN_STRIPS, true>, grid, block, lds, s, lp, seq_off, qa, pq, aa, oa, po, ga, pg, da, pd, sc, lf);
            FCHECK(hipGetLastError());
            return;
        }
        throw std::runtime_error("the layer-stack timeline is built for head_dim 64 and 128");
    }
    switch (qa.W.bits) {
        case 16: go(k_layers<HD, 16, false>, grid, block, lds, s, lp, seq_off, qa, pq, aa, oa, po, ga, pg, da, pd, sc, lf); break;
        case 8:
            if (g16) go(k_layers<HD, 8, true>, grid, block, lds, s, lp, seq_off, qa, pq, aa, oa, po, ga, pg, da, pd, sc, lf);
            else go(k_layers<HD, 8, false>, grid, block, lds, s, lp, seq_off, qa, pq, aa, oa, po, ga, pg, da, pd, sc, lf);
            break;
        default:
            if (g16) go(k_layers<HD, 4, true>, grid, block, lds, s, lp, seq_off, qa, pq, aa, oa, po, ga, pg, da, pd, sc, lf);
            else go(k_layers<HD, 4, false>, grid, block, lds, s, lp, seq_off, qa, pq, aa, oa, po, ga, pg, da, pd, sc, lf);
            break;
    }
    FCHECK(hipGetLastError());
}

void layer_stack(const LayerPtrs* lp, int layers, size_t seq_off, const MMArgs& qa, const MMPlan& pq, float* attn_scratch, int* attn_cnt,
                 uint8_t* af, const MMArgs& oa, const MMPlan& po, const MMArgs& ga, const MMPlan& pg, const MMArgs& da,
                 const MMPlan& pd, const MMScratch& sc, int* ctl, hipStream_t s, unsigned long long* timeline) {
    const int heads = qa.heads, kvh = qa.kv_heads, hd = qa.hd, t = qa.n;
    if (const char* why = layer_stack_unfit(t, heads, kvh, hd, pq, po, pg, pd)) throw std::runtime_error(why);
    if (pd.nsplit > 1 && (!sc.part || !sc.cnt)) throw std::runtime_error("split matrix launch without scratch");
    if (layers < 1) throw std::runtime_error("the layer stack needs at least one layer");
    const AttnArgs aa = make_attn_args(qa.out, qa.ldo, t, heads, kvh, hd, qa.pos0, AttnRows{}, nullptr, nullptr, attn_scratch, attn_cnt, af);
    LayerFlows lf;
    lf.ctl = ctl;
    lf.layers = layers;
    lf.tl = timeline;
    lf.gu_per = 128 * pd.wide * pd.kw / (16 * GU_STRIPS);
    lf.m_a = std::min<int>(FL_MIRRORS, po.nrb);
    lf.m_o = std::min<int>(FL_MIRRORS, pg.nrb);
    lf.m_d = std::min<int>(FL_MIRRORS, pq.nrb);
    lf.m_g = std::min<int>(FLOW_GU_MIRRORS, pd.nrb);
    switch (hd) {
        case 16: launch_layers<16>(lp, layers, seq_off, qa, pq, aa, oa, po, ga, pg, da, pd, sc, lf, s); break;
        case 32: launch_layers<32>(lp, layers, seq_off, qa, pq, aa, oa, po, ga, pg, da, pd, sc, lf, s); break;
        case 64: launch_layers<64>(lp, layers, seq_off, qa, pq, aa, oa, po, ga, pg, da, pd, sc, lf, s); break;
        default: launch_layers<128>(lp, layers, seq_off, qa, pq, aa, oa, po, ga, pg, da, pd, sc, lf, s); break;
    }
}

int mm_head(const MMArgs& a, const MMPlan& p, const MMScratch& sc, hipStream_t s) {
    if (a.fin_cnt && (a.arg_off != 0 || a.n > HEAD_FIN_MAX || !a.fin_ctl || !a.fin_block || !a.fin_amax || !a.fin_host || !a.row0))
        throw std::runtime_error("the head's own final reduction takes one launch of at most 128 tokens and all its buffers");
    // LDS: fragments, 1 / rms, per-wavefront partials, then the final reduction's flag and argmax.
    const size_t lds = size_t(a.W.n_chunks) * (tile_chunk_cols(a.W.bits) / 32) * 3 * 1024 + FTOK * 4 + HEAD_WAVES_MAX * FTOK * 8 +
                       (a.fin_cnt ? 4 * (1 + HEAD_FIN_MAX) : 0);
    const int copy_slots = a.W.n_chunks * (tile_chunk_cols(a.W.bits) / 32) * 3 * 64;  // 16-byte fragment slots of a tile
    const int min_threads = 64 * std::min(head_waves<true>(), head_waves<false>());
    // One tile whose full fragments do not fit: the live tokens' slots only.
    const size_t lds_cmp = lds - size_t(copy_slots) * 16 + size_t(copy_slots / 64) * 4 * std::min(a.n, FTOK) * 16;
    const bool cmp = p.rg == 1 && p.s == 4 && p.tiles == 1 && (lds > HEAD_LDS_MAX || copy_slots > HEAD_BMAX * min_threads) &&
                     lds_cmp <= HEAD_LDS_MAX;
    if (!cmp && (p.rg != 1 || p.s != 4 || lds > HEAD_LDS_MAX || copy_slots > HEAD_BMAX * min_threads)) {
        MMArgs g = a;
        g.fin_cnt = nullptr;
        launch<EPI_HEAD, 4>(g, p, sc, s);
        if (a.fin_cnt) {
            // The generic path leaves the final reduction to its own kernel and a copy.
            head_argmax_final(a.arg_val, a.arg_idx, a.arg_stride, p.nrb, a.row0, a.n, a.fin_amax, a.fin_block,
                              reinterpret_cast<uint32_t*>(a.fin_ctl + FLOW_ACC), s);
            FCHECK(hipMemcpyAsync(a.fin_host, a.fin_ctl, (FLOW_ACC + 2) * 4, hipMemcpyDeviceToHost, s));
        }
        return p.nrb;
    }
    // One workgroup per CU (the fragments fill most of its LDS).
    const int n_groups = p.nrb;
    const bool g16 = a.W.bits != 16 && a.W.group == 16;
    const bool mt = p.tiles > 1 && !cmp;
    const int waves = g16 ? head_waves<true>() : (mt ? head_waves<false, true>() : head_waves<false>());
    const int blocks = std::min(device_cu_count(), (n_groups + waves - 1) / waves);
    const dim3 grid(blocks, p.tiles), block(64 * waves);
    if (cmp) {
        switch (a.W.bits) {
            case 16: go(k_head<16, false, true>, grid, block, lds_cmp, s, a, n_groups); break;
            case 8:
                if (g16) go(k_head<8, true, true>, grid, block, lds_cmp, s, a, n_groups);
                else go(k_head<8, false, true>, grid, block, lds_cmp, s, a, n_groups);
                break;
            default:
                if (g16) go(k_head<4, true, true>, grid, block, lds_cmp, s, a, n_groups);
                else go(k_head<4, false, true>, grid, block, lds_cmp, s, a, n_groups);
                break;
        }
        FCHECK(hipGetLastError());
        return blocks;
    }
    switch (a.W.bits) {
        case 16:
            if (mt) go(k_head<16, false, false, true>, grid, block, lds, s, a, n_groups);
            else go(k_head<16, false>, grid, block, lds, s, a, n_groups);
            break;
        case 8:
            if (g16) go(k_head<8, true>, grid, block, lds, s, a, n_groups);
            else if (mt) go(k_head<8, false, false, true>, grid, block, lds, s, a, n_groups);
            else go(k_head<8, false>, grid, block, lds, s, a, n_groups);
            break;
        default:
            if (g16) go(k_head<4, true>, grid, block, lds, s, a, n_groups);
            else if (mt) go(k_head<4, false, false, true>, grid, block, lds, s, a, n_groups);
            else go(k_head<4, false>, grid, block, lds, s, a, n_groups);
            break;
    }
    FCHECK(hipGetLastError());
    return blocks;
}

// Wavefront w of workgroup b reduces tokens 16 b + w, then 16 more workgroups on (lane-strided
// partials, loads issued eight at a time, then a shuffle tree; `beats` is a total order, so the
// grouping does not matter). With a verify block (one workgroup), thread 0 then applies greedy
// acceptance (src/spec.rs:119-127): m = first i < n - 1 with amax[i] != block[i + 1] (else
// n - 1), next = amax[m].
__global__ __launch_bounds__(1024) void k_head_final(const float* __restrict__ pv, const int* __restrict__ pi, int arg_stride,
                                                     int nblocks, const float* __restrict__ row0, int n,
                                                     uint32_t* __restrict__ amax, const uint32_t* __restrict__ block,
                                                     uint32_t* __restrict__ acc) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    for (int i = blockIdx.x * 16 + w; i < n; i += 16 * gridDim.x) {
        const size_t base = size_t(i / FTOK) * arg_stride * FTOK + i % FTOK;
        float v = NAN;
        int ix = 0x7fffffff;
        for (int b0 = lane; b0 < nblocks; b0 += 8 * 64) {
            float xv[8];
            int xi[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int b = b0 + 64 * u;
                xv[u] = NAN;
                xi[u] = 0x7fffffff;
                if (b < nblocks) {
                    xv[u] = pv[base + size_t(b) * FTOK];
                    xi[u] = pi[base + size_t(b) * FTOK];
                }
            }
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (beats(xv[u], xi[u], v, ix)) {
                    v = xv[u];
                    ix = xi[u];
                }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(v, o, 64);
            const int oi = __shfl_xor(ix, o, 64);
            if (beats(ov, oi, v, ix)) {
                v = ov;
                ix = oi;
            }
        }
        if (lane == 0) amax[i] = isnan(row0[i]) ? 0u : uint32_t(ix);
    }
    if (!block) return;
    __syncthreads();
    if (threadIdx.x == 0) {
        int m = 0;
        while (m < n - 1 && amax[m] == block[m + 1]) m++;
        acc[0] = uint32_t(m);
        acc[1] = amax[m];
    }
}

void head_argmax_final(const float* pv, const int* pi, int arg_stride, int nblocks, const float* row0, int n, uint32_t* amax,
                       const uint32_t* block, uint32_t* acc, hipStream_t s) {
    // One workgroup when it also decides the acceptance (which needs every row), else one per
    // 16 rows.
    const int nwg = block ? 1 : (n + 15) / 16;
    hipLaunchKernelGGL(k_head_final, dim3(nwg), dim3(1024), 0, s, pv, pi, arg_stride, nblocks, row0, n, amax, block, acc);
    FCHECK(hipGetLastError());
}

__global__ void k_accept_batch(const uint32_t* __restrict__ amax, const uint32_t* __restrict__ tok, const int* __restrict__ first,
                               const int* __restrict__ len, int n_seq, const int* __restrict__ ctl, uint32_t* __restrict__ out) {
    for (int q = blockIdx.x * blockDim.x + threadIdx.x; q < n_seq; q += gridDim.x * blockDim.x) {
        const int f = first[q], n = len[q];
        int m = 0;
        while (m < n - 1 && amax[f + m] == tok[f + m + 1]) m++;
        out[1 + 2 * q] = uint32_t(m);
        out[2 + 2 * q] = amax[f + m];
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) out[0] = uint32_t(ctl[FLOW_ERR]);
}

__global__ void k_chain_step(const int* __restrict__ ctl, int* __restrict__ stage, uint32_t* __restrict__ out, int i, int n) {
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        const int next = ctl[FLOW_ACC + 1];
        out[i] = uint32_t(next);
        out[n] = uint32_t(ctl[FLOW_ERR]);
        stage[0] += 1;
        stage[1] = next;
    }
}

void chain_step(const int* ctl, int* stage, uint32_t* out, int i, int n, hipStream_t s) {
    hipLaunchKernelGGL(k_chain_step, dim3(1), dim3(64), 0, s, ctl, stage, out, i, n);
    FCHECK(hipGetLastError());
}

void accept_greedy_batch(const uint32_t* amax, const uint32_t* tok, const int* first, const int* len, int n_seq, const int* ctl,
                         uint32_t* out, hipStream_t s) {
    hipLaunchKernelGGL(k_accept_batch, dim3(1), dim3(256), 0, s, amax, tok, first, len, n_seq, ctl, out);
    FCHECK(hipGetLastError());
}

}  // namespace ls
