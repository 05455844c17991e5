// The persistent layer pass for gfx950: every layer of a one-tile pass (at most 16 tokens) in one
// launch of one workgroup per CU. Each workgroup owns a fixed set of units per layer (a q|k|v
// strip, an attention key-block set, an o strip, a gate|up row block, a down row block and K
// split) and runs them in dataflow order, layer after layer. The units, their plans and their
// arithmetic are those of the per-layer launches (fused.hip), so the pass gives the same bits.
//
// Units hand their outputs to later units through tagged 16-byte units ({three words, tag}, tag =
// (epoch << 6) | layer) in an exchange area, and raise a flag line per unit with the same tag. A
// producer raises its flag right after issuing its stores (coherent sc1 stores, no wait for them);
// a consumer wavefront polls only the flags of the producers of its own K range, reads their
// units through the coherent path and reads again any unit whose tag is not yet this pass's. So a
// handoff costs one store-to-load trip, not a store acknowledgement, a counter update and a
// separate read. The area has two sets of buffers (even and odd layers): a unit of layer l + 2
// cannot run before every unit of layer l has read its inputs, since every unit of layer l feeds
// the residual rows that layer l + 1 needs.
//
// Every wait is bounded and also stops once the control block's error word is set; a wait that
// gives up sets it, and the launch then drains (its results are invalid and the host reports it).
// All workgroups must be resident at once: the grid is one workgroup per CU and the launch asks
// for more than half of a CU's LDS.
#include "pass.hpp"

#include "attn_dev.hpp"
#include "frag_dev.hpp"
#include "mm_dev.hpp"

#include <hip/hip_ext.h>

#include <algorithm>
#include <cmath>
#include <stdexcept>
#include <string>

namespace ls {

#define PCHECK(x)                                                                                         \
    do {                                                                                                  \
        hipError_t e_ = (x);                                                                              \
        if (e_ != hipSuccess) throw std::runtime_error(std::string("HIP: ") + hipGetErrorString(e_)); \
    } while (0)

constexpr unsigned PASS_SPIN = 1u << 22;  // polls before a wait gives up
constexpr int PASS_THREADS = 512;
constexpr int PS_UNIT_STAGES = 5;  // stages with units of their own: QKV, ATT, O, GU, DN
// Timeline stamps per unit: [0] start, [1 + w] wavefront w's input in registers, [9] wavefront 0's
// 1 / rms known, [10] every wavefront's products summed, [11] epilogue stores issued, [12] done,
// [13] wavefront 0's producers' flags seen; [14], [15] the number of times wavefront 0 fetched
// its input and its sums of squares again because a unit was stale; [16 + w] wavefront w's
// products done; [24] the flag's store acknowledged (with a timeline only, the unit waits for it).
constexpr int TL_STAMPS = 32;
enum { TL_START = 0, TL_IN = 1, TL_RMS = 9, TL_SUM = 10, TL_STORES = 11, TL_DONE = 12, TL_FLAGS = 13, TL_REIN = 14, TL_RERMS = 15,
       TL_MFMA = 16, TL_ACK = 24 };

// Units of 16 bytes.
__host__ __device__ constexpr int state_units(int hd) { return (hd + 2 + 2) / 3; }  // m, l, o[hd]
__host__ __device__ constexpr int piece_units(int rows) { return (rows + 2) / 3; }
// LDS of an attention unit: per-wavefront (max, sum) and outputs, its state, the other sets' states.
__host__ __device__ constexpr size_t pass_attn_lds(int hd) {
    return size_t(2 * AWV * ATQ + AWV * ATQ * (hd + 4) + ATQ * (2 + hd) * ASPLIT) * 4;
}

struct PassArgs {
    const LayerPtrs* lp;
    int layers;
    size_t seq_off;
    MMArgs qa, oa, ga, da;
    MMPlan pq, po, pg, pd;
    PassArea A;
    int* ctl;
    const int* epoch;
    uint64_t* timeline;
    int off[PS_UNIT_STAGES];  // workgroup of unit 0 of each stage
    int units[PS_UNIT_STAGES];
    int nt;  // tokens of the pass
    float scale;  // 1 / sqrt(head_dim)
};

// A buffer resource from values the wavefront holds in vector registers (the arguments' LDS
// copy): made uniform first, so that it lives in scalar registers and the loads through it need
// no per-lane descriptor loop.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t prsrc(const void* p, size_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(a)), hi = __builtin_amdgcn_readfirstlane(uint32_t(a >> 32));
    const int n = __builtin_amdgcn_readfirstlane(int(std::min<size_t>(bytes, 0x7ffffffc)));
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>((uint64_t(hi) << 32) | lo), 0, n, BUF_DWORD3);
}
__device__ __forceinline__ int pass_tag(int epoch, int l) { return (epoch << 6) | (l & 63); }
// The thread index through an empty asm: the per-unit address arithmetic that depends on it is
// redone for each unit instead of being hoisted out of the layer loop, where it would stay live
// (in registers) across every other stage.
__device__ __forceinline__ int ptid() {
    int t = int(threadIdx.x);
    asm volatile("" : "+v"(t));
    return t;
}
__device__ __forceinline__ bool pass_failed(const PassArgs& a) {
    return __hip_atomic_load(a.ctl + FLOW_ERR, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}
__device__ __forceinline__ void pass_fail(const PassArgs& a) {
    __hip_atomic_store(a.ctl + FLOW_ERR, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Byte offset of flag line (layer l, stage, unit) in the flag area.
__device__ __forceinline__ int flag_off(int l, int st, int u) { return ((((l & 1) * PS_STAGES + st) * PASS_MAXU) + u) * 64; }
// Byte offset of layer l's buffer set in the exchange area.
__device__ __forceinline__ size_t set_off(const PassArgs& a, int l) { return size_t(l & 1) * a.A.set_bytes; }

// One lane raises the flag after every wavefront of the workgroup has issued its stores.
__device__ __forceinline__ void raise_flag(const PassArgs& a, __amdgpu_buffer_rsrc_t rf, int l, int st, int u, int tag,
                                           uint64_t* stamp = nullptr) {
    __syncthreads();
    if (ptid() == 0) {
        __builtin_amdgcn_raw_buffer_store_b32(uint32_t(tag), rf, flag_off(l, st, u), 0, CPOL_SC1);
        if (stamp) {
            __builtin_amdgcn_s_waitcnt(0);
            stamp[TL_ACK] = __builtin_amdgcn_s_memrealtime();
        }
    }
}

// Lanes [0, n) of the calling wavefront poll flags p0 .. p0 + n - 1 of (l, st) until each holds
// tag (n <= 64). False when the pass has failed (then nothing is waited for any more).
__device__ __forceinline__ bool wave_wait(const PassArgs& a, __amdgpu_buffer_rsrc_t rf, int l, int st, int p0, int n, int tag) {
    if (n <= 0) return true;
    const int lane = ptid() & 63;
    const int off = flag_off(l, st, p0 + min(lane, n - 1));
    for (unsigned spins = 0;; spins++) {
        const int v = lane < n ? int(__builtin_amdgcn_raw_buffer_load_b32(rf, off, 0, CPOL_SC1)) : tag;
        if (__all(v == tag)) return true;
        if ((spins & 63) == 0 && pass_failed(a)) return false;
        if (spins > PASS_SPIN) {
            if (lane == 0) pass_fail(a);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Calls fetch() (which loads this lane's units and says whether all their tags are this pass's)
// again on the lanes that got a stale unit, until the wavefront has everything.
template <class F>
__device__ __forceinline__ unsigned wave_fetch(const PassArgs& a, F fetch) {
    bool ok = fetch();
    unsigned spins = 0;
    for (; !__all(ok); spins++) {
        if ((spins & 63) == 63 && pass_failed(a)) break;
        if (spins > PASS_SPIN) {
            if ((ptid() & 63) == 0) pass_fail(a);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
        if (!ok) ok = fetch();
    }
    return spins;  // fetches after the first
}

// Tagged fragment slot (k-step ks, column group kg, token tok): 4 units {h, m, l, tag} of the
// value pairs (2j, 2j + 1), j < 4, so that a lane's three MFMA B operands are the units' first
// three words. Layout [ks][kg][16 tokens][4 units].
__device__ __forceinline__ int tfrag_off(int ks, int kg, int tok) { return ((ks * 4 + kg) * 16 + tok) * 64; }

__device__ __forceinline__ void tfrag_store(__amdgpu_buffer_rsrc_t r, size_t base, size_t stride, int copies, int ks, int kg, int tok,
                                            const float* v, int tag) {
    const int at = int(base) + tfrag_off(ks, kg, tok);
    u32x4 u[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        uint32_t h0, m0, l0, h1, m1, l1;
        split3(v[2 * j], h0, m0, l0);
        split3(v[2 * j + 1], h1, m1, l1);
        u[j] = u32x4{h0 | (h1 << 16), m0 | (m1 << 16), l0 | (l1 << 16), uint32_t(tag)};
    }
    for (int c = 0; c < copies; c++)
#pragma unroll
        for (int j = 0; j < 4; j++) __builtin_amdgcn_raw_buffer_store_b128(u[j], r, at + int(c * stride) + 16 * j, 0, CPOL_SC1);
}

// The lane's B operands of k-step ks (lane l: token l % 16, column group l / 16); tokens past nt
// get zeros. tfrag_issue loads the lane's 4 units (a lane past nt, or a k-step with nothing to
// load, reads an in-bounds unit it then ignores), tfrag_take unpacks them and checks the tags:
// the loads of all a wavefront's k-steps go out before the first is waited for.
__device__ __forceinline__ void tfrag_issue(__amdgpu_buffer_rsrc_t r, size_t base, int ks, int nt, bool real, u32x4* u) {
    const int lane = ptid() & 63, tok = lane & 15, kg = lane >> 4;
    const int at = int(base) + (real && tok < nt ? tfrag_off(ks, kg, tok) : 0);
#pragma unroll
    for (int j = 0; j < 4; j++) u[j] = __builtin_amdgcn_raw_buffer_load_b128(r, at + 16 * j, 0, CPOL_SC1);
}
__device__ __forceinline__ bool tfrag_take(const u32x4* u, int nt, bool real, int tag, uint4* B) {
    const bool on = real && (ptid() & 15) < nt;
    B[0] = on ? make_uint4(u[0][0], u[1][0], u[2][0], u[3][0]) : make_uint4(0, 0, 0, 0);
    B[1] = on ? make_uint4(u[0][1], u[1][1], u[2][1], u[3][1]) : make_uint4(0, 0, 0, 0);
    B[2] = on ? make_uint4(u[0][2], u[1][2], u[2][2], u[3][2]) : make_uint4(0, 0, 0, 0);
    return !on || (int(u[0][3]) == tag && int(u[1][3]) == tag && int(u[2][3]) == tag && int(u[3][3]) == tag);
}

// Residual rows of a 16-row strip for one token: 6 units, rows 3j .. 3j + 2 in unit j < 5, then
// (row 15, the strip's sum of squares, 0). Layout [strip][16 tokens][6 units].
__device__ __forceinline__ int rows_off(int strip, int tok, int j) { return ((strip * 16 + tok) * 6 + j) * 16; }

// Unit j of strip `strip` for token tok; x(r) gives row r of the strip (LDS), ss its sum of squares.
template <class X>
__device__ __forceinline__ void rows_store(__amdgpu_buffer_rsrc_t r, size_t base, int strip, int tok, int j, X x, float ss, int tag) {
    const float a = x(3 * j), b = j < 5 ? x(3 * j + 1) : ss, c = j < 5 ? x(3 * j + 2) : 0.0f;
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(a), __float_as_uint(b), __float_as_uint(c), uint32_t(tag)}, r,
                                           int(base) + rows_off(strip, tok, j), 0, CPOL_SC1);
}

// ---------------------------------------------------------------------------------------
// Matrix units
// ---------------------------------------------------------------------------------------
// Where a matrix unit's input fragments come from: written before the launch in the standard
// layout (prev_stage < 0), or tagged fragments of layer in_l's set whose columns come in blocks
// of cpp per producer unit of stage prev_stage. With a normalised input (a.ss for the standard
// layout; norm for the tagged one) 1 / rms comes from the producers' sums of squares, one per
// 16-column slot and token. Unit bx reads copy bx % P.A.repl of both.
struct PIn {
    int prev_stage = -1;
    int in_l = 0;
    size_t frag = 0, frag_r = 0;  // fragments: copy 0, bytes between copies
    size_t ss = 0;                // sums of squares (copy 0; P.A.ss_r between copies)
    int cpp = 16;
    bool norm = false;
};

template <int BITS, int EPI, bool G16, int S>
__device__ __forceinline__ void pass_mm(const PassArgs& P, const MMArgs& a, const TMat& W, const float* __restrict__ rowvec, float* kcache,
                                        float* vcache, const MMPlan& p, const PIn& in, int l, int bx, int E, __amdgpu_buffer_rsrc_t rx,
                                        __amdgpu_buffer_rsrc_t rf, uint8_t* smem, uint64_t* stamp) {
    const int tag = pass_tag(E, l), tag_in = pass_tag(E, in.in_l);
    constexpr int Q = Steps<BITS>::Q, CPW = Steps<BITS>::CPW;
    const int nw = p.rg * p.kw;
    const int wv = __builtin_amdgcn_readfirstlane(ptid() >> 6), lane = ptid() & 63;
    const int rb = bx / p.nsplit, sp = bx % p.nsplit;
    const int rows_wg = 16 * S * p.rg, row0 = rb * rows_wg;
    const int nt = P.nt;
    const int rgi = wv / p.kw, kw = wv % p.kw;
    const int s0 = (rb * p.rg + rgi) * S;
    const int c0 = (sp * p.kw + kw) * CPW;
    const int nch = min(CPW, W.n_chunks - c0);
    const bool active = wv < nw;

    const size_t red_bytes = p.kw > 1 ? size_t(nw) * S * 64 * 16 : 0;
    float* tl = reinterpret_cast<float*>(smem + red_bytes);
    float* inv = tl + rows_wg * FTOK;
    float* vec = inv + FTOK;                // per-row vector (bias or the output norm)
    float* xs = vec + rows_wg;              // residual rows [rows_wg][16]
    float* rcos = xs + rows_wg * FTOK;      // RoPE tables [16][half]
    float* rsin = rcos + FTOK * (EPI == EPI_QKV ? a.hd / 2 : 0);
    int* tpos = reinterpret_cast<int*>(rsin + FTOK * (EPI == EPI_QKV ? a.hd / 2 : 0));  // [position][cache row]
    float* ov = reinterpret_cast<float*>(tpos + 2 * FTOK);  // q|k|v outputs [16][16] by tile row

    // Order of the unit's first memory operations: the epilogue operands (into registers, written
    // to LDS after the products), one poll of the producers' flags, then the weights. A unit that
    // starts after its inputs are ready (its workgroup's previous unit ended late) so learns that
    // before its weights arrive, and fetches its input while they are in flight.
    const int t = ptid();
    const int ks0 = c0 * Q, nks = active ? max(0, nch) * Q : 0;
    const int real_ks = W.cols / 32;  // k-steps past the matrix's columns are padding: zero inputs
    const bool tagged = in.prev_stage >= 0;
    // Only wavefront 0 polls (every waiting wavefront polling the same few flag lines slows each
    // poll down): for the producers of the unit's k-steps, or of every column with a normalised
    // input (1 / rms needs all their sums of squares). The others wait for it at a barrier.
    const bool rms_here = tagged && wv == 0 && in.norm;
    int q0 = 0, qn = 0;
    if (tagged && wv == 0) {
        const int u_ks0 = sp * p.kw * CPW * Q, u_ks1 = min(min((sp + 1) * p.kw * CPW, W.n_chunks) * Q, real_ks);
        if (in.norm) qn = (W.cols + in.cpp - 1) / in.cpp;
        else if (u_ks1 > u_ks0) {
            q0 = u_ks0 * 32 / in.cpp;
            qn = (u_ks1 * 32 - 1) / in.cpp - q0 + 1;
        }
    }
    constexpr bool down = EPI == EPI_RESID && S == DOWN_STRIPS;  // o runs one strip per wavefront, down DOWN_STRIPS
    const int half = EPI == EPI_QKV ? a.hd / 2 : 0;
    float r_vec = 0.0f, r_cos = 0.0f, r_sin = 0.0f;
    u32x4 r_res = {0, 0, 0, 0};
    int res_tag = 0;
    size_t res_base = 0;
    if constexpr (EPI == EPI_QKV) {
        const int qk = (a.heads + a.kv_heads) * a.hd;
        if (t < rows_wg && row0 + t < W.rows) r_vec = rowvec[qkv_ref_row(row0 + t, a.hd, qk)];
        if (t < nt * half) {
            const size_t at = size_t(*a.pos0 + t / half) * half + t % half;
            r_cos = a.rope_cos[at];
            r_sin = a.rope_sin[at];
        }
    } else if constexpr (EPI == EPI_RESID) {
        if (t < rows_wg && row0 + t < W.rows) r_vec = rowvec[row0 + t];
        // The residual rows (split 0 of down adds them): written before the launch (layer 0's o) or
        // tagged rows of an earlier unit, long written when this unit starts: o of layer l reads
        // the rows down of layer l - 1 left, down the rows o left. Their tags are checked after
        // the products (no flag wait).
        if (!down || sp == 0) {
            if (!down && l == 0) {
                if (t < rows_wg * FTOK && t % FTOK < nt) r_res[0] = __float_as_uint(a.out[size_t(t % FTOK) * a.ldo + row0 + t / FTOK]);
            } else {
                const int src_l = down ? l : l - 1;
                res_tag = pass_tag(E, src_l);
                res_base = set_off(P, src_l) + (down ? P.A.xar : P.A.xr);
                if (t < (rows_wg / 16) * nt * 6) {
                    const int st = t / (nt * 6), tok = (t / 6) % nt, j = t % 6;
                    r_res = __builtin_amdgcn_raw_buffer_load_b128(rx, int(res_base) + rows_off(row0 / 16 + st, tok, j), 0, CPOL_SC1);
                }
            }
        }
    }
    const int pv = qn > 0 ? int(__builtin_amdgcn_raw_buffer_load_b32(rf, flag_off(in.in_l, in.prev_stage, q0 + min(lane, qn - 1)), 0, CPOL_SC1))
                          : tag_in;

    uint4 raw[CPW][S];
    uint4 B[CPW * Q][3];
    uint2 scl[CPW][scale_slots<BITS, G16>()][S];
    if (active) {
        const uint8_t* wb = W.data + (size_t(s0) * W.n_chunks * 64 + lane) * 16;
        const size_t sst = size_t(W.n_chunks) * 1024;
#pragma unroll
        for (int c = 0; c < CPW; c++)
            if (c < nch) {
                load_chunk<S>(wb, sst, c0 + c, raw[c]);
                if constexpr (BITS != 16) load_scales<BITS, G16, S>(W, s0, c0 + c, (c0 + nch) * Q, scl[c]);
            }
    }

    // Input fragments of this wavefront's k-steps.
    if (in.prev_stage < 0) {
        if (active && nks > 0) {
            const uint4* fb = reinterpret_cast<const uint4*>(a.frags) + lane;
#pragma unroll
            for (int c = 0; c < CPW; c++)
                if (c < nch)
#pragma unroll
                    for (int q = 0; q < Q; q++)
#pragma unroll
                        for (int u = 0; u < 3; u++) B[c * Q + q][u] = fb[(((c0 + c) * Q + q) * 3 + u) * 64];
        }
    } else {
        if (qn > 0 && !__all(pv == tag_in)) wave_wait(P, rf, in.in_l, in.prev_stage, q0, qn, tag_in);
        if (stamp && t == 0) stamp[TL_FLAGS] = __builtin_amdgcn_s_memrealtime();
        __syncthreads();
        if (rms_here) {
            // 1 / rms per token (src/kernels.rs:217-228 up to the summation order): lane (part,
            // token) adds slots part, part + 4, ... in order, then a fixed shuffle tree, as rms_finish.
            const size_t sbase = set_off(P, in.in_l) + in.ss + size_t(bx % P.A.repl) * P.A.ss_r;
            const int tok = lane & 15, part = lane >> 4, slots = ss_slots(W.cols);
            float v = 0.0f;
            for (int k0 = 0; 4 * k0 < slots; k0 += 16) {  // uniform: past the last slot a lane adds zeros
                float x[16];
                const unsigned re = wave_fetch(P, [&]() {
                    // every lane loads (lanes with nothing to add an in-bounds unit they ignore)
                    u32x2 u[16];
#pragma unroll
                    for (int k = 0; k < 16; k++) {
                        const int sl = part + 4 * (k0 + k);
                        const bool on = sl < slots && tok < nt;
                        u[k] = __builtin_amdgcn_raw_buffer_load_b64(rx, int(sbase) + (on ? (sl * 16 + tok) * 8 : 0), 0, CPOL_SC1);
                    }
                    bool ok = true;
#pragma unroll
                    for (int k = 0; k < 16; k++) {
                        const int sl = part + 4 * (k0 + k);
                        const bool on = sl < slots && tok < nt;
                        x[k] = on ? __uint_as_float(u[k][0]) : 0.0f;
                        ok &= !on || int(u[k][1]) == tag_in;
                    }
                    return ok;
                });
#pragma unroll
                for (int k = 0; k < 16; k++) v += x[k];
                if (stamp && lane == 0) stamp[TL_RERMS] = re;
            }
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            if (lane < FTOK) inv[lane] = 1.0f / sqrtf(v / float(W.cols) + a.eps);
            if (stamp && lane == 0) stamp[TL_RMS] = __builtin_amdgcn_s_memrealtime();
        }
        if (active && nks > 0) {
            const size_t fbase = set_off(P, in.in_l) + in.frag + size_t(bx % P.A.repl) * in.frag_r;
            const unsigned re = wave_fetch(P, [&]() {
                u32x4 u[CPW * Q][4];
#pragma unroll
                for (int c = 0; c < CPW; c++)
#pragma unroll
                    for (int q = 0; q < Q; q++) {
                        const int ks = (c0 + c) * Q + q;
                        tfrag_issue(rx, fbase, ks, nt, c < nch && ks < real_ks, u[c * Q + q]);
                    }
                bool ok = true;
#pragma unroll
                for (int c = 0; c < CPW; c++)
#pragma unroll
                    for (int q = 0; q < Q; q++) {
                        const int ks = (c0 + c) * Q + q;
                        ok &= tfrag_take(u[c * Q + q], nt, c < nch && ks < real_ks, tag_in, B[c * Q + q]);
                    }
                return ok;
            });
            if (stamp && t == 0) stamp[TL_REIN] = re;
        }
    }
    if (stamp && lane == 0) stamp[TL_IN + wv] = __builtin_amdgcn_s_memrealtime();

    f32x4 total[S], acc[S];
#pragma unroll
    for (int r = 0; r < S; r++) total[r] = acc[r] = f32x4{0, 0, 0, 0};
    if (active) {
#pragma unroll
        for (int c = 0; c < CPW; c++)
            if (c < nch) chunk_mfma<BITS, G16, S, true>(W, s0, c0 + c, c0 * Q, (c0 + nch) * Q, &B[c * Q], raw[c], acc, total, scl[c]);
    }
    if (stamp && lane == 0) stamp[TL_MFMA + wv] = __builtin_amdgcn_s_memrealtime();
    // 1 / rms of an input written before the launch (wavefront 0; src/kernels.rs:217-228 up to the
    // summation order), from the sums of squares stored with it.
    if (wv == 0 && in.prev_stage < 0 && a.ss) {
        RmsLoads r;
        rms_issue(a, 0, r);
        rms_finish(a, 0, W.cols, r, inv);
    }
    // The epilogue operands into LDS (made visible by the barrier below).
    if (t < rows_wg) vec[t] = r_vec;
    if constexpr (EPI == EPI_QKV) {
        if (t < nt) tpos[t] = tpos[FTOK + t] = *a.pos0 + t;
        if (t < nt * half) {
            rcos[t] = r_cos;  // [token][half]: t = token * half + j
            rsin[t] = r_sin;
        }
    } else if constexpr (EPI == EPI_RESID) {
        if (!down || sp == 0) {
            if (!down && l == 0) {
                if (t < rows_wg * FTOK) xs[t] = __uint_as_float(r_res[0]);  // [row][token]: t = row * FTOK + token
            } else if (t < (rows_wg / 16) * nt * 6) {
                const int st = t / (nt * 6), tok = (t / 6) % nt, j = t % 6;
                unsigned spins = 0;
                while (int(r_res[3]) != res_tag) {  // stale (not seen in practice): read it again
                    if ((++spins & 63) == 0 && pass_failed(P)) break;
                    if (spins > PASS_SPIN) {
                        pass_fail(P);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                    r_res = __builtin_amdgcn_raw_buffer_load_b128(rx, int(res_base) + rows_off(row0 / 16 + st, tok, j), 0, CPOL_SC1);
                }
#pragma unroll
                for (int k = 0; k < 3; k++)
                    if (3 * j + k < 16) xs[(16 * st + 3 * j + k) * FTOK + tok] = __uint_as_float(r_res[k]);
            }
        }
    }
    // Row-group tile: the kw wavefront sums added in wavefront order (as mm_body).
    if (p.kw > 1) {
        f32x4* red = reinterpret_cast<f32x4*>(smem);
        if (active)
#pragma unroll
            for (int r = 0; r < S; r++) red[(wv * S + r) * 64 + lane] = total[r];
        __syncthreads();
        for (int e = ptid(); e < p.rg * S * 64; e += PASS_THREADS) {
            const int g = e / (S * 64), r = (e / 64) % S, ln = e % 64;
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
    } else if (active) {
#pragma unroll
        for (int r = 0; r < S; r++)
#pragma unroll
            for (int i = 0; i < 4; i++) tl[(16 * (S * rgi + r) + 4 * (lane >> 4) + i) * FTOK + (lane & 15)] = total[r][i];
    }
    __syncthreads();
    if (stamp && ptid() == 0) stamp[TL_SUM] = __builtin_amdgcn_s_memrealtime();

    if constexpr (EPI == EPI_QKV) {
        // q|k|v: 1 / rms, bias, RoPE on q and k rows (src/kernels.rs:242-252), as mm_body; the K/V
        // rows go to the cache (read by later passes), and every row to the tagged q|k|v buffer for
        // this layer's attention: a strip holds two octets of 8 reference dims per token.
        const int hd = a.hd, half = hd / 2, h = a.heads * hd, kvd = a.kv_heads * hd;
        for (int e = ptid(); e < rows_wg * FTOK; e += PASS_THREADS) {
            const int rl = e / FTOK, tok = e % FTOK, row = row0 + rl;
            if (tok >= nt || row >= W.rows) continue;
            const int crow = tpos[FTOK + tok];
            const float iv = a.ss ? inv[tok] : 1.0f;
            float v = __fadd_rn(a.ss ? __fmul_rn(tl[e], iv) : tl[e], vec[rl]);
            int ref = row;
            if (row < h + kvd) {
                const int r = row % hd, j = r >> 1, pr = rl ^ 1;
                const float pv = __fadd_rn(a.ss ? __fmul_rn(tl[pr * FTOK + tok], iv) : tl[pr * FTOK + tok], vec[pr]);
                const float c = rcos[tok * half + j], sn = rsin[tok * half + j];
                if ((r & 1) == 0) {
                    v = __fsub_rn(__fmul_rn(v, c), __fmul_rn(pv, sn));
                    ref = row - r + j;
                } else {
                    v = __fadd_rn(__fmul_rn(v, c), __fmul_rn(pv, sn));
                    ref = row - r + half + j;
                }
            }
            ov[rl * FTOK + tok] = v;
            if (ref >= h && ref < h + kvd) kcache[size_t(crow) * kvd + (ref - h)] = v;
            else if (ref >= h + kvd) vcache[size_t(crow) * kvd + (ref - h - kvd)] = v;
        }
        __syncthreads();
        // Octets of this strip: q and k strips hold dims 8 r' + [0, 8) (even tile rows) and
        // half + 8 r' + [0, 8) (odd tile rows) of their head; v strips 16 r' + [0, 16) in order.
        const int noct = (h + 2 * kvd) / 8;
        const bool paired = row0 < h + kvd;
        const int head_base = row0 - row0 % hd, rp = (row0 % hd) / 16;
        const size_t qbase = set_off(P, l) + P.A.qkvx;
        for (int e = ptid(); e < nt * 2 * 3; e += PASS_THREADS) {
            const int tok = e / 6, o = (e / 3) % 2, j = e % 3;
            const int dim0 = paired ? head_base + o * half + 8 * rp : row0 + 8 * o;  // reference dim of the octet's first value
            float w3[3];
#pragma unroll
            for (int k = 0; k < 3; k++) {
                const int m = 3 * j + k;  // value m of the octet
                const int trow = paired ? 2 * m + o : 8 * o + m;
                w3[k] = m < 8 ? ov[trow * FTOK + tok] : 0.0f;
            }
            __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(w3[0]), __float_as_uint(w3[1]), __float_as_uint(w3[2]), uint32_t(tag)},
                                                   rx, int(qbase) + ((tok * noct + dim0 / 8) * 3 + j) * 16, 0, CPOL_SC1);
        }
        if (stamp && ptid() == 0) stamp[TL_STORES] = __builtin_amdgcn_s_memrealtime();
        raise_flag(P, rf, l, PS_QKV, rb, tag, stamp);
    } else if constexpr (EPI == EPI_SILU) {
        const int hw = rows_wg / 2;
        for (int e = ptid(); e < hw * FTOK; e += PASS_THREADS) {
            const int tok = e % FTOK;
            float v = 0.0f;
            if (tok < nt) {
                float g = tl[e], up = tl[hw * FTOK + e];
                if (in.norm) {
                    g = __fmul_rn(g, inv[tok]);
                    up = __fmul_rn(up, inv[tok]);
                }
                v = __fmul_rn(g / (1.0f + expf(-g)), up);
            }
            tl[e] = v;
        }
        __syncthreads();
        const size_t fbase = set_off(P, l) + P.A.actf;
        for (int q = ptid(); q < (hw / 8) * nt; q += PASS_THREADS) {
            const int cg = q / nt, tok = q % nt, col = hw * rb + 8 * cg;
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = tl[(8 * cg + j) * FTOK + tok];
            tfrag_store(rx, fbase, P.A.actf_r, P.A.repl, col / 32, (col % 32) / 8, tok, v, tag);
        }
        if (stamp && ptid() == 0) stamp[TL_STORES] = __builtin_amdgcn_s_memrealtime();
        raise_flag(P, rf, l, PS_GU, rb, tag, stamp);
    } else {
        // Residual epilogues: o (one strip, nsplit 1) or down (row blocks of 32, K split; split 0
        // adds the pieces of the others in split order, as the last-arriver fixup does).
        const int elems = rows_wg * FTOK;
        if (p.nsplit > 1) {
            const int PU = piece_units(rows_wg);
            const size_t pbase = set_off(P, l) + P.A.dnp;
            if (sp != 0) {
                for (int e = ptid(); e < nt * PU; e += PASS_THREADS) {
                    const int tok = e / PU, j = e % PU;
                    float w3[3];
#pragma unroll
                    for (int k = 0; k < 3; k++) {
                        const int rl = 3 * j + k;
                        w3[k] = rl < rows_wg ? tl[rl * FTOK + tok] : 0.0f;
                    }
                    __builtin_amdgcn_raw_buffer_store_b128(
                        u32x4{__float_as_uint(w3[0]), __float_as_uint(w3[1]), __float_as_uint(w3[2]), uint32_t(tag)}, rx,
                        int(pbase) + (((rb * p.nsplit + sp) * 16 + tok) * PU + j) * 16, 0, CPOL_SC1);
                }
                if (stamp && ptid() == 0) stamp[TL_STORES] = __builtin_amdgcn_s_memrealtime();
                raise_flag(P, rf, l, PS_DNP, bx, tag, stamp);
                return;
            }
            // Split 0: wait for the other splits of this row block, then sum in split order.
            if (wv == 0) wave_wait(P, rf, l, PS_DNP, bx + 1, p.nsplit - 1, tag);
            __syncthreads();
            for (int e = ptid(); e < nt * rows_wg; e += PASS_THREADS) {
                const int tok = e / rows_wg, rl = e % rows_wg, j = rl / 3, k = rl % 3;
                // every split's piece loaded at once (again while one is stale), then split 0's
                // piece and the others added in split order
                float pc[MAX_SPLIT];
                unsigned spins = 0;
                for (bool ok = false; !ok;) {
                    u32x4 u[MAX_SPLIT];
#pragma unroll
                    for (int s2 = 1; s2 < MAX_SPLIT; s2++)
                        if (s2 < p.nsplit)
                            u[s2] = __builtin_amdgcn_raw_buffer_load_b128(rx, int(pbase) + (((rb * p.nsplit + s2) * 16 + tok) * PU + j) * 16, 0,
                                                                          CPOL_SC1);
                    ok = true;
#pragma unroll
                    for (int s2 = 1; s2 < MAX_SPLIT; s2++)
                        if (s2 < p.nsplit) {
                            ok &= int(u[s2][3]) == tag;
                            pc[s2] = __uint_as_float(k == 0 ? u[s2][0] : k == 1 ? u[s2][1] : u[s2][2]);
                        }
                    if (!ok) {
                        if ((++spins & 63) == 0 && pass_failed(P)) break;
                        if (spins > PASS_SPIN) {
                            pass_fail(P);
                            break;
                        }
                        __builtin_amdgcn_s_sleep(1);
                    }
                }
                float sum = tl[rl * FTOK + tok];
#pragma unroll
                for (int s2 = 1; s2 < MAX_SPLIT; s2++)
                    if (s2 < p.nsplit) sum += pc[s2];
                tl[rl * FTOK + tok] = sum;
            }
            __syncthreads();
        }
        (void)elems;
        // The residual rows are in LDS (the last wavefront fetched them before the products).
        const int strips = rows_wg / 16;
        const bool last = down && l + 1 == P.layers;
        for (int e = ptid(); e < rows_wg * FTOK; e += PASS_THREADS) {
            const int rl = e / FTOK, tok = e % FTOK;
            tl[e] = tok < nt && row0 + rl < W.rows ? __fadd_rn(xs[e], tl[e]) : 0.0f;
        }
        __syncthreads();
        if (last) {
            // After the last layer: the standard layouts the head reads after this launch (x rows,
            // fragments of x * final norm, sums of squares), plain stores.
            for (int e = ptid(); e < rows_wg * FTOK; e += PASS_THREADS) {
                const int rl = e / FTOK, tok = e % FTOK;
                if (tok < nt) a.out[size_t(tok) * a.ldo + row0 + rl] = tl[e];
            }
            for (int q = ptid(); q < (rows_wg / 8) * FTOK; q += PASS_THREADS) {
                const int cg = q / FTOK, tok = q % FTOK, col = row0 + 8 * cg;
                float v[8];
#pragma unroll
                for (int j = 0; j < 8; j++) v[j] = __fmul_rn(tl[(8 * cg + j) * FTOK + tok], vec[8 * cg + j]);
                write_slot(a.ofrags, col / 32, tok + 16 * ((col % 32) / 8), v);
            }
            for (int q = ptid(); q < strips * FTOK; q += PASS_THREADS) {
                const int g = q / FTOK, tok = q % FTOK;
                a.oss[(row0 / 16 + g) * FTOK + tok] = ss16([&](int c) { return tl[(16 * g + c) * FTOK + tok]; }, 16);
            }
            return;
        }
        // Tagged outputs for the next stage: rows (+ sums of squares) and fragments of rows * norm.
        const size_t rbase = set_off(P, l) + (down ? P.A.xr : P.A.xar);
        const size_t fbase = set_off(P, l) + (down ? P.A.xf : P.A.xaf);
        const size_t sbase = set_off(P, l) + (down ? P.A.xss : P.A.xass);
        for (int e = ptid(); e < strips * nt * 6; e += PASS_THREADS) {
            const int st = e / (nt * 6), tok = (e / 6) % nt, j = e % 6;
            auto xrow = [&](int c) { return tl[(16 * st + c) * FTOK + tok]; };
            const float ssv = j == 5 ? ss16(xrow, 16) : 0.0f;
            rows_store(rx, rbase, row0 / 16 + st, tok, j, xrow, ssv, tag);
            if (j == 5)
                for (int c = 0; c < P.A.repl; c++)
                    __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(ssv), uint32_t(tag)}, rx,
                                                          int(sbase + c * P.A.ss_r) + ((row0 / 16 + st) * 16 + tok) * 8, 0, CPOL_SC1);
        }
        for (int q = ptid(); q < (rows_wg / 8) * nt; q += PASS_THREADS) {
            const int cg = q / nt, tok = q % nt, col = row0 + 8 * cg;
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = __fmul_rn(tl[(8 * cg + j) * FTOK + tok], vec[8 * cg + j]);
            tfrag_store(rx, fbase, down ? P.A.xf_r : P.A.xaf_r, P.A.repl, col / 32, (col % 32) / 8, tok, v, tag);
        }
        if (stamp && ptid() == 0) stamp[TL_STORES] = __builtin_amdgcn_s_memrealtime();
        raise_flag(P, rf, l, down ? PS_FIX : PS_O, rb, tag, stamp);
    }
}

// ---------------------------------------------------------------------------------------
// Attention units
// ---------------------------------------------------------------------------------------
// Unit (head, s) of attn_body's decomposition: AWV wavefronts, key block b taken by wavefront
// b mod (AWV ASPLIT) of workgroup (b mod (AWV ASPLIT)) / AWV, online softmax per wavefront, the
// wavefronts merged in order in LDS. q and the keys and values of this pass's positions come from
// the tagged q|k|v buffer, older keys and values from the cache. Set 0 then merges the sets in set
// order, as the last-arriver merge does, and writes the head's output fragments.
// N consecutive reference dims of token tok starting at dim, from the tagged q|k|v buffer: the
// octets that hold them are read whole (static register indices) and the run picked out of them.
// N is a power of two; a run shorter than an octet starts at a multiple of N.
// Lanes with on false load an in-bounds unit, get zeros and pass the tag check, so that the loads
// of a lane's runs go out together.
__device__ __forceinline__ bool octet_load(__amdgpu_buffer_rsrc_t rx, size_t base, int noct, int tok, int o, float* v, int tag, bool on) {
    const int at = int(base) + (on ? (tok * noct + o) * 3 * 16 : 0);
    u32x4 u[3];
#pragma unroll
    for (int j = 0; j < 3; j++) u[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, at + j * 16, 0, CPOL_SC1);
    bool ok = true;
#pragma unroll
    for (int j = 0; j < 3; j++) {
        ok &= !on || int(u[j][3]) == tag;
#pragma unroll
        for (int k = 0; k < 3; k++)
            if (3 * j + k < 8) v[3 * j + k] = on ? __uint_as_float(u[j][k]) : 0.0f;
    }
    return ok;
}
template <int N>
__device__ __forceinline__ bool octet_get(__amdgpu_buffer_rsrc_t rx, size_t base, int noct, int tok, int dim, float* out, int tag, bool on) {
    bool ok = true;
    if constexpr (N >= 8) {
#pragma unroll
        for (int q = 0; q < N / 8; q++) ok &= octet_load(rx, base, noct, tok, dim / 8 + q, out + 8 * q, tag, on);
    } else {
        float v[8];
        ok = octet_load(rx, base, noct, tok, dim / 8, v, tag, on);
        const int off = dim % 8;
#pragma unroll
        for (int i = 0; i < N; i++) {
            float x = v[i];
#pragma unroll
            for (int cand = N; cand < 8; cand += N)
                if (off == cand) x = v[cand + i];
            out[i] = x;
        }
    }
    return ok;
}

template <int HD>
__device__ __forceinline__ void pass_attn(const PassArgs& P, int l, int head, int s, int tag, __amdgpu_buffer_rsrc_t rx, __amdgpu_buffer_rsrc_t rf,
                          uint8_t* smem, uint64_t* stamp) {
    constexpr int H4 = HD / 4, DB = HD / 16;
    const MMArgs& qa = P.qa;
    const LayerPtrs& L = P.lp[l];
    const float* __restrict__ kc = L.kc + P.seq_off;
    const float* __restrict__ vc = L.vc + P.seq_off;
    const int heads = qa.heads, kv_heads = qa.kv_heads, nq = P.nt;
    const int tid = ptid(), w = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
    const int kv = kv_heads * HD, grp = head / (heads / kv_heads), col0 = grp * HD;
    const int h = heads * HD, noct = (h + 2 * kv) / 8;
    const int pos0 = *qa.pos0;
    const int last_key = pos0 + nq - 1, nb = last_key / AKB + 1;
    const int first = s * AWV + w, stride = ASPLIT * AWV;
    const size_t qbase = set_off(P, l) + P.A.qkvx;

    float(*sm_m)[ATQ] = reinterpret_cast<float(*)[ATQ]>(smem);
    float(*sm_l)[ATQ] = reinterpret_cast<float(*)[ATQ]>(smem + AWV * ATQ * 4);
    constexpr int HP = HD + 4;
    float* sm_o = reinterpret_cast<float*>(smem + 2 * AWV * ATQ * 4);
    // this set's state per token after the wavefront merge: [token][2 + HD] (m, l, o)
    float* st = sm_o + AWV * ATQ * HP;

    AttnBlock<HD> ba;
    const int nold = pos0 / AKB;  // blocks below hold only cached keys
    // a block's keys: cached ones from the caches, this pass's from the tagged buffer
    auto load_block = [&](AttnBlock<HD>& r, int b) -> bool {
        if (b < nold) {
            attn_load<HD>(r, b, last_key, kc, vc, kv, col0, g, c);
            return true;
        }
        // keys of this pass from the tagged buffer (every lane loads; others get zeros), cached
        // ones from the cache
        const int key = AKB * b + c;
        const bool knew = key >= pos0 && key <= last_key;
        bool ok = octet_get<H4>(rx, qbase, noct, knew ? key - pos0 : 0, h + col0 + g * H4, r.k, tag, knew);
        if (key < pos0) {
            const float* kp = kc + size_t(key) * kv + col0 + g * H4;
#pragma unroll
            for (int j = 0; j < H4; j++) r.k[j] = kp[j];
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int vk = AKB * b + 4 * g + u;
            if (vk > last_key) {
#pragma unroll
                for (int db = 0; db < DB; db++) r.v[u * DB + db] = 0.0f;
            } else if (vk < pos0) {
                const float* vp = vc + size_t(vk) * kv + col0 + DB * c;
#pragma unroll
                for (int db = 0; db < DB; db++) r.v[u * DB + db] = vp[db];
            } else {
                ok &= octet_get<DB>(rx, qbase, noct, vk - pos0, h + kv + col0 + DB * c, &r.v[u * DB], tag, true);
            }
        }
        return ok;
    };
    if (first < nb && first < nold) load_block(ba, first);
    // q and this pass's keys: the q strips of this head and the k and v strips of its group
    // (wavefront 0 polls, the others wait for it at a barrier)
    const int sph = HD / 16;
    if (w == 0) {
        wave_wait(P, rf, l, PS_QKV, head * sph, sph, tag);
        wave_wait(P, rf, l, PS_QKV, heads * sph + grp * sph, sph, tag);
        wave_wait(P, rf, l, PS_QKV, (heads + kv_heads) * sph + grp * sph, sph, tag);
        if (stamp && tid == 0) stamp[TL_FLAGS] = __builtin_amdgcn_s_memrealtime();
    }
    __syncthreads();
    float qr[H4];
    const unsigned re = wave_fetch(P, [&]() {
        bool ok = octet_get<H4>(rx, qbase, noct, c < nq ? c : 0, head * HD + g * H4, qr, tag, c < nq);
        if (first < nb && first >= nold) ok &= load_block(ba, first);
        return ok;
    });
    if (stamp && tid == 0) stamp[TL_REIN] = re;
    if (stamp && lane == 0) stamp[TL_IN + w] = __builtin_amdgcn_s_memrealtime();

    float M = -INFINITY, Lp = 0.0f;
    attn_f32x4 O[DB];
#pragma unroll
    for (int db = 0; db < DB; db++) O[db] = attn_f32x4{0, 0, 0, 0};
    const float scale = P.scale;
    auto block = [&](int b, const AttnBlock<HD>& r) {
        attn_f32x4 sc = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < H4; j++) sc = mfma_f32(r.k[j], qr[j], sc);
        float sv[4];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int key = AKB * b + 4 * g + i;
            sv[i] = (c < nq && key <= pos0 + c) ? sc[i] * scale : -INFINITY;
            mx = fmaxf(mx, sv[i]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float Mn = fmaxf(M, mx);
        const float corr = M == -INFINITY ? 0.0f : expf(M - Mn);
        float pr[4], ls = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            pr[i] = sv[i] == -INFINITY ? 0.0f : expf(sv[i] - Mn);
            ls += pr[i];
        }
        Lp = __builtin_fmaf(Lp, corr, ls);
        M = Mn;
#pragma unroll
        for (int db = 0; db < DB; db++) {
            attn_f32x4 acc = {0, 0, 0, 0};
#pragma unroll
            for (int u = 0; u < 4; u++) acc = mfma_f32(r.v[u * DB + db], pr[u], acc);
#pragma unroll
            for (int i = 0; i < 4; i++) O[db][i] = __builtin_fmaf(O[db][i], corr, acc[i]);
        }
    };
    for (int b = first; b < nb; b += stride) {
        if (b != first) wave_fetch(P, [&]() { return load_block(ba, b); });
        block(b, ba);
    }

    // The wavefronts merged in wavefront order (attn_body).
    float Lw0 = Lp + __shfl_xor(Lp, 16, 64);
    Lw0 += __shfl_xor(Lw0, 32, 64);
    if (g == 0) {
        sm_m[w][c] = M;
        sm_l[w][c] = Lw0;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float* dst = &sm_o[(w * ATQ + c) * HP + DB * (4 * g + i)];
#pragma unroll
        for (int db = 0; db < DB; db++) dst[db] = O[db][i];
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
        float* sr = st + tk * (2 + HD);
        if (d == 0) {
            sr[0] = Mx;
            sr[1] = Lw;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) sr[2 + d + i] = ow[i];
    }
    __syncthreads();
    if (stamp && tid == 0) stamp[TL_SUM] = __builtin_amdgcn_s_memrealtime();
    constexpr int SU = state_units(HD);
    const size_t sbase = set_off(P, l) + P.A.atts;
    if (s != 0) {
        for (int e = tid; e < nq * SU; e += AWV * 64) {
            const int tk = e / SU, j = e % SU;
            const float* sr = st + tk * (2 + HD);
            float w3[3];
#pragma unroll
            for (int k = 0; k < 3; k++) w3[k] = 3 * j + k < 2 + HD ? sr[3 * j + k] : 0.0f;
            __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(w3[0]), __float_as_uint(w3[1]), __float_as_uint(w3[2]), uint32_t(tag)},
                                                   rx, int(sbase) + (((head * ASPLIT + s) * 16 + tk) * SU + j) * 16, 0, CPOL_SC1);
        }
        if (stamp && tid == 0) stamp[TL_STORES] = __builtin_amdgcn_s_memrealtime();
        raise_flag(P, rf, l, PS_ATT, head * ASPLIT + s, tag, stamp);
        return;
    }
    // Set 0 merges the sets in set order (attn_body's last-arriver merge): the other sets' states
    // into LDS beside its own, then each thread (row, sub) merges DPT dims.
    float* peers = st + ATQ * (2 + HD);  // [set 1..][token][2 + HD]
    if (w == 0) wave_wait(P, rf, l, PS_ATT, head * ASPLIT + 1, ASPLIT - 1, tag);
    __syncthreads();
    {
        // every thread's units loaded at once (again while one is stale)
        constexpr int PER = ((ASPLIT - 1) * ATQ * SU + AWV * 64 - 1) / (AWV * 64);
        const int total = (ASPLIT - 1) * nq * SU;
        unsigned spins = 0;
        for (bool ok = false; !ok;) {
            u32x4 u[PER];
#pragma unroll
            for (int i = 0; i < PER; i++) {
                const int e = tid + i * AWV * 64;
                const int s2 = 1 + e / (nq * SU), tk = (e / SU) % nq, j = e % SU;
                u[i] = __builtin_amdgcn_raw_buffer_load_b128(
                    rx, int(sbase) + (e < total ? (((head * ASPLIT + s2) * 16 + tk) * SU + j) * 16 : 0), 0, CPOL_SC1);
            }
            ok = true;
#pragma unroll
            for (int i = 0; i < PER; i++) {
                const int e = tid + i * AWV * 64;
                if (e >= total) continue;
                const int s2 = 1 + e / (nq * SU), tk = (e / SU) % nq, j = e % SU;
                ok &= int(u[i][3]) == tag;
                float* sr = peers + ((s2 - 1) * ATQ + tk) * (2 + HD);
#pragma unroll
                for (int k = 0; k < 3; k++)
                    if (3 * j + k < 2 + HD) sr[3 * j + k] = __uint_as_float(u[i][k]);
            }
            if (!ok) {
                if ((++spins & 63) == 0 && pass_failed(P)) break;
                if (spins > PASS_SPIN) {
                    pass_fail(P);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
    }
    __syncthreads();
    constexpr int DPT = HD / 16;
    float* Os = sm_o;  // [ATQ][HD] output rows
    const int row = tid >> 4, sub = tid & 15;
    if (row < nq) {
        float mv[ASPLIT], lv[ASPLIT], ovv[ASPLIT][DPT];
#pragma unroll
        for (int k = 0; k < ASPLIT; k++) {
            const float* sr = k == 0 ? st + row * (2 + HD) : peers + ((k - 1) * ATQ + row) * (2 + HD);
            mv[k] = sr[0];
            lv[k] = sr[1];
#pragma unroll
            for (int u = 0; u < DPT; u++) ovv[k][u] = sr[2 + sub * DPT + u];
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
            for (int u = 0; u < DPT; u++) o[u] = __builtin_fmaf(ovv[k][u], e, o[u]);
        }
        const float inv = 1.0f / Lt;
#pragma unroll
        for (int u = 0; u < DPT; u++) Os[row * HD + sub * DPT + u] = o[u] * inv;
    }
    __syncthreads();
    const size_t fbase = set_off(P, l) + P.A.af;
    for (int q = tid; q < nq * (HD / 8); q += AWV * 64) {
        const int i = q / (HD / 8), sl = q % (HD / 8), col = head * HD + 8 * sl;
        tfrag_store(rx, fbase, P.A.af_r, P.A.repl, col / 32, (col % 32) / 8, i, Os + i * HD + 8 * sl, tag);
    }
    if (stamp && tid == 0) stamp[TL_STORES] = __builtin_amdgcn_s_memrealtime();
    raise_flag(P, rf, l, PS_MRG, head, tag, stamp);
}

// ---------------------------------------------------------------------------------------
// The kernel
// ---------------------------------------------------------------------------------------
// LDS of a pass workgroup: the units' space, then a copy of the arguments. The units read the
// arguments from that copy: it is memory the loop writes (LDS), so the compiler does not hoist the
// values derived from them out of the layer loop and keep them live (in registers) across it.
constexpr size_t PASS_ARGS_LDS = 4096;
__host__ __device__ constexpr size_t pass_lds(int hd) {
    return (pass_attn_lds(hd) + PASS_ARGS_LDS > (size_t(96) << 10) ? pass_attn_lds(hd) + PASS_ARGS_LDS : (size_t(96) << 10));
}

template <int HD, int BITS, bool G16>
__global__ __launch_bounds__(PASS_THREADS) void k_pass(PassArgs Pk) {
    extern __shared__ __align__(16) uint8_t smem[];
    static_assert(sizeof(PassArgs) <= PASS_ARGS_LDS && sizeof(PassArgs) % 4 == 0, "pass arguments fit their LDS copy");
    PassArgs* Ps = reinterpret_cast<PassArgs*>(smem + pass_lds(HD) - PASS_ARGS_LDS);
    for (int i = ptid(); i < int(sizeof(PassArgs) / 4); i += PASS_THREADS)
        reinterpret_cast<int*>(Ps)[i] = reinterpret_cast<const int*>(&Pk)[i];
    __syncthreads();
    const PassArgs& P = *Ps;
    const int G = int(gridDim.x), wg = int(blockIdx.x);
    const int E = *P.epoch;
    const __amdgpu_buffer_rsrc_t rx = prsrc(P.A.base, 2 * P.A.set_bytes);
    const __amdgpu_buffer_rsrc_t rf = prsrc(P.A.flags, P.A.flag_bytes);
#pragma clang loop unroll(disable)
    for (int l = 0; l < P.layers; l++) {
        const LayerPtrs& L = P.lp[l];
        const int tag = pass_tag(E, l);
#pragma clang loop unroll(disable)
        for (int st = 0; st < PS_UNIT_STAGES; st++) {
            int u = (wg - P.off[st] + G) % G;
            if (u >= P.units[st]) continue;
            asm volatile("" : "+s"(u));
            uint64_t* stamp = P.timeline ? P.timeline + ((size_t(wg) * P.layers + l) * PS_UNIT_STAGES + st) * TL_STAMPS : nullptr;
            if (stamp && ptid() == 0) stamp[TL_START] = __builtin_amdgcn_s_memrealtime();
            if (st == 0) {
                PIn in;
                if (l > 0) {
                    in.prev_stage = PS_FIX;
                    in.in_l = l - 1;
                    in.frag = P.A.xf;
                    in.frag_r = P.A.xf_r;
                    in.ss = P.A.xss;
                    in.cpp = 32;
                    in.norm = true;
                }
                pass_mm<BITS, EPI_QKV, G16, 1>(P, P.qa, L.qkv, L.b_qkv, L.kc + P.seq_off, L.vc + P.seq_off, P.pq, in, l, u, E, rx, rf, smem,
                                               stamp);
            } else if (st == 1) {
                pass_attn<HD>(P, l, u / ASPLIT, u % ASPLIT, tag, rx, rf, smem, stamp);
            } else if (st == 2) {
                PIn in;
                in.prev_stage = PS_MRG;
                in.in_l = l;
                in.frag = P.A.af;
                in.frag_r = P.A.af_r;
                in.cpp = HD;
                pass_mm<BITS, EPI_RESID, G16, 1>(P, P.oa, L.o, L.post_norm, nullptr, nullptr, P.po, in, l, u, E, rx, rf, smem, stamp);
            } else if (st == 3) {
                PIn in;
                in.prev_stage = PS_O;
                in.in_l = l;
                in.frag = P.A.xaf;
                in.frag_r = P.A.xaf_r;
                in.ss = P.A.xass;
                in.cpp = 16;
                in.norm = true;
                pass_mm<BITS, EPI_SILU, G16, gu_wave_strips(BITS, G16 ? 16 : 32)>(P, P.ga, L.gu, nullptr, nullptr, nullptr, P.pg, in, l, u, E,
                                                                                  rx, rf, smem, stamp);
            } else {
                PIn in;
                in.prev_stage = PS_GU;
                in.in_l = l;
                in.frag = P.A.actf;
                in.frag_r = P.A.actf_r;
                in.cpp = 16 * GU_STRIPS;
                pass_mm<BITS, EPI_RESID, G16, DOWN_STRIPS>(P, P.da, L.down, L.next_norm, nullptr, nullptr, P.pd, in, l, u, E, rx, rf, smem,
                                                           stamp);
            }
            __syncthreads();
            if (stamp && ptid() == 0) stamp[TL_DONE] = __builtin_amdgcn_s_memrealtime();
        }
    }
}

// ---------------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------------
static size_t up256(size_t v) { return (v + 255) & ~size_t(255); }

PassArea pass_area_shape(int hidden, int heads, int kv_heads, int hd, int inter, const MMPlan& pd, int repl) {
    if (repl < 1 || repl > PASS_MAX_REPL) throw std::runtime_error("pass buffer copies out of range");
    PassArea A;
    A.repl = repl;
    const int h = heads * hd, kvd = kv_heads * hd;
    const size_t frag_ks = size_t(4) * 16 * 64;  // one k-step of tagged fragments
    size_t off = 0;
    auto take = [&](size_t& at, size_t bytes) {
        at = off;
        off = up256(off + bytes);
    };
    // copies 256 bytes past a multiple of 256, so that copy r starts on another channel
    auto take_r = [&](size_t& at, size_t& stride, size_t bytes) {
        at = off;
        stride = up256(bytes) + 256;
        off = up256(off + size_t(repl) * stride);
    };
    take(A.qkvx, size_t(16) * ((h + 2 * kvd) / 8) * 3 * 16);
    take(A.atts, size_t(heads) * ASPLIT * 16 * state_units(hd) * 16);
    take_r(A.af, A.af_r, size_t(tile_kpad(h) / 32) * frag_ks);
    take(A.xar, size_t(hidden / 16) * 16 * 6 * 16);
    take_r(A.xaf, A.xaf_r, size_t(tile_kpad(hidden) / 32) * frag_ks);
    take_r(A.actf, A.actf_r, size_t(tile_kpad(inter) / 32) * frag_ks);
    take(A.dnp, size_t(pd.nrb) * pd.nsplit * 16 * piece_units(16 * pd.s * pd.rg) * 16);
    take(A.xr, size_t(hidden / 16) * 16 * 6 * 16);
    take_r(A.xf, A.xf_r, size_t(tile_kpad(hidden) / 32) * frag_ks);
    take_r(A.xass, A.ss_r, size_t(hidden / 16) * 16 * 8);
    size_t ss_r2 = 0;
    take_r(A.xss, ss_r2, size_t(hidden / 16) * 16 * 8);
    A.set_bytes = off;
    if (2 * A.set_bytes > size_t(1) << 31) throw std::runtime_error("pass exchange area above 2 GiB");
    A.flag_bytes = size_t(2) * PS_STAGES * PASS_MAXU * 64;
    return A;
}

PassArea pass_area_bind(const PassArea& shape, uint8_t* base, int* flags) {
    PassArea A = shape;
    A.base = base;
    A.flags = flags;
    return A;
}

size_t pass_timeline_words(int layers) { return size_t(device_cu_count()) * layers * PS_UNIT_STAGES * TL_STAMPS; }

const char* layer_pass_unfit(int t, int heads, int kv_heads, int hd, const MMPlan& pq, const MMPlan& po, const MMPlan& pg,
                             const MMPlan& pd) {
    if (t > FTOK) return "the persistent pass takes one token tile";
    if (pq.wide != 1 || po.wide != 1 || pg.wide != 1 || pd.wide != 1) return "the persistent pass takes 128-column K shares";
    if (hd != 16 && hd != 32 && hd != 64) return "head_dim must be 16, 32 or 64";
    if ((heads * hd) % 32 || hd % 16) return "q|k|v rows must fill whole k-steps";
    if (heads % kv_heads) return "heads must be a multiple of kv_heads";
    if (pq.nsplit != 1 || pq.rg != 1 || pq.s != 1 || 64 * pq.kw > PASS_THREADS) return "q|k|v plan";
    if (po.nsplit != 1 || po.rg != 1 || po.s != 1 || 64 * po.kw > PASS_THREADS) return "o plan";
    if (pg.nsplit != 1 || 64 * pg.rg * pg.kw > PASS_THREADS || pg.s * pg.rg != 2 * GU_STRIPS) return "gate|up plan";
    if (pd.s != DOWN_STRIPS || pd.rg != 1 || 64 * pd.kw > PASS_THREADS || pd.nsplit > MAX_SPLIT) return "down plan";
    const int G = device_cu_count();
    if (pq.nrb > G || ASPLIT * heads > G || po.nrb > G || pg.nrb > G || pd.nrb * pd.nsplit > G || G > PASS_MAXU)
        return "a stage has more units than the device has CUs";
    if (po.nrb > 64 || pd.nrb > 64) return "more producers than a wavefront polls";
    return nullptr;
}

template <class K>
static void launch_k(K kernel, size_t lds, hipStream_t s, const PassArgs& P) {
    hipLaunchKernelGGL(kernel, dim3(device_cu_count()), dim3(PASS_THREADS), lds, s, P);
}

template <int HD>
static void launch_pass(const PassArgs& P, int bits, bool g16, hipStream_t s) {
    // One workgroup per CU: more than half of a CU's LDS (attention at head_dim 128 needs more).
    const size_t lds = pass_lds(HD);
    switch (bits) {
        case 16: launch_k(k_pass<HD, 16, false>, lds, s, P); break;
        case 8:
            if (g16) launch_k(k_pass<HD, 8, true>, lds, s, P);
            else launch_k(k_pass<HD, 8, false>, lds, s, P);
            break;
        default:
            if (g16) launch_k(k_pass<HD, 4, true>, lds, s, P);
            else launch_k(k_pass<HD, 4, false>, lds, s, P);
            break;
    }
    PCHECK(hipGetLastError());
}

void layer_pass(const LayerPtrs* lp, int layers, size_t seq_off, const MMArgs& qa, const MMPlan& pq, const MMArgs& oa,
                const MMPlan& po, const MMArgs& ga, const MMPlan& pg, const MMArgs& da, const MMPlan& pd, const PassArea& area,
                int* ctl, const int* epoch, uint64_t* timeline, hipStream_t s) {
    if (const char* why = layer_pass_unfit(qa.n, qa.heads, qa.kv_heads, qa.hd, pq, po, pg, pd)) throw std::runtime_error(why);
    if (layers < 1 || layers > 63) throw std::runtime_error("the persistent pass takes 1 to 63 layers");
    if (!area.base || !area.flags || !epoch || !ctl) throw std::runtime_error("persistent pass without its exchange area");
    const int G = device_cu_count();
    PassArgs P;
    P.lp = lp;
    P.layers = layers;
    P.seq_off = seq_off;
    P.qa = qa;
    P.oa = oa;
    P.ga = ga;
    P.da = da;
    P.pq = pq;
    P.po = po;
    P.pg = pg;
    P.pd = pd;
    P.A = area;
    P.ctl = ctl;
    P.epoch = epoch;
    P.timeline = timeline;
    P.nt = qa.n;
    P.scale = 1.0f / sqrtf(float(qa.hd));
    P.units[0] = pq.nrb;
    P.units[1] = ASPLIT * qa.heads;
    P.units[2] = po.nrb;
    P.units[3] = pg.nrb;
    P.units[4] = pd.nrb * pd.nsplit;
    // Consecutive stages on different workgroups, so that a workgroup's next unit has its weights
    // in flight well before its input arrives.
    P.off[0] = 0;
    P.off[1] = P.units[0] % G;
    P.off[2] = (P.off[1] + P.units[1]) % G;
    P.off[3] = (P.off[2] + P.units[2]) % G;
    P.off[4] = (P.off[3] + P.units[3]) % G;
    const bool g16 = qa.W.bits != 16 && qa.W.group == 16;
    switch (qa.hd) {
        case 16: launch_pass<16>(P, qa.W.bits, g16, s); break;
        case 32: launch_pass<32>(P, qa.W.bits, g16, s); break;
        default: launch_pass<64>(P, qa.W.bits, g16, s); break;
    }
}

}  // namespace ls
