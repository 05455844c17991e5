// Device helpers that write B fragments (fused.hpp describes the layout). Only for .hip sources.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "fused.hpp"

namespace ls {

// Cache policy of data handed between workgroups of one launch: sc1, coherent across the L2s
// of the XCDs.
constexpr int CPOL_SC1 = 16;
// Cache policy of data read once (weights): nt, streamed past the caches.
constexpr int CPOL_NT = 2;
constexpr int BUF_DWORD3 = 0x00020000;  // raw buffer resource word 3 on gfx9

// f32 value -> three bf16 terms (truncations) whose sum is the value exactly.
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

// Fragment slot (k-step ks, lane ln) of a tile: 8 values, columns 32 ks + 8 (ln / 16) + [0, 8) of
// token ln % 16.
__device__ __forceinline__ void write_slot(uint8_t* tile_frags, int ks, int ln, const float* v) {
    uint32_t H[4], M[4], L[4];
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        uint32_t h0, m0, l0, h1, m1, l1;
        split3(v[j], h0, m0, l0);
        split3(v[j + 1], h1, m1, l1);
        H[j / 2] = h0 | (h1 << 16);
        M[j / 2] = m0 | (m1 << 16);
        L[j / 2] = l0 | (l1 << 16);
    }
    uint4* o = reinterpret_cast<uint4*>(tile_frags + (size_t(ks) * 3 * 64 + ln) * 16);
    o[0] = make_uint4(H[0], H[1], H[2], H[3]);
    o[64] = make_uint4(M[0], M[1], M[2], M[3]);
    o[128] = make_uint4(L[0], L[1], L[2], L[3]);
}

// The same slot written through the coherent (sc1) path, for fragments read by later workgroups
// of the same launch. r covers the fragment buffer; tile_off is the tile's byte offset in it.
__device__ __forceinline__ void write_slot_coherent(__amdgpu_buffer_rsrc_t r, size_t tile_off, int ks, int ln, const float* v) {
    typedef uint32_t u32x4_ __attribute__((ext_vector_type(4)));
    uint32_t H[4], M[4], L[4];
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        uint32_t h0, m0, l0, h1, m1, l1;
        split3(v[j], h0, m0, l0);
        split3(v[j + 1], h1, m1, l1);
        H[j / 2] = h0 | (h1 << 16);
        M[j / 2] = m0 | (m1 << 16);
        L[j / 2] = l0 | (l1 << 16);
    }
    const int at = int(tile_off + (size_t(ks) * 3 * 64 + ln) * 16);
    __builtin_amdgcn_raw_buffer_store_b128(u32x4_{H[0], H[1], H[2], H[3]}, r, at, 0, 16);
    __builtin_amdgcn_raw_buffer_store_b128(u32x4_{M[0], M[1], M[2], M[3]}, r, at + 64 * 16, 0, 16);
    __builtin_amdgcn_raw_buffer_store_b128(u32x4_{L[0], L[1], L[2], L[3]}, r, at + 128 * 16, 0, 16);
}

// Waits of the in-launch dataflow (see Flow). Thread 0 polls with atomic adds of zero: a plain
// load, even at agent scope, can keep hitting this XCD's L2 copy of the line for microseconds,
// while an atomic is served at the coherence point. The zero is hidden from the compiler, which
// would otherwise turn the idempotent atomic back into a load. After a bounded number of sleeps
// the wait records an error and goes on, so every wave ends.
constexpr unsigned FLOW_SPIN_LIMIT = 1u << 22;

// A flow without a control block (a stage whose input was written before the launch) does not
// wait. Every 64 polls the wait also reads the error word, so that once one wait of a launch
// has given up, the others stop waiting at once and the launch drains.
// Consumer `who` (0, 1, ... among the counter's consumers) polls copy who % mirrors. With
// consumers > 0 the consumers count themselves and the last one puts the counter back to zero;
// with consumers == 0 a later workgroup of the launch does that (Flow::zero0).
__device__ __forceinline__ void flow_wait(const Flow& fl, int j, int who) {
    if (!fl.ctl) return;
    if (threadIdx.x == 0) {
        int* c0 = fl.ctl + FLOW_CNT0 + FLOW_CNT_STRIDE * (fl.base + j * fl.mirrors);
        int* cnt = c0 + FLOW_CNT_STRIDE * (who % fl.mirrors);
        const int want = fl.want > 0 ? fl.want : min(fl.producers, fl.per * (j + 1)) - fl.per * j;
        int zero = 0;
        asm volatile("" : "+v"(zero));
        unsigned spins = 0;
        while (__hip_atomic_fetch_add(cnt, zero, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < want) {
            if (++spins > FLOW_SPIN_LIMIT) {
                __hip_atomic_store(fl.ctl + FLOW_ERR, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            if ((spins & 63) == 0 && __hip_atomic_fetch_add(fl.ctl + FLOW_ERR, zero, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
                break;
            __builtin_amdgcn_s_sleep(2);
        }
        if (fl.stamp) *fl.stamp = __builtin_amdgcn_s_memrealtime();
        if (fl.consumers > 0) {
            const int old = __hip_atomic_fetch_add(c0 + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (old == fl.consumers - 1) {
                for (int m = 0; m < fl.mirrors; m++) __hip_atomic_store(c0 + FLOW_CNT_STRIDE * m, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(c0 + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    __syncthreads();
}

// The counter slots a producer puts back to zero (Flow::zero0, zero1), issued with its outputs so
// that the wait before its signal covers them too.
__device__ __forceinline__ void flow_zero(const Flow& fl) {
    for (int i = threadIdx.x; i < fl.nzero0; i += blockDim.x)
        __hip_atomic_store(fl.ctl + FLOW_CNT0 + FLOW_CNT_STRIDE * (fl.zero0 + i), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int i = threadIdx.x; i < fl.nzero1; i += blockDim.x)
        __hip_atomic_store(fl.ctl + FLOW_CNT0 + FLOW_CNT_STRIDE * (fl.zero1 + i), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Producer r: every output store of this workgroup has completed (s_waitcnt), then its counter
// moves. A flow without a control block has no consumers in this launch: nothing to signal.
// (qkv_signal below is the producer side for q|k|v -> attention.)
__device__ __forceinline__ void flow_signal(const Flow& fl, int r) {
    if (!fl.ctl) return;
    flow_zero(fl);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (int(threadIdx.x) < fl.mirrors)
        __hip_atomic_fetch_add(fl.ctl + FLOW_CNT0 + FLOW_CNT_STRIDE * (fl.base + (r / fl.per) * fl.mirrors + int(threadIdx.x)), 1,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// q|k|v strip r (16 rows: q heads, then k heads, then v heads, hd / 16 strips each) is stored:
// count it for every head that reads it, counter base + head (a q strip: its head; a k or v
// strip: the heads of its group). These counters have one copy (ATTN_SPLIT consumers each).
__device__ __forceinline__ void qkv_signal(const Flow& fl, int r, int heads, int kv_heads, int hd) {
    flow_zero(fl);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x != 0) return;
    const int sph = hd / 16, qs = heads * sph, ks = kv_heads * sph, group = heads / kv_heads;
    int h0 = 0, nh = 0;
    if (r < qs) {
        h0 = r / sph;
        nh = 1;
    } else if (r < qs + 2 * ks) {
        h0 = ((r - qs) % ks) / sph * group;
        nh = group;
    }
    for (int h = h0; h < h0 + nh; h++)
        __hip_atomic_fetch_add(fl.ctl + FLOW_CNT0 + FLOW_CNT_STRIDE * (fl.base + h), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace ls
