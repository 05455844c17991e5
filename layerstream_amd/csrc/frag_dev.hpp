// Device helpers that write B fragments (fused.hpp describes the layout). Only for .hip sources.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace ls {

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

}  // namespace ls
