// kernels::matmul (src/kernels.rs:196-203) without any device allocation, for callers that cannot
// allocate (code under HIP graph capture, allocation-free serving loops). It runs the kernels of
// the allocating operator (tile repack, input fragments, the residual matrix kernel) on the same
// inputs, so its output is bit-identical; what that operator allocates per call (the tile-layout
// copy of the weights, the input fragments, the split-K pieces and counters) lives here in one
// file-scope device array instead. Every GPU that runs this holds its own copy of the array until
// the process ends. Calls on one GPU share it: calls that overlap in time on one GPU race.
#include "static_mm.hpp"

#include <algorithm>
#include <mutex>
#include <stdexcept>
#include <string>

namespace ls {

#define SCHECK(x)                                                                                         \
    do {                                                                                                  \
        hipError_t e_ = (x);                                                                              \
        if (e_ != hipSuccess) throw std::runtime_error(std::string("HIP: ") + hipGetErrorString(e_)); \
    } while (0)

// The scratch array. In host code its name is only a stand-in for the symbol: the device address
// comes from hipGetSymbolAddress, once per device, and only that address is handed to kernels.
static __device__ __align__(256) uint8_t scratch[STATIC_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
uint8_t* g_ptr[MAX_DEVICES] = {};

size_t up256(size_t v) { return (v + 255) & ~size_t(255); }

struct Layout {
    size_t data = 0, scales = 0, frags = 0, part = 0, cnt = 0, total = 0;
};

Layout layout_of(const TMat& shape, const MMPlan& plan, int cols) {
    Layout L;
    size_t off = 0;
    L.data = off;
    off = up256(off + tile_data_bytes(shape));
    L.scales = off;
    off = up256(off + tile_scale_bytes(shape));
    L.frags = off;
    off = up256(off + frag_tile_bytes(cols) * size_t(plan.tiles));
    L.part = off;
    off = up256(off + mm_part_floats(plan) * 4);
    L.cnt = off;
    off = up256(off + mm_counters(plan) * 4);
    L.total = off;
    return L;
}
}  // namespace

// This device's copy of the array (its address is looked up on the first call on each device).
static uint8_t* scratch_ptr() {
    int dev = 0;
    SCHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= MAX_DEVICES) throw std::runtime_error("device ordinal out of range for the static scratch table");
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            throw std::runtime_error(std::string("the static scratch array has no device address: ") + hipGetErrorString(e));
        g_ptr[dev] = static_cast<uint8_t*>(p);
    }
    return g_ptr[dev];
}

// Fill kernel (in place of memsets, which a graph capture would record as memset nodes).
__global__ __launch_bounds__(256) void k_fill32(uint32_t* __restrict__ p, uint32_t v, size_t n) {
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) p[i] = v;
}

static void fill32(void* p, uint32_t v, size_t bytes, hipStream_t s) {
    const size_t n = bytes / 4;
    if (!n) return;
    const unsigned blocks = unsigned(std::min<size_t>((n + 255) / 256, 1024));
    hipLaunchKernelGGL(k_fill32, dim3(blocks), dim3(256), 0, s, static_cast<uint32_t*>(p), v, n);
    SCHECK(hipGetLastError());
}

size_t matmul_static_bytes(int bits, int group, int rows, int cols, int t) {
    const TMat shape = tile_shape(bits, group, rows, cols);
    return layout_of(shape, mm_plan(shape, 1, 8, t, 1), cols).total;
}

void matmul_static(int bits, int group, const uint8_t* w, int rows, int cols, const float* x, int t, float* y, hipStream_t s) {
    const TMat shape = tile_shape(bits, group, rows, cols);
    const MMPlan plan = mm_plan(shape, 1, 8, t, 1);
    const Layout L = layout_of(shape, plan, cols);
    if (L.total > STATIC_SCRATCH_BYTES)
        throw std::invalid_argument("a " + std::to_string(rows) + " x " + std::to_string(cols) + " matrix over " + std::to_string(t) +
                                    " inputs needs " + std::to_string(L.total) + " bytes of scratch, above the static limit of " +
                                    std::to_string(STATIC_SCRATCH_BYTES));
    uint8_t* base = scratch_ptr();
    const TMat W = tile_bind(shape, base + L.data, reinterpret_cast<uint16_t*>(base + L.scales));
    // Padding of the tile copy: zero weights (int4: the nibble 8 stores zero) and zero scales.
    fill32(base + L.data, bits == 4 ? 0x88888888u : 0u, tile_data_bytes(shape), s);
    if (bits != 16) fill32(base + L.scales, 0, tile_scale_bytes(shape), s);
    tile_repack(w, rows, W, 0, rows, rows, s);
    // y = W x through the residual kernel, y starting at zero; the fragments of the tokens past t
    // stay zero; split-K counters start at zero (the array keeps whatever the last call left).
    fill32(y, 0, size_t(t) * rows * 4, s);
    fill32(base + L.frags, 0, frag_tile_bytes(cols) * size_t(plan.tiles), s);
    x_frags(x, t, cols, nullptr, base + L.frags, nullptr, s);
    fill32(base + L.cnt, 0, mm_counters(plan) * 4, s);
    MMArgs a;
    a.W = W;
    a.frags = base + L.frags;
    a.frag_stride = frag_tile_bytes(cols);
    a.n = t;
    a.out = y;
    a.ldo = rows;
    mm_residual(a, plan, MMScratch{reinterpret_cast<float*>(base + L.part), reinterpret_cast<int*>(base + L.cnt)}, s);
}

}  // namespace ls
