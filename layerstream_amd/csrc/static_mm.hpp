// The matrix operator without device allocation (static_mm.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "fused.hpp"

namespace ls {

// Size of the file-scope device array that holds the operator's scratch (per GPU).
constexpr size_t STATIC_SCRATCH_BYTES = size_t(32) << 20;
// Scratch bytes one call needs (the tile-layout weights, input fragments, split-K pieces and
// counters).
size_t matmul_static_bytes(int bits, int group, int rows, int cols, int t);
// y[t][rows] = W x on stream s (asynchronous) with every buffer beyond w, x and y in the static
// array. Throws std::invalid_argument when the call needs more than STATIC_SCRATCH_BYTES.
void matmul_static(int bits, int group, const uint8_t* w, int rows, int cols, const float* x, int t, float* y, hipStream_t s);

}  // namespace ls
