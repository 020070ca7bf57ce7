// Single-token f32 dot of the GGUF types without an int8 path (quant.rs:
// 377-441): one add chain per row, products formed by other wavefronts,
// weights in their GGUF row layout.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

// LDS bytes of a launch with rows of k elements (x is staged whole).
size_t pi_gemv_row_lds_bytes(uint32_t k);
// y[r] = dot_row_scalar(type, W + r * row_bytes, k, x) for r < rows; x and y
// in device memory.  Types: Q4_1, Q5_0, Q5_1, Q8_1, Q2_K, Q3_K, Q5_K, Q8_K and
// BF16 (k a multiple of 32).
hipError_t pi_launch_gemv_row(uint32_t type, const uint8_t *w, uint64_t row_bytes, uint32_t rows, uint32_t k,
                              const float *x, float *y, hipStream_t s);
