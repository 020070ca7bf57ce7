// Launchers of the gfx950 kernels outside the decode step (pi_kernels.hip).
// All launch on `s` and return hipSuccess or the launch error; none
// synchronizes.
#pragma once

#include <hip/hip_runtime_api.h>

#include "pi_common.h"

// Decode-step state kept in HBM so one captured graph serves every position.
struct pi_state {
    int32_t  pos;     // position of the token being evaluated
    uint32_t tok;     // token being evaluated
    uint32_t n_gen;   // generated ids written so far
    uint32_t i;       // prompt index during prefill
};

enum pi_gemv_mode { PI_GEMV_OUT = 0, PI_GEMV_RESIDUAL = 1, PI_GEMV_SUMS = 2 };

// Native GGML rows -> lane-interleaved tiles (layout in pi_common.h).
hipError_t pi_launch_repack(const uint8_t *src_native, uint8_t *dst, const pi_layout &L, hipStream_t s);

// Q8Act::prepare (quant_int.rs:17-56); x feature-major [k][b].
hipError_t pi_launch_q8(const float *x, uint32_t k, uint32_t b, int8_t *q, float *d, int32_t *sum,
                        hipStream_t s);

// Fills n positions of every (layer, kv head) with N(0,1) draws.
// dst = src for `words` 16-byte words (both 16-byte aligned).
hipError_t pi_launch_copy16(const void *src, void *dst, uint64_t words, hipStream_t s);
hipError_t pi_launch_kv_fill(float *kc, float *vc, uint32_t n_layer_heads, uint32_t n_ctx,
                             uint32_t dh, uint32_t n, uint64_t seed, hipStream_t s);

// Workgroups of the head GEMV, i.e. argmax partials reduced by the step kernel.
constexpr uint32_t PI_HEAD_BLOCKS = 512;
