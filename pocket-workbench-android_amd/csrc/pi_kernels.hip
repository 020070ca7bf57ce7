// gfx950 kernels of the pocketinfer backend outside the decode step:
// weight repacking, Q8 activation quantization and the seeded KV fill.
#include <hip/hip_runtime.h>

#include "pi_gemv.h"
#include "pi_kernels.h"

using pig::q8_block32;

namespace {

// ---------------------------------------------------------------------------
// Repack: native GGML rows -> lane-interleaved tiles (layout in pi_common.h).
// One thread per unit.
// ---------------------------------------------------------------------------
__global__ void k_repack(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, pi_layout L,
                         uint64_t row_bytes, uint32_t blk_bytes, uint32_t qofs, uint32_t dofs,
                         uint32_t base_chunks, uint32_t base_df) {
    uint64_t n = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint64_t total = (uint64_t)L.rows * L.upr;
    if (n >= total) return;
    uint32_t r = (uint32_t)(n / L.upr), u = (uint32_t)(n % L.upr);
    uint32_t t = r / L.rpw;
    uint32_t lane = (uint32_t)(n - (uint64_t)t * L.lpt);
    uint32_t lanes = (t == L.ntiles - 1) ? (L.rows - t * L.rpw) * L.upr : L.lpt;
    uint8_t *tile = dst + (uint64_t)t * L.tile_bytes;
    const uint8_t *row = src + (uint64_t)r * row_bytes;
    for (uint32_t b = 0; b < L.g; b++) {
        const uint8_t *blk = row + (uint64_t)(u * L.g + b) * blk_bytes;
        for (uint32_t c = 0; c < base_chunks; c++) {
            uint8_t *o = tile + ((uint64_t)(b * base_chunks + c) * lanes + lane) * 16u;
            for (int i = 0; i < 16; i++) o[i] = blk[qofs + 16 * c + i];
        }
        if (base_df) {
            uint8_t *o = tile + (uint64_t)lanes * L.qc * 16u + ((uint64_t)b * lanes + lane) * 2u;
            o[0] = blk[dofs];
            o[1] = blk[dofs + 1];
        }
    }
}

__global__ void k_q8(const float *__restrict__ x, uint32_t k, uint32_t b, int8_t *__restrict__ q,
                     float *__restrict__ d, int32_t *__restrict__ sum) {
    uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t seg = gid >> 5, j = gid & 31u, nb = k / 32;
    bool ok = seg < nb * b;
    uint32_t bi = ok ? seg / nb : 0, blk = ok ? seg % nb : 0;
    float v = ok ? x[(uint64_t)(blk * 32 + j) * b + bi] : 0.0f;
    // all 32 lanes of a segment share `ok`; out-of-range segments only shuffle
    q8_block32(v, (int)j, q + (uint64_t)bi * k + blk * 32, d + (uint64_t)bi * nb + blk, sum + (uint64_t)bi * nb + blk, ok);
}

// N(0,1) fill: counter-based SplitMix64 and Box-Muller.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__global__ void k_kv_fill(float *kc, float *vc, uint32_t nlh, uint32_t n_ctx, uint32_t dh, uint32_t n, uint64_t seed) {
    const uint64_t per = (uint64_t)n * dh, total = (uint64_t)nlh * per;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (uint64_t)gridDim.x * blockDim.x) {
        uint64_t lh = i / per, r = i % per;
        uint64_t dst = lh * (uint64_t)n_ctx * dh + r;
        uint64_t z = mix64(seed ^ mix64(i));
        float u1 = ((float)(z >> 40) + 0.5f) * (1.0f / 16777216.0f);
        float u2 = (float)((z >> 16) & 0xFFFFFFu) * (1.0f / 16777216.0f);
        float rad = sqrtf(-2.0f * logf(u1));
        kc[dst] = rad * cospif(2.0f * u2);
        vc[dst] = rad * sinpif(2.0f * u2);
    }
}

}  // namespace

hipError_t pi_launch_repack(const uint8_t *src, uint8_t *dst, const pi_layout &L, hipStream_t s) {
    uint32_t bb = (uint32_t)pi_type_block_bytes(L.type);
    uint32_t qofs = (L.type == PI_TYPE_Q4_0 || L.type == PI_TYPE_Q8_0) ? 2u : 0u;
    uint32_t dofs = (L.type == PI_TYPE_Q6_K) ? 208u : 0u;
    uint64_t units = (uint64_t)L.rows * L.upr;
    uint64_t rb = (uint64_t)(L.k / pi_base_elems(L.type)) * bb;
    uint32_t blocks = (uint32_t)((units + 255) / 256);
    hipLaunchKernelGGL(k_repack, dim3(blocks), dim3(256), 0, s, src, dst, L, rb, bb, qofs, dofs,
                       pi_base_chunks(L.type), pi_base_dfields(L.type));
    return hipGetLastError();
}

hipError_t pi_launch_q8(const float *x, uint32_t k, uint32_t b, int8_t *q, float *d, int32_t *sum, hipStream_t s) {
    uint64_t threads = (uint64_t)(k / 32) * b * 32;
    uint32_t blocks = (uint32_t)((threads + 255) / 256);
    hipLaunchKernelGGL(k_q8, dim3(blocks), dim3(256), 0, s, x, k, b, q, d, sum);
    return hipGetLastError();
}

hipError_t pi_launch_kv_fill(float *kc, float *vc, uint32_t nlh, uint32_t n_ctx, uint32_t dh, uint32_t n, uint64_t seed,
                             hipStream_t s) {
    hipLaunchKernelGGL(k_kv_fill, dim3(4096), dim3(256), 0, s, kc, vc, nlh, n_ctx, dh, n, seed);
    return hipGetLastError();
}
