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

// N(0,1) fill of positions [0, n) of every (layer, kv head): pi_kv_normal.
__global__ void k_kv_fill(float *kc, float *vc, uint32_t nlh, uint32_t n_ctx, uint32_t dh, uint32_t n, uint64_t seed) {
    const uint64_t per = (uint64_t)n * dh, total = (uint64_t)nlh * per;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t lh = (uint32_t)(i / per), r = (uint32_t)(i % per);
        const uint32_t p = r / dh, d = r % dh;
        float k, v;
        pi_kv_normal(seed, lh, p, d, &k, &v);
        const uint64_t dst = (uint64_t)lh * n_ctx * dh + r;
        kc[dst] = k;
        vc[dst] = v;
    }
}

// dst[i] = src[i] for n 16-byte words: a plain streaming copy (one read and
// one write of each byte) whose counter readings calibrate HBM traffic.
__global__ void k_copy16(const uint4 *__restrict__ src, uint4 *__restrict__ dst, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

}  // namespace

hipError_t pi_launch_copy16(const void *src, void *dst, uint64_t words, hipStream_t s) {
    if (!words) return hipSuccess;
    hipLaunchKernelGGL(k_copy16, dim3(8192), dim3(256), 0, s, (const uint4 *)src, (uint4 *)dst, words);
    return hipGetLastError();
}

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
