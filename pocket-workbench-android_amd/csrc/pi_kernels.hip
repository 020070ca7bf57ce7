// gfx950 kernels of the pocketinfer decode backend.
//
// Numerics: built with -ffp-contract=off, so a*b+c is two rounded operations
// as in the reference (Rust never contracts).  Division and sqrt are the
// correctly rounded HIP defaults.  Integer block sums use v_dot4_i32_i8 and
// are exact; every float term of a GEMV is formed with the operation order of
// quant_int.rs and summed per row in the reference's block order, so GEMV
// outputs are bit-identical to the CPU lanes path for the same Q8 input.
#include <hip/hip_runtime.h>

#include "pi_detmath.h"
#include "pi_kernels.h"

namespace {

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }
__device__ __forceinline__ float h2f(uint32_t bits) { return pi_f16_to_f32((uint16_t)(bits & 0xFFFFu)); }
__device__ __forceinline__ int comp(const int4 &v, int i) { return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w)); }
__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xFFu; }

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

// ---------------------------------------------------------------------------
// Q8 quantization of one 32-element block by 32 lanes (quant_int.rs:33-55).
// amax is an exact max; d = amax/127 and inv = 1/d are correctly rounded;
// roundf is half away from zero; NaN products map to 0 like Rust's `as i32`.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void q8_block32(float v, int j, int8_t *qout, float *dout, int32_t *sout,
                                           bool store = true) {
    float a = (v == v) ? fabsf(v) : 0.0f;
#pragma unroll
    for (int off = 16; off; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 32));
    float dd = a / 127.0f;
    float inv = dd > 0.0f ? 1.0f / dd : 0.0f;
    float r = roundf(v * inv);
    if (r < -127.0f) r = -127.0f;
    if (r > 127.0f) r = 127.0f;
    int iv = (r != r) ? 0 : (int)r;
    if (store) qout[j] = (int8_t)iv;
    int s = iv;
#pragma unroll
    for (int off = 16; off; off >>= 1) s += __shfl_xor(s, off, 32);
    if (store && j == 0) {
        *dout = dd;
        *sout = s;
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

// ---------------------------------------------------------------------------
// GEMV over the tiled layout.  One wavefront per tile, four per block; the
// kernel is persistent over tiles so each lane loads its activation slice
// once.  Terms go to LDS and the row's first lane sums them in block order.
// ---------------------------------------------------------------------------
template <uint32_t T> struct QT;
template <> struct QT<PI_TYPE_Q4_K> { static constexpr int BE = 256, BC = 9, DF = 0, TPB = 8; };
template <> struct QT<PI_TYPE_Q6_K> { static constexpr int BE = 256, BC = 13, DF = 1, TPB = 16; };
template <> struct QT<PI_TYPE_Q4_0> { static constexpr int BE = 32, BC = 1, DF = 1, TPB = 1; };
template <> struct QT<PI_TYPE_Q8_0> { static constexpr int BE = 32, BC = 2, DF = 1, TPB = 1; };

// Q4_K base block (quant_int.rs:330-371): c[0] = d, dmin, scales; c[1..8] = qs.
__device__ __forceinline__ void terms_q4k(const int4 *c, const int4 *a, const float *ad, const int *as,
                                          float *term, int *isum) {
    float d = h2f((uint32_t)c[0].x), dmin = h2f((uint32_t)c[0].x >> 16);
    uint32_t S[3] = {(uint32_t)c[0].y, (uint32_t)c[0].z, (uint32_t)c[0].w};
#pragma unroll
    for (int sb = 0; sb < 8; sb++) isum[sb] = 0;
#pragma unroll
    for (int g = 0; g < 4; g++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int4 w = c[1 + 2 * g + h];
#pragma unroll
            for (int m = 0; m < 4; m++) {
                uint32_t wm = (uint32_t)comp(w, m);
                int lo = (int)(wm & 0x0F0F0F0Fu), hi = (int)((wm >> 4) & 0x0F0F0F0Fu);
                isum[2 * g] = sdot4(lo, comp(a[4 * g + h], m), isum[2 * g]);
                isum[2 * g + 1] = sdot4(hi, comp(a[4 * g + 2 + h], m), isum[2 * g + 1]);
            }
        }
#pragma unroll
    for (int sb = 0; sb < 8; sb++) {
        uint32_t s, m;  // get_scale_min_k4 (quant_int.rs:245-252)
        if (sb < 4) {
            s = byte_of(S[sb / 4], sb % 4) & 63u;
            m = byte_of(S[(sb + 4) / 4], (sb + 4) % 4) & 63u;
        } else {
            uint32_t b8 = byte_of(S[(sb + 4) / 4], (sb + 4) % 4);
            s = (b8 & 0xFu) | ((byte_of(S[(sb - 4) / 4], (sb - 4) % 4) >> 6) << 4);
            m = (b8 >> 4) | ((byte_of(S[sb / 4], sb % 4) >> 6) << 4);
        }
        term[sb] = d * ad[sb] * (float)s * (float)isum[sb] - ad[sb] * dmin * (float)m * (float)as[sb];
    }
}

// Q6_K base block (quant_int.rs:373-419): c[0..7] = ql, c[8..11] = qh,
// c[12] = scales; terms in the visiting order (half, g, s).
__device__ __forceinline__ void terms_q6k(const int4 *c, uint32_t dbits, const int4 *a, const float *ad,
                                          const int *asum16, float *term, int *isum) {
    float d = h2f(dbits);
    int acc[16];
#pragma unroll
    for (int t = 0; t < 16; t++) acc[t] = 0;
#pragma unroll
    for (int half = 0; half < 2; half++)
#pragma unroll
        for (int m = 0; m < 8; m++) {
            uint32_t qa = (uint32_t)comp(c[half * 4 + m / 4], m % 4);
            uint32_t qb = (uint32_t)comp(c[half * 4 + 2 + m / 4], m % 4);
            uint32_t qh = (uint32_t)comp(c[8 + half * 2 + m / 4], m % 4);
            int v0 = (int)((qa & 0x0F0F0F0Fu) | ((qh & 0x03030303u) << 4));
            int v1 = (int)((qb & 0x0F0F0F0Fu) | (((qh >> 2) & 0x03030303u) << 4));
            int v2 = (int)(((qa >> 4) & 0x0F0F0F0Fu) | (((qh >> 4) & 0x03030303u) << 4));
            int v3 = (int)(((qb >> 4) & 0x0F0F0F0Fu) | (((qh >> 6) & 0x03030303u) << 4));
            int g = m / 4, base = half * 8 + g * 4;
            acc[base + 0] = sdot4(v0, comp(a[8 * half + 0 + m / 4], m % 4), acc[base + 0]);
            acc[base + 1] = sdot4(v1, comp(a[8 * half + 2 + m / 4], m % 4), acc[base + 1]);
            acc[base + 2] = sdot4(v2, comp(a[8 * half + 4 + m / 4], m % 4), acc[base + 2]);
            acc[base + 3] = sdot4(v3, comp(a[8 * half + 6 + m / 4], m % 4), acc[base + 3]);
        }
    const uint32_t SC[4] = {(uint32_t)c[12].x, (uint32_t)c[12].y, (uint32_t)c[12].z, (uint32_t)c[12].w};
#pragma unroll
    for (int half = 0; half < 2; half++)
#pragma unroll
        for (int g = 0; g < 2; g++)
#pragma unroll
            for (int s = 0; s < 4; s++) {
                int t = half * 8 + g * 4 + s;
                int idx = half * 8 + g + 2 * s;
                float scale = (float)(int8_t)byte_of(SC[idx / 4], idx % 4);
                isum[t] = acc[t] - 32 * asum16[t];
                term[t] = d * scale * ad[4 * half + s] * (float)isum[t];
            }
}

// Q4_0 base block (quant_int.rs:303-328): lo nibbles -> 0..15, hi -> 16..31.
__device__ __forceinline__ void terms_q40(const int4 &c, uint32_t dbits, const int4 *a, float ad, int as,
                                          float *term, int *isum) {
    int s = 0;
#pragma unroll
    for (int m = 0; m < 4; m++) {
        uint32_t w = (uint32_t)comp(c, m);
        s = sdot4((int)(w & 0x0F0F0F0Fu), comp(a[0], m), s);
        s = sdot4((int)((w >> 4) & 0x0F0F0F0Fu), comp(a[1], m), s);
    }
    *isum = s;
    float d = h2f(dbits);
    *term = d * ad * ((float)s - 8.0f * (float)as);
}

// Q8_0 base block (quant_int.rs:282-301).
__device__ __forceinline__ void terms_q80(const int4 &c0, const int4 &c1, uint32_t dbits, const int4 *a, float ad,
                                          float *term, int *isum) {
    int s = 0;
#pragma unroll
    for (int m = 0; m < 4; m++) {
        s = sdot4(comp(c0, m), comp(a[0], m), s);
        s = sdot4(comp(c1, m), comp(a[1], m), s);
    }
    *isum = s;
    float d = h2f(dbits);
    *term = d * ad * (float)s;
}

// NMAT = 1: one matrix (the standalone GEMV).  NMAT = 3: up to three matrices
// of one type and row length sharing the activation (Q/K/V, gate/up); their
// tiles are numbered back to back, S.tile0[m] being the first tile of m.
template <uint32_t T, int G, int MODE, int NMAT>
__global__ __launch_bounds__(256) void k_gemv(pi_gemv_set S, pi_layout L, const int8_t *__restrict__ aq,
                                              const float *__restrict__ adv, const int32_t *__restrict__ asv,
                                              int32_t *__restrict__ sums) {
    constexpr int BE = QT<T>::BE, BC = QT<T>::BC, DF = QT<T>::DF, TPB = QT<T>::TPB;
    constexpr int TPU = TPB * G;          // terms per unit
    constexpr int QC = BC * G;            // chunks per unit
    constexpr int AI4 = BE * G / 16;      // int4 of activation per unit
    constexpr int NQ8 = BE * G / 32;      // Q8 blocks per unit
    __shared__ float lds[4][TPU][64];

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const uint32_t upr = L.upr;
    const uint32_t u = (uint32_t)lane % upr;
    const bool lane_ok = (uint32_t)lane < L.lpt;

    int4 a[AI4];
    float ad[NQ8];
    int as[NQ8];
    int asum16[T == PI_TYPE_Q6_K ? 16 : 1];
    if (lane_ok) {
        const int4 *ap = reinterpret_cast<const int4 *>(aq + (uint64_t)u * BE * G);
#pragma unroll
        for (int i = 0; i < AI4; i++) a[i] = ap[i];
#pragma unroll
        for (int i = 0; i < NQ8; i++) {
            ad[i] = adv[u * NQ8 + i];
            as[i] = asv[u * NQ8 + i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < AI4; i++) a[i] = make_int4(0, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < NQ8; i++) { ad[i] = 0.0f; as[i] = 0; }
    }
    if constexpr (T == PI_TYPE_Q6_K) {
        // sums of the activation over each 16-element group, (half, g, s) order
#pragma unroll
        for (int half = 0; half < 2; half++)
#pragma unroll
            for (int g = 0; g < 2; g++)
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    int acc = 0;
                    const int4 &v = a[8 * half + 2 * s + g];
#pragma unroll
                    for (int m = 0; m < 4; m++) acc = sdot4(0x01010101, comp(v, m), acc);
                    asum16[half * 8 + g * 4 + s] = acc;
                }
    }

    for (uint32_t tbase = blockIdx.x * 4u; tbase < L.ntiles; tbase += gridDim.x * 4u) {
        const uint32_t gtile = tbase + (uint32_t)wave;
        const bool active = gtile < L.ntiles;
        uint32_t m = 0;
        if constexpr (NMAT > 1) m = (gtile >= S.tile0[1]) + (gtile >= S.tile0[2]);
        const uint32_t tile = gtile - S.tile0[m];
        const uint32_t rows = S.rows[m];
        uint32_t lanes = 0;
        if (active) lanes = (gtile == S.tile0[m + 1] - 1) ? (rows - tile * L.rpw) * upr : L.lpt;
        if (active && (uint32_t)lane < lanes) {
            const uint8_t *tb = S.w[m] + (uint64_t)tile * L.tile_bytes;
            int4 c[QC];
#pragma unroll
            for (int j = 0; j < QC; j++)
                c[j] = *reinterpret_cast<const int4 *>(tb + ((uint64_t)j * lanes + (uint32_t)lane) * 16u);
            uint32_t dbits[DF ? G : 1];
            if constexpr (DF) {
                const uint16_t *dp = reinterpret_cast<const uint16_t *>(tb + (uint64_t)lanes * QC * 16u);
#pragma unroll
                for (int b = 0; b < G; b++) dbits[b] = dp[(uint64_t)b * lanes + (uint32_t)lane];
            }
            float term[TPU];
            int isum[TPU];
#pragma unroll
            for (int b = 0; b < G; b++) {
                if constexpr (T == PI_TYPE_Q4_K)
                    terms_q4k(c + 9 * b, a + 16 * b, ad + 8 * b, as + 8 * b, term + 8 * b, isum + 8 * b);
                else if constexpr (T == PI_TYPE_Q6_K)
                    terms_q6k(c + 13 * b, dbits[b], a + 16 * b, ad + 8 * b, asum16, term + 16 * b, isum + 16 * b);
                else if constexpr (T == PI_TYPE_Q4_0)
                    terms_q40(c[b], dbits[b], a + 2 * b, ad[b], as[b], term + b, isum + b);
                else
                    terms_q80(c[2 * b], c[2 * b + 1], dbits[b], a + 2 * b, ad[b], term + b, isum + b);
            }
            if constexpr (MODE == PI_GEMV_SUMS) {
                const uint32_t row = tile * L.rpw + (uint32_t)lane / upr;
                const uint64_t per_row = (uint64_t)upr * TPU;
                int32_t *dst = sums + row * per_row + (uint64_t)u * TPU;
#pragma unroll
                for (int t = 0; t < TPU; t++) dst[t] = isum[t];
            } else {
#pragma unroll
                for (int t = 0; t < TPU; t++) lds[wave][t][lane] = term[t];
            }
        }
        if constexpr (MODE != PI_GEMV_SUMS) {
            __syncthreads();
            if (active && (uint32_t)lane < L.rpw) {
                const uint32_t row = tile * L.rpw + (uint32_t)lane;
                if (row < rows) {
                    float acc = 0.0f;
                    for (uint32_t uu = 0; uu < upr; uu++) {
                        const uint32_t src = (uint32_t)lane * upr + uu;
#pragma unroll
                        for (int t = 0; t < TPU; t++) acc += lds[wave][t][src];
                    }
                    const float o = 0.0f + acc;  // Pool::matmul zeroes out, lanes add acc
                    float *y = S.y[m];
                    if constexpr (MODE == PI_GEMV_OUT) y[row] = o;
                    else y[row] = y[row] + o;  // x[i] += proj[i] (model.rs:1095-1097)
                }
            }
            __syncthreads();
        }
    }
}

// ---------------------------------------------------------------------------
// RMSNorm + Q8 (model.rs:777-823 then quant_int.rs:17-56), one block.
// NEON = true is the batch-1 order of the aarch64 build: f32_sum_sq
// (simd.rs:45-64), eight FMA chains over stride-8 elements, lane-wise
// a0 + a1, then (t0 + t1) + (t2 + t3) and a scalar tail.  NEON = false is the
// scalar loop used for batches of more than one token.  The chains run in
// lanes 0..7 of the first wavefront.
// ---------------------------------------------------------------------------
template <bool NEON>
__global__ __launch_bounds__(256) void k_rmsnorm_q8(const float *__restrict__ x, const float *__restrict__ w,
                                                    uint32_t ne, float eps, float *__restrict__ out,
                                                    int8_t *__restrict__ q, float *__restrict__ d,
                                                    int32_t *__restrict__ sum) {
    extern __shared__ float sm[];  // ne floats + 16
    float *nx = sm, *red = sm + ne;
    for (uint32_t i = threadIdx.x; i < ne; i += blockDim.x) nx[i] = x[i];
    __syncthreads();
    if constexpr (NEON) {
        if (threadIdx.x < 8) {
            const uint32_t j = threadIdx.x, nfull = ne / 8;
            float acc = 0.0f;
#pragma unroll 8
            for (uint32_t i = 0; i < nfull; i++) {
                const float v = nx[8 * i + j];
                acc = __builtin_fmaf(v, v, acc);
            }
            red[j] = acc;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float t0 = red[0] + red[4], t1 = red[1] + red[5], t2 = red[2] + red[6], t3 = red[3] + red[7];
            float ss = (t0 + t1) + (t2 + t3);
            for (uint32_t i = ne / 8 * 8; i < ne; i++) ss += nx[i] * nx[i];
            red[8] = 1.0f / sqrtf(ss / (float)ne + eps);
        }
    } else {
        if (threadIdx.x == 0) {
            float ss = 0.0f;
#pragma unroll 8
            for (uint32_t i = 0; i < ne; i++) ss += nx[i] * nx[i];
            red[8] = 1.0f / sqrtf(ss / (float)ne + eps);
        }
    }
    __syncthreads();
    const float s = red[8];
    for (uint32_t i = threadIdx.x; i < ne; i += blockDim.x) {
        float v = nx[i] * s * w[i];
        nx[i] = v;
        if (out) out[i] = v;
    }
    __syncthreads();
    const uint32_t nb = ne / 32, seg0 = threadIdx.x >> 5, j = threadIdx.x & 31u, nseg = blockDim.x >> 5;
    for (uint32_t blk = seg0; blk < nb; blk += nseg) q8_block32(nx[blk * 32 + j], (int)j, q + blk * 32, d + blk, sum + blk);
}

// SwiGLU (model.rs:1111-1115) + Q8: one 32-element block per 32 lanes.
__global__ __launch_bounds__(256) void k_swiglu_q8(const float *__restrict__ gate, const float *__restrict__ up,
                                                   uint32_t n, int8_t *__restrict__ q, float *__restrict__ d,
                                                   int32_t *__restrict__ sum) {
    uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t blk = gid >> 5, j = gid & 31u;
    if (blk >= n / 32) return;  // whole 32-lane segments exit together
    float g = gate[blk * 32 + j];
    float sgl = g / (1.0f + pi_expf(-g));
    float v = sgl * up[blk * 32 + j];
    q8_block32(v, (int)j, q + blk * 32, d + blk, sum + blk);
}

// ---------------------------------------------------------------------------
// Embedding: dequant_row of one token (quant.rs:102-359 formulas).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_embed(const uint8_t *__restrict__ E, uint32_t type, uint32_t ne,
                                               uint64_t row_bytes, const pi_state *__restrict__ st,
                                               float *__restrict__ x) {
    const uint8_t *row = E + (uint64_t)st->tok * row_bytes;
    for (uint32_t e = blockIdx.x * blockDim.x + threadIdx.x; e < ne; e += gridDim.x * blockDim.x) {
        float v = 0.0f;
        if (type == PI_TYPE_F32) {
            memcpy(&v, row + 4 * (uint64_t)e, 4);
        } else if (type == PI_TYPE_Q4_K) {
            const uint8_t *b = row + (uint64_t)(e / 256) * 144;
            uint32_t j = e % 256, g = j / 64, hi = (j % 64) >= 32, l = j % 32, is = 2 * g + hi;
            float dd = h2f((uint32_t)b[0] | ((uint32_t)b[1] << 8)), dm = h2f((uint32_t)b[2] | ((uint32_t)b[3] << 8));
            const uint8_t *sc = b + 4;
            uint32_t s, m;
            if (is < 4) { s = sc[is] & 63u; m = sc[is + 4] & 63u; }
            else { s = (sc[is + 4] & 0xFu) | ((sc[is - 4] >> 6) << 4); m = (sc[is + 4] >> 4) | ((sc[is] >> 6) << 4); }
            uint32_t qv = hi ? (b[16 + g * 32 + l] >> 4) : (b[16 + g * 32 + l] & 0xFu);
            float d1 = dd * (float)s, m1 = dm * (float)m;
            v = d1 * (float)qv - m1;
        } else if (type == PI_TYPE_Q6_K) {
            const uint8_t *b = row + (uint64_t)(e / 256) * 210;
            uint32_t j = e % 256, half = j / 128, r = j % 128, s4 = r / 32, l = r % 32;
            uint32_t qlv = b[half * 64 + l + (s4 & 1u) * 32];
            qlv = (s4 >= 2) ? (qlv >> 4) : (qlv & 0xFu);
            uint32_t qhv = (b[128 + half * 32 + l] >> (2 * s4)) & 3u;
            int qq = (int)(qlv | (qhv << 4)) - 32;
            float dd = h2f((uint32_t)b[208] | ((uint32_t)b[209] << 8));
            float scv = (float)(int8_t)b[192 + half * 8 + l / 16 + 2 * s4];
            v = dd * scv * (float)qq;
        } else if (type == PI_TYPE_Q4_0) {
            const uint8_t *b = row + (uint64_t)(e / 32) * 18;
            uint32_t j = e % 32;
            uint32_t qv = j < 16 ? (b[2 + j] & 0xFu) : (b[2 + j - 16] >> 4);
            v = ((float)qv - 8.0f) * h2f((uint32_t)b[0] | ((uint32_t)b[1] << 8));
        } else if (type == PI_TYPE_Q8_0) {
            const uint8_t *b = row + (uint64_t)(e / 32) * 34;
            v = (float)(int8_t)b[2 + e % 32] * h2f((uint32_t)b[0] | ((uint32_t)b[1] << 8));
        }
        x[e] = v;
    }
}

// ---------------------------------------------------------------------------
// RoPE on q and k (adjacent pairs, cached cos/sin) and KV write.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_rope_kv(float *__restrict__ q, const float *__restrict__ k,
                                                 const float *__restrict__ v, const float *__restrict__ ct,
                                                 const float *__restrict__ stb, const pi_state *__restrict__ st,
                                                 float *__restrict__ kc, float *__restrict__ vc, uint32_t n_head,
                                                 uint32_t n_kv, uint32_t dh, uint32_t half, uint32_t n_ctx) {
    const uint32_t pos = (uint32_t)st->pos;
    const float *cb = ct + (uint64_t)pos * half, *sb = stb + (uint64_t)pos * half;
    const uint32_t npair = dh / 2;
    const uint32_t nq = n_head * npair, nk = n_kv * npair;
    for (uint32_t t = blockIdx.x * blockDim.x + threadIdx.x; t < nq + nk; t += gridDim.x * blockDim.x) {
        if (t < nq) {
            uint32_t h = t / npair, i = t % npair;
            if (i < half) {
                uint32_t i0 = h * dh + 2 * i;
                float x0 = q[i0], x1 = q[i0 + 1];
                q[i0] = x0 * cb[i] - x1 * sb[i];
                q[i0 + 1] = x0 * sb[i] + x1 * cb[i];
            }
        } else {
            uint32_t tt = t - nq, h = tt / npair, i = tt % npair;
            uint32_t i0 = h * dh + 2 * i;
            float x0 = k[i0], x1 = k[i0 + 1];
            if (i < half) {
                float r0 = x0 * cb[i] - x1 * sb[i];
                float r1 = x0 * sb[i] + x1 * cb[i];
                x0 = r0;
                x1 = r1;
            }
            uint64_t base = ((uint64_t)h * n_ctx + pos) * dh + 2 * i;
            kc[base] = x0;
            kc[base + 1] = x1;
            vc[base] = v[i0];
            vc[base + 1] = v[i0 + 1];
        }
    }
}

// ---------------------------------------------------------------------------
// Attention (model.rs:993-1087) in the aarch64 order.
// Part 1, parallel over positions: one wavefront per (head, 64 positions)
// stages the key rows in LDS (rows padded to 65 floats, so a lane reading its
// own row hits distinct banks) and each lane forms one score.  NEON = true
// is f32_dot (simd.rs:17-43): two 4-lane product accumulators over steps of
// 8, s = vaddvq(acc0), s += vaddvq(acc1); NEON = false the scalar loop of
// batches of more than one token.  s *= 1/sqrt(head_dim).
// ---------------------------------------------------------------------------
template <bool NEON>
__global__ __launch_bounds__(64) void k_attn_scores(const float *__restrict__ q, const float *__restrict__ kc,
                                                    const pi_state *__restrict__ st, uint32_t group, uint32_t n_ctx,
                                                    float scale, float *__restrict__ scores) {
    constexpr uint32_t DH = 64;
    const uint32_t h = blockIdx.x, c = blockIdx.y, lane = threadIdx.x;
    const int pos = st->pos;
    const int p0 = (int)c * 64;
    if (p0 > pos) return;
    const int np = min(64, pos + 1 - p0);
    __shared__ float kt[64][DH + 1];
    __shared__ float qs[DH];
    qs[lane] = q[h * DH + lane];
    const float *kb = kc + ((uint64_t)(h / group) * n_ctx + (uint32_t)p0) * DH;
#pragma unroll
    for (int it = 0; it < 16; it++) {
        const int r = it * 4 + (int)(lane >> 4), col = (int)(lane & 15u) * 4;
        if (r < np) {
            const float4 v = *reinterpret_cast<const float4 *>(kb + (uint64_t)r * DH + col);
            kt[r][col] = v.x;
            kt[r][col + 1] = v.y;
            kt[r][col + 2] = v.z;
            kt[r][col + 3] = v.w;
        }
    }
    __syncthreads();
    if ((int)lane < np) {
        const float *kr = kt[lane];
        float s;
        if constexpr (NEON) {
            float a0[4] = {0.f, 0.f, 0.f, 0.f}, a1[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (uint32_t i = 0; i < DH; i += 8)
#pragma unroll
                for (uint32_t j = 0; j < 4; j++) {
                    a0[j] = a0[j] + qs[i + j] * kr[i + j];
                    a1[j] = a1[j] + qs[i + 4 + j] * kr[i + 4 + j];
                }
            s = (a0[0] + a0[1]) + (a0[2] + a0[3]);
            s += (a1[0] + a1[1]) + (a1[2] + a1[3]);
        } else {
            s = 0.0f;
#pragma unroll
            for (uint32_t dd = 0; dd < DH; dd++) s += qs[dd] * kr[dd];
        }
        scores[(uint64_t)h * n_ctx + (uint32_t)p0 + lane] = s * scale;
    }
}

// Part 2, one block per head: max (exact in any order), e_p = exp(s_p - max)
// in parallel (written over the scores), then two serial chains in the
// reference order: wavefront 1 sums e_p over positions, wavefront 0 (lane =
// dimension) accumulates o += e_p * v_p (f32_axpy, skipping e_p == 0).  The
// output o * (1/sum) is quantized as two Q8 blocks.
__global__ __launch_bounds__(256) void k_attn_softmax_v(float *__restrict__ scores, const float *__restrict__ vc,
                                                        const pi_state *__restrict__ st, uint32_t group,
                                                        uint32_t n_ctx, float *__restrict__ attn,
                                                        int8_t *__restrict__ q8, float *__restrict__ d8,
                                                        int32_t *__restrict__ s8) {
    constexpr uint32_t DH = 64;
    const uint32_t h = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const int n = st->pos + 1;
    float *E = scores + (uint64_t)h * n_ctx;
    __shared__ float red[8];
    float m = -INFINITY;
    for (int p = (int)tid; p < n; p += 256) m = fmaxf(m, E[p]);
#pragma unroll
    for (int off = 32; off; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int p = (int)tid; p < n; p += 256) E[p] = pi_expf(E[p] - m);
    __syncthreads();
    const float *vb = vc + (uint64_t)(h / group) * n_ctx * DH;
    float acc = 0.0f;
    if (wave == 0) {
#pragma unroll 8
        for (int p = 0; p < n; p++) {
            const float ep = E[p];
            const float v = vb[(uint64_t)p * DH + lane];
            acc = (ep != 0.0f) ? acc + ep * v : acc;
        }
    } else if (wave == 1 && lane == 0) {
        float sum = 0.0f;
#pragma unroll 8
        for (int p = 0; p < n; p++) sum += E[p];
        red[4] = sum > 0.0f ? 1.0f / sum : 0.0f;
    }
    __syncthreads();
    if (wave == 0) {
        const float o = acc * red[4];
        attn[h * DH + lane] = o;
        const uint32_t blk = h * 2 + lane / 32;
        q8_block32(o, (int)(lane % 32), q8 + blk * 32, d8 + blk, s8 + blk);
    }
}


// ---------------------------------------------------------------------------
// Greedy argmax: candidate (v, i) beats (bv, bi) iff v > bv, or v == bv and
// i < bi (first max wins; NaN never wins), as sampler.rs:26-36.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void amax_merge(float &bv, uint32_t &bi, float v, uint32_t i) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

__global__ __launch_bounds__(256) void k_argmax_partial(const float *__restrict__ x, uint32_t n,
                                                        float *__restrict__ pv, uint32_t *__restrict__ pi) {
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) amax_merge(bv, bi, x[i], i);
#pragma unroll
    for (int off = 32; off; off >>= 1) {
        float ov = __shfl_xor(bv, off, 64);
        uint32_t oi = __shfl_xor(bi, off, 64);
        amax_merge(bv, bi, ov, oi);
    }
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) amax_merge(bv, bi, sv[w], si[w]);
        pv[blockIdx.x] = bv;
        pi[blockIdx.x] = bi;
    }
}

__global__ __launch_bounds__(256) void k_argmax_final(const float *__restrict__ pv, const uint32_t *__restrict__ pidx,
                                                      uint32_t np, pi_state *__restrict__ st,
                                                      uint32_t *__restrict__ ids) {
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (uint32_t i = threadIdx.x; i < np; i += blockDim.x) amax_merge(bv, bi, pv[i], pidx[i]);
#pragma unroll
    for (int off = 32; off; off >>= 1) {
        float ov = __shfl_xor(bv, off, 64);
        uint32_t oi = __shfl_xor(bi, off, 64);
        amax_merge(bv, bi, ov, oi);
    }
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) amax_merge(bv, bi, sv[w], si[w]);
        if (bi == 0xFFFFFFFFu) bi = 0;
        st->tok = bi;
        if (ids) ids[st->n_gen] = bi;
        st->n_gen += 1;
        st->pos += 1;
    }
}

__global__ void k_advance(pi_state *st, const uint32_t *prompt) {
    st->pos += 1;
    st->i += 1;
    st->tok = prompt[st->i];
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

template <uint32_t T, int G, int NMAT>
hipError_t launch_gemv_tg(const pi_gemv_set &S, const pi_layout &L, const int8_t *aq, const float *ad,
                          const int32_t *as, int32_t *sums, int mode, int max_blocks, hipStream_t s) {
    uint32_t blocks = (L.ntiles + 3) / 4;
    if (max_blocks > 0 && blocks > (uint32_t)max_blocks) blocks = (uint32_t)max_blocks;
    if (mode == PI_GEMV_OUT)
        hipLaunchKernelGGL((k_gemv<T, G, PI_GEMV_OUT, NMAT>), dim3(blocks), dim3(256), 0, s, S, L, aq, ad, as, sums);
    else if (mode == PI_GEMV_RESIDUAL)
        hipLaunchKernelGGL((k_gemv<T, G, PI_GEMV_RESIDUAL, NMAT>), dim3(blocks), dim3(256), 0, s, S, L, aq, ad, as, sums);
    else if constexpr (NMAT == 1)
        hipLaunchKernelGGL((k_gemv<T, G, PI_GEMV_SUMS, 1>), dim3(blocks), dim3(256), 0, s, S, L, aq, ad, as, sums);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

template <uint32_t T, int NMAT>
hipError_t launch_gemv_t(const pi_gemv_set &S, const pi_layout &L, const int8_t *aq, const float *ad,
                         const int32_t *as, int32_t *sums, int mode, int max_blocks, hipStream_t s) {
    if constexpr (T == PI_TYPE_Q4_K || T == PI_TYPE_Q6_K) {
        return L.g == 1 ? launch_gemv_tg<T, 1, NMAT>(S, L, aq, ad, as, sums, mode, max_blocks, s) : hipErrorInvalidValue;
    } else {
        switch (L.g) {
        case 1: return launch_gemv_tg<T, 1, NMAT>(S, L, aq, ad, as, sums, mode, max_blocks, s);
        case 2: return launch_gemv_tg<T, 2, NMAT>(S, L, aq, ad, as, sums, mode, max_blocks, s);
        case 3: return launch_gemv_tg<T, 3, NMAT>(S, L, aq, ad, as, sums, mode, max_blocks, s);
        case 4: return launch_gemv_tg<T, 4, NMAT>(S, L, aq, ad, as, sums, mode, max_blocks, s);
        case 6: return launch_gemv_tg<T, 6, NMAT>(S, L, aq, ad, as, sums, mode, max_blocks, s);
        case 8: return launch_gemv_tg<T, 8, NMAT>(S, L, aq, ad, as, sums, mode, max_blocks, s);
        default: return hipErrorInvalidValue;
        }
    }
}

template <int NMAT>
hipError_t launch_gemv_any(const pi_gemv_set &S, const pi_layout &L, const int8_t *aq, const float *ad,
                           const int32_t *as, int32_t *sums, int mode, int max_blocks, hipStream_t s) {
    switch (L.type) {
    case PI_TYPE_Q4_K: return launch_gemv_t<PI_TYPE_Q4_K, NMAT>(S, L, aq, ad, as, sums, mode, max_blocks, s);
    case PI_TYPE_Q6_K: return launch_gemv_t<PI_TYPE_Q6_K, NMAT>(S, L, aq, ad, as, sums, mode, max_blocks, s);
    case PI_TYPE_Q4_0: return launch_gemv_t<PI_TYPE_Q4_0, NMAT>(S, L, aq, ad, as, sums, mode, max_blocks, s);
    case PI_TYPE_Q8_0: return launch_gemv_t<PI_TYPE_Q8_0, NMAT>(S, L, aq, ad, as, sums, mode, max_blocks, s);
    default: return hipErrorInvalidValue;
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

hipError_t pi_launch_gemv(const uint8_t *w, const pi_layout &L, const int8_t *aq, const float *ad, const int32_t *as,
                          float *y, int32_t *sums, int mode, int max_blocks, hipStream_t s) {
    pi_gemv_set S{};
    S.w[0] = w;
    S.y[0] = y;
    S.rows[0] = L.rows;
    S.tile0[0] = 0;
    S.tile0[1] = S.tile0[2] = S.tile0[3] = L.ntiles;
    S.n = 1;
    return launch_gemv_any<1>(S, L, aq, ad, as, sums, mode, max_blocks, s);
}

hipError_t pi_launch_gemv_group(const pi_gemv_set &S, const pi_layout &L, const int8_t *aq, const float *ad,
                                const int32_t *as, int mode, int max_blocks, hipStream_t s) {
    if (mode == PI_GEMV_SUMS || S.n < 1 || S.n > 3) return hipErrorInvalidValue;
    pi_layout G = L;
    G.ntiles = S.tile0[3];
    return launch_gemv_any<3>(S, G, aq, ad, as, nullptr, mode, max_blocks, s);
}

hipError_t pi_launch_rmsnorm_q8(const float *x, const float *w, uint32_t ne, float eps, float *out, int8_t *q,
                                float *d, int32_t *sum, bool neon, hipStream_t s) {
    size_t shm = (size_t)ne * 4 + 64;
    if (neon)
        hipLaunchKernelGGL(k_rmsnorm_q8<true>, dim3(1), dim3(256), shm, s, x, w, ne, eps, out, q, d, sum);
    else
        hipLaunchKernelGGL(k_rmsnorm_q8<false>, dim3(1), dim3(256), shm, s, x, w, ne, eps, out, q, d, sum);
    return hipGetLastError();
}

hipError_t pi_launch_swiglu_q8(const float *gate, const float *up, uint32_t n, int8_t *q, float *d, int32_t *sum,
                               hipStream_t s) {
    uint32_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(k_swiglu_q8, dim3(blocks), dim3(256), 0, s, gate, up, n, q, d, sum);
    return hipGetLastError();
}

hipError_t pi_launch_embed(const uint8_t *E, uint32_t type, uint32_t ne, uint64_t row_bytes, const pi_state *st, float *x,
                           hipStream_t s) {
    uint32_t blocks = (ne + 255) / 256;
    hipLaunchKernelGGL(k_embed, dim3(blocks), dim3(256), 0, s, E, type, ne, row_bytes, st, x);
    return hipGetLastError();
}

hipError_t pi_launch_rope_kv(float *q, const float *k, const float *v, const float *ct, const float *stb,
                             const pi_state *st, float *kc, float *vc, uint32_t n_head, uint32_t n_kv, uint32_t dh,
                             uint32_t half, uint32_t n_ctx, hipStream_t s) {
    uint32_t work = (n_head + n_kv) * (dh / 2);
    uint32_t blocks = (work + 255) / 256;
    hipLaunchKernelGGL(k_rope_kv, dim3(blocks), dim3(256), 0, s, q, k, v, ct, stb, st, kc, vc, n_head, n_kv, dh, half, n_ctx);
    return hipGetLastError();
}

hipError_t pi_launch_attention(const float *q, const float *kc, const float *vc, const pi_state *st, uint32_t n_head,
                               uint32_t n_kv, uint32_t dh, uint32_t n_ctx, float scale, float *scores, uint32_t nchunk,
                               float *attn_out, int8_t *q8, float *d8, int32_t *s8, bool neon, hipStream_t s) {
    if (dh != 64) return hipErrorInvalidValue;
    const uint32_t group = n_head / n_kv;
    if (neon)
        hipLaunchKernelGGL(k_attn_scores<true>, dim3(n_head, nchunk), dim3(64), 0, s, q, kc, st, group, n_ctx, scale,
                           scores);
    else
        hipLaunchKernelGGL(k_attn_scores<false>, dim3(n_head, nchunk), dim3(64), 0, s, q, kc, st, group, n_ctx, scale,
                           scores);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_attn_softmax_v, dim3(n_head), dim3(256), 0, s, scores, vc, st, group, n_ctx, attn_out, q8, d8, s8);
    return hipGetLastError();
}

hipError_t pi_launch_argmax(const float *logits, uint32_t n, float *pv, uint32_t *pidx, pi_state *st, uint32_t *ids,
                            hipStream_t s) {
    hipLaunchKernelGGL(k_argmax_partial, dim3(PI_ARGMAX_BLOCKS), dim3(256), 0, s, logits, n, pv, pidx);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, s, pv, pidx, PI_ARGMAX_BLOCKS, st, ids);
    return hipGetLastError();
}

hipError_t pi_launch_advance(pi_state *st, const uint32_t *prompt, hipStream_t s) {
    hipLaunchKernelGGL(k_advance, dim3(1), dim3(1), 0, s, st, prompt);
    return hipGetLastError();
}

hipError_t pi_launch_kv_fill(float *kc, float *vc, uint32_t nlh, uint32_t n_ctx, uint32_t dh, uint32_t n, uint64_t seed,
                             hipStream_t s) {
    hipLaunchKernelGGL(k_kv_fill, dim3(4096), dim3(256), 0, s, kc, vc, nlh, n_ctx, dh, n, seed);
    return hipGetLastError();
}
