// Device-side core of the quantized GEMVs (gfx950), shared by the standalone
// GEMV and the fused decode kernels.
//
// Work split: a wavefront owns whole tiles of the lane-interleaved layout
// (pi_common.h): lane l of a tile holds unit l % upr of row l / upr, i.e. G
// consecutive base blocks of one row.  Each lane keeps the matching slice of
// the Q8 activation in registers for the whole kernel, loads its unit with
// 16-byte loads (one contiguous span per load instruction across the wave),
// forms the per-sub-block terms exactly as quant_int.rs does, and writes them
// to a wave-private LDS strip.  One lane per row then sums the row's terms
// strictly left to right, which is the float order of the reference's lanes
// path (acc += term over blocks and sub-blocks, then out = 0 + acc,
// quant_int.rs:330-419 and model.rs:241-321).  Integer sums use v_dot4_i32_i8
// and are exact.  No block-wide barrier is used inside the tile loop; the next
// tile's weights are loaded before the current one is consumed.
#pragma once

#include <hip/hip_runtime.h>

#include "pi_common.h"
#include "pi_detmath.h"

namespace pig {

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }
__device__ __forceinline__ float h2f(uint32_t bits) { return pi_f16_to_f32((uint16_t)(bits & 0xFFFFu)); }
__device__ __forceinline__ int comp(const int4 &v, int i) { return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w)); }
__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xFFu; }
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// Base-block geometry per type: elements, 16-byte chunks in the Q plane,
// f16 fields in the D plane, float terms per block.
template <uint32_t T> struct QT;
template <> struct QT<PI_TYPE_Q4_K> { static constexpr int BE = 256, BC = 9, DF = 0, TPB = 8; };
template <> struct QT<PI_TYPE_Q6_K> { static constexpr int BE = 256, BC = 13, DF = 1, TPB = 16; };
template <> struct QT<PI_TYPE_Q4_0> { static constexpr int BE = 32, BC = 1, DF = 1, TPB = 1; };
template <> struct QT<PI_TYPE_Q8_0> { static constexpr int BE = 32, BC = 2, DF = 1, TPB = 1; };

// ---------------------------------------------------------------------------
// Q8 quantization of one 32-element block held by one lane (quant_int.rs:33-55):
// amax ignores NaN; d = amax/127 and inv = 1/d correctly rounded; roundf is
// half away from zero; the clamp keeps NaN and `as i32` maps NaN to 0.
// Writes 8 packed words of quants, d and the block sum.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void q8_lane(const float (&v)[32], uint32_t *qw, float *dout, int32_t *sout) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) {
        const float a = fabsf(v[j]);
        if (a > amax) amax = a;
    }
    const float dd = amax / 127.0f;
    const float inv = dd > 0.0f ? 1.0f / dd : 0.0f;
    int s = 0;
#pragma unroll
    for (int w = 0; w < 8; w++) {
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            float r = roundf(v[4 * w + b] * inv);
            if (r < -127.0f) r = -127.0f;
            if (r > 127.0f) r = 127.0f;
            const int iv = (r != r) ? 0 : (int)r;
            s += iv;
            word |= ((uint32_t)iv & 0xFFu) << (8 * b);
        }
        qw[w] = word;
    }
    *dout = dd;
    *sout = s;
}

// The same rule for a block spread over 32 consecutive lanes (lane j of the
// half-wave holds element j); used where the values already live in lanes.
__device__ __forceinline__ void q8_block32(float v, int j, int8_t *qout, float *dout, int32_t *sout, bool store) {
    float a = (v == v) ? fabsf(v) : 0.0f;
#pragma unroll
    for (int off = 16; off; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 32));
    const float dd = a / 127.0f;
    const float inv = dd > 0.0f ? 1.0f / dd : 0.0f;
    float r = roundf(v * inv);
    if (r < -127.0f) r = -127.0f;
    if (r > 127.0f) r = 127.0f;
    const int iv = (r != r) ? 0 : (int)r;
    if (store) qout[j] = (int8_t)iv;
    int s = iv;
#pragma unroll
    for (int off = 16; off; off >>= 1) s += __shfl_xor(s, off, 32);
    if (store && j == 0) {
        *dout = dd;
        *sout = s;
    }
}

// ---------------------------------------------------------------------------
// Activation slice of one unit (G base blocks) in registers.
// ---------------------------------------------------------------------------
template <uint32_t T, int G> struct Slice {
    static constexpr int BE = QT<T>::BE;
    static constexpr int AI4 = BE * G / 16;  // int4 of quants
    static constexpr int NQ8 = BE * G / 32;  // Q8 blocks
    int4 a[AI4];
    float ad[NQ8];
    int as[NQ8];
    int asum16[T == PI_TYPE_Q6_K ? 16 : 1];  // Q6_K: 16-element sums, (half, g, s) order

    // q, d, s: Q8 activation of a whole row (k quants); u: unit index.
    __device__ __forceinline__ void load(const int8_t *q, const float *d, const int32_t *s, uint32_t u) {
        const int4 *ap = reinterpret_cast<const int4 *>(q + (uint64_t)u * BE * G);
#pragma unroll
        for (int i = 0; i < AI4; i++) a[i] = ap[i];
#pragma unroll
        for (int i = 0; i < NQ8; i++) {
            ad[i] = d[u * NQ8 + i];
            as[i] = s[u * NQ8 + i];
        }
        if constexpr (T == PI_TYPE_Q6_K) {
#pragma unroll
            for (int half = 0; half < 2; half++)
#pragma unroll
                for (int g = 0; g < 2; g++)
#pragma unroll
                    for (int ss = 0; ss < 4; ss++) {
                        int acc = 0;
                        const int4 &v = a[8 * half + 2 * ss + g];
#pragma unroll
                        for (int m = 0; m < 4; m++) acc = sdot4(0x01010101, comp(v, m), acc);
                        asum16[half * 8 + g * 4 + ss] = acc;
                    }
        }
    }
};

// ---------------------------------------------------------------------------
// Weights of one unit.
// ---------------------------------------------------------------------------
template <uint32_t T, int G> struct Unit {
    static constexpr int QC = QT<T>::BC * G;
    static constexpr int ND = QT<T>::DF ? G : 1;
    int4 c[QC];
    uint32_t db[ND];

    // tb: tile base; lanes: units in this tile; l: this lane's unit (< lanes).
    __device__ __forceinline__ void load(const uint8_t *tb, uint32_t lanes, uint32_t l) {
#pragma unroll
        for (int j = 0; j < QC; j++)
            c[j] = *reinterpret_cast<const int4 *>(tb + ((uint64_t)j * lanes + l) * 16u);
        if constexpr (QT<T>::DF) {
            const uint16_t *dp = reinterpret_cast<const uint16_t *>(tb + (uint64_t)lanes * QC * 16u);
#pragma unroll
            for (int b = 0; b < G; b++) db[b] = dp[(uint64_t)b * lanes + l];
        }
    }
};

// Q4_K block (quant_int.rs:330-371): c[0] = d, dmin, scales; c[1..8] = qs.
// term[sb] = ((d*da)*s)*isum - ((da*dmin)*m)*asum for sub-blocks sb = 0..7.
__device__ __forceinline__ void terms_q4k(const int4 *c, const int4 *a, const float *ad, const int *as, float *term,
                                          int *isum) {
    const float d = h2f((uint32_t)c[0].x), dmin = h2f((uint32_t)c[0].x >> 16);
    const uint32_t S[3] = {(uint32_t)c[0].y, (uint32_t)c[0].z, (uint32_t)c[0].w};
#pragma unroll
    for (int sb = 0; sb < 8; sb++) isum[sb] = 0;
#pragma unroll
    for (int g = 0; g < 4; g++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int4 w = c[1 + 2 * g + h];
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const uint32_t wm = (uint32_t)comp(w, m);
                const int lo = (int)(wm & 0x0F0F0F0Fu), hi = (int)((wm >> 4) & 0x0F0F0F0Fu);
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
            const uint32_t b8 = byte_of(S[(sb + 4) / 4], (sb + 4) % 4);
            s = (b8 & 0xFu) | ((byte_of(S[(sb - 4) / 4], (sb - 4) % 4) >> 6) << 4);
            m = (b8 >> 4) | ((byte_of(S[sb / 4], sb % 4) >> 6) << 4);
        }
        term[sb] = d * ad[sb] * (float)s * (float)isum[sb] - ad[sb] * dmin * (float)m * (float)as[sb];
    }
}

// Q6_K block (quant_int.rs:373-419): c[0..7] = ql, c[8..11] = qh, c[12] =
// scales; 16-element sums in the visiting order (half, g, s);
// term = ((d*scale)*da)*isum.
__device__ __forceinline__ void terms_q6k(const int4 *c, uint32_t dbits, const int4 *a, const float *ad,
                                          const int *asum16, float *term, int *isum) {
    const float d = h2f(dbits);
    int acc[16];
#pragma unroll
    for (int t = 0; t < 16; t++) acc[t] = 0;
#pragma unroll
    for (int half = 0; half < 2; half++)
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const uint32_t qa = (uint32_t)comp(c[half * 4 + m / 4], m % 4);
            const uint32_t qb = (uint32_t)comp(c[half * 4 + 2 + m / 4], m % 4);
            const uint32_t qh = (uint32_t)comp(c[8 + half * 2 + m / 4], m % 4);
            const int v0 = (int)((qa & 0x0F0F0F0Fu) | ((qh & 0x03030303u) << 4));
            const int v1 = (int)((qb & 0x0F0F0F0Fu) | (((qh >> 2) & 0x03030303u) << 4));
            const int v2 = (int)(((qa >> 4) & 0x0F0F0F0Fu) | (((qh >> 4) & 0x03030303u) << 4));
            const int v3 = (int)(((qb >> 4) & 0x0F0F0F0Fu) | (((qh >> 6) & 0x03030303u) << 4));
            const int g = m / 4, base = half * 8 + g * 4;
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
                const int t = half * 8 + g * 4 + s;
                const int idx = half * 8 + g + 2 * s;
                const float scale = (float)(int8_t)byte_of(SC[idx / 4], idx % 4);
                isum[t] = acc[t] - 32 * asum16[t];
                term[t] = d * scale * ad[4 * half + s] * (float)isum[t];
            }
}

// Q4_0 block (quant_int.rs:303-328): lo nibbles -> 0..15, hi -> 16..31;
// term = (d*da)*(isum - 8*asum).
__device__ __forceinline__ void terms_q40(const int4 &c, uint32_t dbits, const int4 *a, float ad, int as, float *term,
                                          int *isum) {
    int s = 0;
#pragma unroll
    for (int m = 0; m < 4; m++) {
        const uint32_t w = (uint32_t)comp(c, m);
        s = sdot4((int)(w & 0x0F0F0F0Fu), comp(a[0], m), s);
        s = sdot4((int)((w >> 4) & 0x0F0F0F0Fu), comp(a[1], m), s);
    }
    *isum = s;
    *term = h2f(dbits) * ad * ((float)s - 8.0f * (float)as);
}

// Q8_0 block (quant_int.rs:282-301): term = (d*da)*isum.
__device__ __forceinline__ void terms_q80(const int4 &c0, const int4 &c1, uint32_t dbits, const int4 *a, float ad,
                                          float *term, int *isum) {
    int s = 0;
#pragma unroll
    for (int m = 0; m < 4; m++) {
        s = sdot4(comp(c0, m), comp(a[0], m), s);
        s = sdot4(comp(c1, m), comp(a[1], m), s);
    }
    *isum = s;
    *term = h2f(dbits) * ad * (float)s;
}

template <uint32_t T, int G>
__device__ __forceinline__ void unit_terms(const Unit<T, G> &U, const Slice<T, G> &A, float *term, int *isum) {
#pragma unroll
    for (int b = 0; b < G; b++) {
        if constexpr (T == PI_TYPE_Q4_K)
            terms_q4k(U.c + 9 * b, A.a + 16 * b, A.ad + 8 * b, A.as + 8 * b, term + 8 * b, isum + 8 * b);
        else if constexpr (T == PI_TYPE_Q6_K)
            terms_q6k(U.c + 13 * b, U.db[b], A.a + 16 * b, A.ad + 8 * b, A.asum16, term + 16 * b, isum + 16 * b);
        else if constexpr (T == PI_TYPE_Q4_0)
            terms_q40(U.c[b], U.db[b], A.a + 2 * b, A.ad[b], A.as[b], term + b, isum + b);
        else
            terms_q80(U.c[2 * b], U.c[2 * b + 1], U.db[b], A.a + 2 * b, A.ad[b], term + b, isum + b);
    }
}

// ---------------------------------------------------------------------------
// Matrices of one type and layout that share an activation, tiles numbered
// back to back (tile0[m] = first tile of matrix m, tile0[n] = total).
// ---------------------------------------------------------------------------
struct MatSet {
    const uint8_t *w[3];
    float *y[3];
    uint32_t rows[3];
    uint32_t tile0[4];
    uint32_t n;
    uint32_t upr, rpw, lpt;
    uint64_t tile_bytes;
};

struct TileRef {
    const uint8_t *base;
    uint32_t m, tile, lanes, row0, nrows;
};

__device__ __forceinline__ TileRef tile_ref(const MatSet &S, uint32_t gt) {
    TileRef r;
    uint32_t m = 0;
    if (S.n > 1 && gt >= S.tile0[1]) m = 1;
    if (S.n > 2 && gt >= S.tile0[2]) m = 2;
    r.m = m;
    r.tile = gt - S.tile0[m];
    r.row0 = r.tile * S.rpw;
    const bool last = gt == S.tile0[m + 1] - 1;
    r.nrows = last ? S.rows[m] - r.row0 : S.rpw;
    r.lanes = last ? r.nrows * S.upr : S.lpt;
    r.base = S.w[m] + (uint64_t)r.tile * S.tile_bytes;
    return r;
}

// Sums n terms of the strip at p strictly left to right, starting from 0.
__device__ __forceinline__ float chain_sum(const float *p, uint32_t n) {
    float acc = 0.0f;
    if ((n & 3u) == 0) {
        const float4 *p4 = reinterpret_cast<const float4 *>(p);
        for (uint32_t i = 0; i < n / 4; i++) {
            const float4 v = p4[i];
            acc += v.x;
            acc += v.y;
            acc += v.z;
            acc += v.w;
        }
    } else {
        for (uint32_t i = 0; i < n; i++) acc += p[i];
    }
    return acc;
}

// Runs the tiles gt = first, first + stride, ... of S on one wavefront.
// strip: this wave's LDS strip of 64 * TPU floats.  For every finished row,
// the lane owning it calls out(m, row, value) with value = 0 + sum of terms.
// Weights of the next tile are requested before the current tile is used
// (two named buffers, so both stay in registers).
template <uint32_t T, int G, typename Out>
__device__ __forceinline__ void consume_tile(const MatSet &S, const Slice<T, G> &A, const Unit<T, G> &U,
                                             const TileRef &R, float *strip, Out &out) {
    constexpr int TPU = QT<T>::TPB * G;
    const uint32_t lane = threadIdx.x & 63u;
    float term[TPU];
    int isum[TPU];
    unit_terms<T, G>(U, A, term, isum);
    if (lane < R.lanes) {
#pragma unroll
        for (int t = 0; t < TPU; t++) strip[lane * TPU + t] = term[t];
    }
    wave_sync();
    const uint32_t per_row = S.upr * TPU;
    if (lane < R.nrows) out(R.m, R.row0 + lane, 0.0f + chain_sum(strip + lane * per_row, per_row));
    wave_sync();
}

template <uint32_t T, int G, typename Out>
__device__ __forceinline__ void run_tiles(const MatSet &S, const Slice<T, G> &A, uint32_t first, uint32_t stride,
                                          float *strip, Out out) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t nt = S.tile0[S.n];
    if (first >= nt) return;
    Unit<T, G> UA, UB;
    TileRef RA = tile_ref(S, first), RB;
    UA.load(RA.base, RA.lanes, min(lane, RA.lanes - 1));
    uint32_t gt = first;
    for (;;) {
        uint32_t gn = gt + stride;
        bool more = gn < nt;
        // always issue the next load (the current tile again when there is none)
        RB = tile_ref(S, more ? gn : gt);
        UB.load(RB.base, RB.lanes, min(lane, RB.lanes - 1));
        consume_tile<T, G>(S, A, UA, RA, strip, out);
        if (!more) break;
        gt = gn;
        gn = gt + stride;
        more = gn < nt;
        RA = tile_ref(S, more ? gn : gt);
        UA.load(RA.base, RA.lanes, min(lane, RA.lanes - 1));
        consume_tile<T, G>(S, A, UB, RB, strip, out);
        if (!more) break;
        gt = gn;
    }
}

// Integer block sums of the tiles (test hook): per 32 elements, or per 16 for
// Q6_K, written row-major.
template <uint32_t T, int G>
__device__ __forceinline__ void run_tiles_sums(const MatSet &S, const Slice<T, G> &A, uint32_t first,
                                               uint32_t stride, int32_t *sums) {
    constexpr int TPU = QT<T>::TPB * G;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t nt = S.tile0[S.n];
    for (uint32_t gt = first; gt < nt; gt += stride) {
        const TileRef R = tile_ref(S, gt);
        Unit<T, G> U;
        U.load(R.base, R.lanes, min(lane, R.lanes - 1));
        float term[TPU];
        int isum[TPU];
        unit_terms<T, G>(U, A, term, isum);
        if (lane < R.lanes) {
            const uint32_t row = R.row0 + lane / S.upr, u = lane % S.upr;
            int32_t *dst = sums + (uint64_t)row * S.upr * TPU + (uint64_t)u * TPU;
#pragma unroll
            for (int t = 0; t < TPU; t++) dst[t] = isum[t];
        }
    }
}

}  // namespace pig
