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

// Global-memory views of generic pointers.  Pointers read from memory (rather
// than passed as kernel arguments) are generic to the compiler, which then
// emits flat loads; a flat load counts on both the vector-memory and the LDS
// wait counters, so any later LDS access waits for every outstanding weight
// load.  Casting to the global address space gives global loads.
// (The host pass of a HIP compile also parses device functions; it never runs
// them and has no address spaces, so the qualifier is applied only when
// compiling for the device.)
#if defined(__HIP_DEVICE_COMPILE__)
#define PI_GLOBAL __attribute__((address_space(1)))
#define PI_CONSTANT __attribute__((address_space(4)))
#else
#define PI_GLOBAL
#define PI_CONSTANT
#endif
template <typename T> __device__ __forceinline__ const PI_GLOBAL T *gld(const T *p) { return (const PI_GLOBAL T *)p; }
template <typename T> __device__ __forceinline__ PI_GLOBAL T *gst(T *p) { return (PI_GLOBAL T *)p; }
// Copy of a descriptor that no thread writes during the kernel, read through
// the constant address space so the fields come in with scalar loads.
template <typename T> __device__ __forceinline__ T cload(const T *p) {
    return *(const PI_CONSTANT T *)p;
}

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }
// f16 bits (low half) -> f32 with v_cvt_f32_f16: exact for every finite and
// infinite value (f16 denormals are kept); a signalling NaN comes back quiet,
// which no term can tell apart, since every use multiplies it.
__device__ __forceinline__ float h2f(uint32_t bits) {
    const unsigned short b = (unsigned short)(bits & 0xFFFFu);
    _Float16 h;
    __builtin_memcpy(&h, &b, sizeof h);
    return (float)h;
}
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
// Lane exchanges through DPP moves (a VALU operand modifier, no LDS round
// trip).  Every lane that is read must be active.
// ---------------------------------------------------------------------------
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within each 8
constexpr int kDppMirror = 0x140;      // lane i <-> 15 - i within each row of 16
constexpr int kDppBcast15 = 0x142;     // lane 15 of row r -> row r + 1
constexpr int kDppBcast31 = 0x143;     // lane 31 -> rows 2 and 3
template <int CTRL, int ROWS = 0xF> __device__ __forceinline__ int dpp(int v) {
    return __builtin_amdgcn_update_dpp(v, v, CTRL, ROWS, 0xF, false);
}
template <int CTRL, int ROWS = 0xF> __device__ __forceinline__ uint32_t dpp(uint32_t v) {
    return (uint32_t)dpp<CTRL, ROWS>((int)v);
}
template <int CTRL, int ROWS = 0xF> __device__ __forceinline__ float dpp(float v) {
    return __int_as_float(dpp<CTRL, ROWS>(__float_as_int(v)));
}
// op over each row of 16 lanes, in every lane of the row (op commutative and
// associative on the values it sees, e.g. max or integer add).
template <typename T, typename Op> __device__ __forceinline__ T row16_allreduce(T v, Op op) {
    v = op(v, dpp<kDppXor1>(v));
    v = op(v, dpp<kDppXor2>(v));
    v = op(v, dpp<kDppHalfMirror>(v));
    v = op(v, dpp<kDppMirror>(v));
    return v;
}
// ... over each group of 32 lanes (ds_swizzle xor 16 for the last step).
template <typename T, typename Op> __device__ __forceinline__ T half32_allreduce(T v, Op op) {
    v = row16_allreduce(v, op);
    int o;
    if constexpr (sizeof(T) == 4) {
        int b;
        __builtin_memcpy(&b, &v, 4);
        o = __builtin_amdgcn_ds_swizzle(b, 0x401F);   // bit mode: and 0x1F, xor 0x10
        T t;
        __builtin_memcpy(&t, &o, 4);
        v = op(v, t);
    }
    return v;
}
// DPP move whose lanes outside ROWS receive `old`.
template <int CTRL, int ROWS> __device__ __forceinline__ float dpp_or(float old, float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROWS, 0xF, false));
}
template <int CTRL, int ROWS> __device__ __forceinline__ uint32_t dpp_or(uint32_t old, uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROWS, 0xF, false);
}
// Maximum over the whole wavefront (every lane active), returned in every
// lane: rows of 16 first, then lane 63 collects the rows through row
// broadcasts and is read as a scalar.
__device__ __forceinline__ float wave_max(float v) {
    auto mx = [](float x, float y) { return fmaxf(x, y); };
    v = row16_allreduce(v, mx);
    v = fmaxf(v, dpp_or<kDppBcast15, 0xA>(v, v));
    v = fmaxf(v, dpp_or<kDppBcast31, 0xC>(v, v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// (value, index) with the larger value, the smaller index on equal values.
__device__ __forceinline__ void argmax_merge(float &bv, uint32_t &bi, float v, uint32_t i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}
template <int CTRL, int ROWS = 0xF> __device__ __forceinline__ void argmax_step(float &v, uint32_t &i) {
    const float ov = dpp_or<CTRL, ROWS>(v, v);
    const uint32_t oi = dpp_or<CTRL, ROWS>(i, i);
    argmax_merge(v, i, ov, oi);
}
// argmax_merge over the whole wavefront (every lane active); the result in
// every lane.  The merge picks one pair by a total order, so the grouping of
// the steps does not change the result.
__device__ __forceinline__ void wave_argmax(float &v, uint32_t &i) {
    argmax_step<kDppXor1>(v, i);
    argmax_step<kDppXor2>(v, i);
    argmax_step<kDppHalfMirror>(v, i);
    argmax_step<kDppMirror>(v, i);
    argmax_step<kDppBcast15, 0xA>(v, i);
    argmax_step<kDppBcast31, 0xC>(v, i);
    v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
    i = (uint32_t)__builtin_amdgcn_readlane((int)i, 63);
}

// clamp(round(y), -127, 127) with round half away from zero, NaN -> 0
// (quant_int.rs:49: (x * inv).round().clamp(-127.0, 127.0) as i32).
// round(y) == trunc(y + copysign(0.5 - 2^-25, y)) for every float |y| < 2^22
// (the sum rounds up past the next integer exactly when the fraction is at
// least one half); clamping the sum to +-127 before truncation gives the same
// clamp, and larger |y| only ever clamps.
__device__ __forceinline__ int q8_round_clamp(float y) {
    const float r = __builtin_amdgcn_fmed3f(y + __builtin_copysignf(0.49999997f, y), -127.0f, 127.0f);
    return (y != y) ? 0 : (int)r;
}

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
            const int iv = q8_round_clamp(v[4 * w + b] * inv);
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
// Returns this lane's quant; d and the block sum are returned in every lane.
__device__ __forceinline__ int q8_block32_core(float v, float &dd, int &sum) {
    float a = (v == v) ? fabsf(v) : 0.0f;
    a = half32_allreduce(a, [](float x, float y) { return fmaxf(x, y); });
    dd = a / 127.0f;
    const float inv = dd > 0.0f ? 1.0f / dd : 0.0f;
    const int iv = q8_round_clamp(v * inv);
    sum = half32_allreduce(iv, [](int x, int y) { return x + y; });
    return iv;
}
__device__ __forceinline__ void q8_block32(float v, int j, int8_t *qout, float *dout, int32_t *sout, bool store) {
    float dd;
    int s;
    const int iv = q8_block32_core(v, dd, s);
    if (store) qout[j] = (int8_t)iv;
    if (store && j == 0) {
        *dout = dd;
        *sout = s;
    }
}

// The same rule for a block held by two adjacent lanes of a wavefront, 16
// elements each (the even lane holds elements 0..15).  Both lanes of the
// pair must call it.  The maximum and the integer sum are exact in any order,
// so they are formed as trees and completed across the pair.  Returns this
// half's 4 quant words, and d and the block sum (in both lanes).
__device__ __forceinline__ void q8_pair_core(const float (&v)[16], uint32_t (&qw)[4], float &dd, int &sum) {
    float m[8];
#pragma unroll
    for (int j = 0; j < 8; j++) m[j] = fmaxf(fabsf(v[2 * j]), fabsf(v[2 * j + 1]));   // maxNum: NaN ignored
#pragma unroll
    for (int w = 4; w; w >>= 1)
#pragma unroll
        for (int j = 0; j < w; j++) m[j] = fmaxf(m[j], m[j + w]);
    float amax = fmaxf(m[0], dpp<kDppXor1>(m[0]));
    amax = fmaxf(amax, 0.0f);   // all-NaN block: 0
    dd = amax / 127.0f;
    const float inv = dd > 0.0f ? 1.0f / dd : 0.0f;
    int iv[16];
#pragma unroll
    for (int j = 0; j < 16; j++) iv[j] = q8_round_clamp(v[j] * inv);
#pragma unroll
    for (int w = 0; w < 4; w++)
        qw[w] = ((uint32_t)iv[4 * w] & 0xFFu) | (((uint32_t)iv[4 * w + 1] & 0xFFu) << 8) |
                (((uint32_t)iv[4 * w + 2] & 0xFFu) << 16) | (((uint32_t)iv[4 * w + 3] & 0xFFu) << 24);
    // block sum of the 16 quants (exact integer dot products with 1)
    int t = 0;
#pragma unroll
    for (int w = 0; w < 4; w++) t = sdot4((int)qw[w], 0x01010101, t);
    sum = t + dpp<kDppXor1>(t);
}
// Writes this half's 4 quant words to qw; the even lane writes d and the sum.
__device__ __forceinline__ void q8_pair(const float (&v)[16], uint32_t half, uint32_t *qw, float *dout,
                                        int32_t *sout) {
    uint32_t w4[4];
    float dd;
    int sum;
    q8_pair_core(v, w4, dd, sum);
#pragma unroll
    for (int w = 0; w < 4; w++) qw[w] = w4[w];
    if (half == 0) {
        *dout = dd;
        *sout = sum;
    }
}

// Calls eat(p[i]) for i = 0..n4-1 in order on a float4 row in LDS.  The
// reads of the next B float4 are in flight while the current B are used; two
// named buffers, reads at fixed offsets from one address.  p[n4 .. n4 + 2B)
// must be readable LDS (loaded and ignored).
template <int B, typename F>
__device__ __forceinline__ void lds_chain4(const float4 *p, uint32_t n4, F &&eat) {
    float4 a[B], b[B];
#pragma unroll
    for (int u = 0; u < B; u++) a[u] = p[u];
    uint32_t i = 0;
    for (; i + 2 * B <= n4; i += 2 * B) {
        const float4 *q = p + i;
#pragma unroll
        for (int u = 0; u < B; u++) b[u] = q[B + u];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < B; u++) eat(a[u]);
        __builtin_amdgcn_sched_barrier(0);   // a is dead before its registers are reloaded
#pragma unroll
        for (int u = 0; u < B; u++) a[u] = q[2 * B + u];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < B; u++) eat(b[u]);
        __builtin_amdgcn_sched_barrier(0);
    }
    // fewer than 2B left: a already holds p[i .. i + B)
    const uint32_t rem = n4 - i;
    if (rem) {
#pragma unroll
        for (int u = 0; u < B; u++) b[u] = p[i + B + u];
#pragma unroll
        for (int u = 0; u < B; u++)
            if ((uint32_t)u < rem) eat(a[u]);
#pragma unroll
        for (int u = 0; u < B; u++)
            if ((uint32_t)(B + u) < rem) eat(b[u]);
    }
}

// acc = fma(v, v, acc) over the row in order: one accumulator of
// simd::f32_sum_sq (simd.rs:45-64).
template <int B>
__device__ __forceinline__ float sumsq_fma_chain(const float4 *p, uint32_t n4) {
    float acc = 0.0f;
    lds_chain4<B>(p, n4, [&](const float4 &v) {
        acc = __builtin_fmaf(v.x, v.x, acc);
        acc = __builtin_fmaf(v.y, v.y, acc);
        acc = __builtin_fmaf(v.z, v.z, acc);
        acc = __builtin_fmaf(v.w, v.w, acc);
    });
    return acc;
}

// ss += v * v over the row in order, product rounded then added: the
// multi-token loop of model.rs:812-822.
template <int B>
__device__ __forceinline__ float sumsq_scalar_chain(const float4 *p, uint32_t n4) {
    float acc = 0.0f;
    lds_chain4<B>(p, n4, [&](const float4 &v) {
        acc += v.x * v.x;
        acc += v.y * v.y;
        acc += v.z * v.z;
        acc += v.w * v.w;
    });
    return acc;
}

// Position of 16-byte chunk k of a Q8 activation kept in LDS.  Within each
// 256-byte row r the chunks are permuted by c -> c ^ (r & 7), so lanes that
// read the same chunk of different rows (one unit each) hit different banks
// instead of all queueing on the same four.  With activation lengths that are
// multiples of 128, a final half row (8 chunks) maps onto itself.
__device__ __forceinline__ uint32_t act_chunk(uint32_t k) { return k ^ ((k >> 4) & 7u); }

// ---------------------------------------------------------------------------
// Activation slice of one unit (G base blocks) in registers.
// ---------------------------------------------------------------------------
template <uint32_t T, int G> struct Slice {
    static constexpr int BE = QT<T>::BE;
    static constexpr int AI4 = BE * G / 16;  // int4 of quants
    static constexpr int NQ8 = BE * G / 32;  // Q8 blocks
    int4 a[AI4];
    float ad[NQ8];
    float as[NQ8];   // block sums, converted once (exact: |sum| <= 4064)
    int asum16[T == PI_TYPE_Q6_K ? 16 : 1];  // Q6_K: 16-element sums, (half, g, s) order

    // q, d, s: Q8 activation of a whole row (k quants); u: unit index.
    __device__ __forceinline__ void load(const int8_t *q, const float *d, const int32_t *s, uint32_t u) {
        const int4 *ap = reinterpret_cast<const int4 *>(q + (uint64_t)u * BE * G);
#pragma unroll
        for (int i = 0; i < AI4; i++) a[i] = ap[i];
        load_scales(d, s, u);
    }
    // The same from an LDS activation whose quant chunks are in act_chunk order.
    __device__ __forceinline__ void load_swz(const int8_t *q, const float *d, const int32_t *s, uint32_t u) {
        const int4 *ap = reinterpret_cast<const int4 *>(q);
#pragma unroll
        for (int i = 0; i < AI4; i++) a[i] = ap[act_chunk(u * AI4 + (uint32_t)i)];
        load_scales(d, s, u);
    }
    __device__ __forceinline__ void load_scales(const float *d, const int32_t *s, uint32_t u) {
#pragma unroll
        for (int i = 0; i < NQ8; i++) {
            ad[i] = d[u * NQ8 + i];
            as[i] = (float)s[u * NQ8 + i];
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
    __device__ __forceinline__ void load(const uint8_t *tb, uint32_t lanes, uint32_t l) { load_part<0, QC>(tb, lanes, l); }
    // Chunks J0 .. J1-1 only (and the D plane with the last chunk), so a unit
    // can be requested in two parts.
    template <int J0, int J1> __device__ __forceinline__ void load_part(const uint8_t *tb, uint32_t lanes, uint32_t l) {
        // Weights are read once per token: non-temporal loads, so they do not
        // evict what is reused from the L2 (code, tagged words, activations).
        typedef int v4i __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int j = J0; j < J1; j++) {
            const v4i t = __builtin_nontemporal_load(gld(reinterpret_cast<const v4i *>(tb + ((uint64_t)j * lanes + l) * 16u)));
            c[j] = make_int4(t.x, t.y, t.z, t.w);
        }
        if constexpr (QT<T>::DF && J1 == QC) {
            const PI_GLOBAL uint16_t *dp = gld(reinterpret_cast<const uint16_t *>(tb + (uint64_t)lanes * QC * 16u));
#pragma unroll
            for (int b = 0; b < G; b++) db[b] = __builtin_nontemporal_load(dp + (uint64_t)b * lanes + l);
        }
    }
};

// Q4_K block (quant_int.rs:330-371): c[0] = d, dmin, scales; c[1..8] = qs.
// term[sb] = ((d*da)*s)*isum - ((da*dmin)*m)*asum for sub-blocks sb = 0..7.
__device__ __forceinline__ void terms_q4k(const int4 *c, const int4 *a, const float *ad, const float *as, float *term,
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
    // get_scale_min_k4 (quant_int.rs:245-252) for the 8 sub-blocks at once,
    // one 6-bit value per byte: scales 0-3 and mins 0-3 are the low 6 bits of
    // bytes 0-3 and 4-7; scale / min j >= 4 takes its low 4 bits from byte 8+j-4
    // (low / high nibble) and its top 2 bits from the top of byte j-4 / j.
    const uint32_t s03 = S[0] & 0x3F3F3F3Fu, m03 = S[1] & 0x3F3F3F3Fu;
    const uint32_t s47 = (S[2] & 0x0F0F0F0Fu) | ((S[0] >> 2) & 0x30303030u);
    const uint32_t m47 = ((S[2] >> 4) & 0x0F0F0F0Fu) | ((S[1] >> 2) & 0x30303030u);
#pragma unroll
    for (int sb = 0; sb < 8; sb++) {
        const float s = (float)byte_of(sb < 4 ? s03 : s47, sb % 4);
        const float m = (float)byte_of(sb < 4 ? m03 : m47, sb % 4);
        term[sb] = d * ad[sb] * s * (float)isum[sb] - ad[sb] * dmin * m * as[sb];
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
__device__ __forceinline__ void terms_q40(const int4 &c, uint32_t dbits, const int4 *a, float ad, float as, float *term,
                                          int *isum) {
    int s = 0;
#pragma unroll
    for (int m = 0; m < 4; m++) {
        const uint32_t w = (uint32_t)comp(c, m);
        s = sdot4((int)(w & 0x0F0F0F0Fu), comp(a[0], m), s);
        s = sdot4((int)((w >> 4) & 0x0F0F0F0Fu), comp(a[1], m), s);
    }
    *isum = s;
    *term = h2f(dbits) * ad * ((float)s - 8.0f * as);
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
// back to back (tile0[m] = first tile of matrix m; tile0[j] = total for
// every j >= n, so tile0[3] is always the total).
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

// A MatSet is read either from a value (kernel argument) or, through SetRef,
// from device memory with scalar loads at each use, so that persistent
// kernels keep no descriptor fields live in registers.
struct SetRef {
    const MatSet *p;
};
__device__ __forceinline__ uint32_t ms_n(const MatSet &S) { return S.n; }
__device__ __forceinline__ uint32_t ms_t0(const MatSet &S, int i) { return S.tile0[i]; }
__device__ __forceinline__ uint32_t ms_rows(const MatSet &S, int i) { return S.rows[i]; }
__device__ __forceinline__ const uint8_t *ms_w(const MatSet &S, int i) { return S.w[i]; }
__device__ __forceinline__ uint32_t ms_upr(const MatSet &S) { return S.upr; }
__device__ __forceinline__ uint32_t ms_rpw(const MatSet &S) { return S.rpw; }
__device__ __forceinline__ uint32_t ms_lpt(const MatSet &S) { return S.lpt; }
__device__ __forceinline__ uint64_t ms_tb(const MatSet &S) { return S.tile_bytes; }
__device__ __forceinline__ uint32_t ms_n(const SetRef &S) { return cload(&S.p->n); }
__device__ __forceinline__ uint32_t ms_t0(const SetRef &S, int i) { return cload(&S.p->tile0[i]); }
__device__ __forceinline__ uint32_t ms_rows(const SetRef &S, int i) { return cload(&S.p->rows[i]); }
__device__ __forceinline__ const uint8_t *ms_w(const SetRef &S, int i) { return cload(&S.p->w[i]); }
__device__ __forceinline__ uint32_t ms_upr(const SetRef &S) { return cload(&S.p->upr); }
__device__ __forceinline__ uint32_t ms_rpw(const SetRef &S) { return cload(&S.p->rpw); }
__device__ __forceinline__ uint32_t ms_lpt(const SetRef &S) { return cload(&S.p->lpt); }
__device__ __forceinline__ uint64_t ms_tb(const SetRef &S) { return cload(&S.p->tile_bytes); }
// total tiles (tile0[j] = total for every j >= n)
template <typename SS> __device__ __forceinline__ uint32_t ms_total(const SS &S) { return ms_t0(S, 3); }

// Tile reference of global tile gt.  A MatSet value (a kernel argument, in
// constant memory) is indexed with the matrix number; through a SetRef the
// fields are read with scalar loads and chosen with selects.
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

__device__ __forceinline__ TileRef tile_ref(const SetRef &S, uint32_t gt) {
    TileRef r;
    const uint32_t n = ms_n(S), t1_ = ms_t0(S, 1), t2_ = ms_t0(S, 2);
    const uint32_t m = (n > 2 && gt >= t2_) ? 2u : ((n > 1 && gt >= t1_) ? 1u : 0u);
    const uint32_t t0 = m == 0 ? ms_t0(S, 0) : (m == 1 ? t1_ : t2_);
    const uint32_t t1 = m == 0 ? t1_ : (m == 1 ? t2_ : ms_t0(S, 3));
    const uint32_t rows = m == 0 ? ms_rows(S, 0) : (m == 1 ? ms_rows(S, 1) : ms_rows(S, 2));
    const uint8_t *w = m == 0 ? ms_w(S, 0) : (m == 1 ? ms_w(S, 1) : ms_w(S, 2));
    const uint32_t rpw = ms_rpw(S);
    r.m = m;
    r.tile = gt - t0;
    r.row0 = r.tile * rpw;
    const bool last = gt == t1 - 1;
    r.nrows = last ? rows - r.row0 : rpw;
    r.lanes = last ? r.nrows * ms_upr(S) : ms_lpt(S);
    r.base = w + (uint64_t)r.tile * ms_tb(S);
    return r;
}

// Folds the n4 float4 at p (LDS) in order with f, B float4 per batch; the
// next batch is read before the current one is folded, so LDS latency is paid
// once per batch pair rather than once per read.
template <int B, typename F>
__device__ __forceinline__ void lds_fold4(const float4 *p, uint32_t n4, F &&f) {
    const uint32_t nb = n4 / B;
    if (nb) {
        float4 cur[B];
#pragma unroll
        for (int u = 0; u < B; u++) cur[u] = p[u];
        for (uint32_t k = 0; k < nb; k++) {
            float4 nxt[B];
            if (k + 1 < nb) {
#pragma unroll
                for (int u = 0; u < B; u++) nxt[u] = p[(k + 1) * B + u];
            }
#pragma unroll
            for (int u = 0; u < B; u++) f(cur[u]);
#pragma unroll
            for (int u = 0; u < B; u++) cur[u] = nxt[u];
        }
    }
    for (uint32_t i = nb * B; i < n4; i++) f(p[i]);
}

// float4 read ahead per step by the per-row term chains (a wavefront's term
// strip); the persistent kernel, at its register limit, uses fewer.
#ifndef PI_CHAIN_B
#define PI_CHAIN_B 9
#endif
// Floats readable after the end of every row a chain_sum reads (strips are
// followed by this much LDS).
constexpr uint32_t kChainPad = 8 * PI_CHAIN_B + 8;

// Sums n terms of the strip at p strictly left to right, starting from 0.
// The next float4 are read while the current ones are added (p[n .. n +
// 8 * PI_CHAIN_B) is read ahead and ignored).
__device__ __forceinline__ float chain_sum(const float *p, uint32_t n) {
    float acc = 0.0f;
    if ((n & 3u) == 0) {
        lds_chain4<PI_CHAIN_B>(reinterpret_cast<const float4 *>(p), n / 4, [&](const float4 &v) {
            acc += v.x;
            acc += v.y;
            acc += v.z;
            acc += v.w;
        });
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
// per_row: terms per row (units per row * TPU).
struct NoMarkG {
    __device__ void operator()(uint32_t) const {}
};
template <uint32_t T, int G, typename Out, typename Mark = NoMarkG>
__device__ __forceinline__ void consume_tile_pr(uint32_t per_row, const Slice<T, G> &A, const Unit<T, G> &U,
                                                const TileRef &R, float *strip, Out &out, Mark mark = Mark{}) {
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
    mark(30);
    if (lane < R.nrows) out(R.m, R.row0 + lane, 0.0f + chain_sum(strip + lane * per_row, per_row));
    wave_sync();
    mark(31);
}

template <uint32_t T, int G, typename SS, typename Out>
__device__ __forceinline__ void consume_tile(const SS &S, const Slice<T, G> &A, const Unit<T, G> &U,
                                             const TileRef &R, float *strip, Out &out) {
    consume_tile_pr<T, G>(ms_upr(S) * (QT<T>::TPB * G), A, U, R, strip, out);
}

// Runs the tiles gt = first, first + stride, ... of S on one wavefront, the
// first of them already loaded into UA (tile reference RA).
template <uint32_t T, int G, typename SS, typename Out>
__device__ __forceinline__ void run_tiles_pre(const SS &S, const Slice<T, G> &A, Unit<T, G> UA, TileRef RA,
                                              uint32_t first, uint32_t stride, float *strip, Out out) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t nt = ms_total(S);
    Unit<T, G> UB;
    TileRef RB;
    uint32_t gt = first;
    for (;;) {
        uint32_t gn = gt + stride;
        bool more = gn < nt;
        // always issue the next load (the current tile again when there is none)
        RB = tile_ref(S, more ? gn : gt);
        UB.load(RB.base, RB.lanes, min(lane, RB.lanes - 1));
        consume_tile<T, G, SS>(S, A, UA, RA, strip, out);
        if (!more) break;
        gt = gn;
        gn = gt + stride;
        more = gn < nt;
        RA = tile_ref(S, more ? gn : gt);
        UA.load(RA.base, RA.lanes, min(lane, RA.lanes - 1));
        consume_tile<T, G, SS>(S, A, UB, RB, strip, out);
        if (!more) break;
        gt = gn;
    }
}

template <uint32_t T, int G, typename SS, typename Out>
__device__ __forceinline__ void run_tiles(const SS &S, const Slice<T, G> &A, uint32_t first, uint32_t stride,
                                          float *strip, Out out) {
    const uint32_t lane = threadIdx.x & 63u;
    if (first >= ms_total(S)) return;
    Unit<T, G> UA;
    const TileRef RA = tile_ref(S, first);
    UA.load(RA.base, RA.lanes, min(lane, RA.lanes - 1));
    run_tiles_pre<T, G, SS>(S, A, UA, RA, first, stride, strip, out);
}

// Integer block sums of the tiles (test hook): per 32 elements, or per 16 for
// Q6_K, written row-major.
template <uint32_t T, int G>
__device__ __forceinline__ void run_tiles_sums(const MatSet &S, const Slice<T, G> &A, uint32_t first,
                                               uint32_t stride, int32_t *sums) {
    constexpr int TPU = QT<T>::TPB * G;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t nt = ms_total(S);
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

// One element of a token_embd row in its native layout (dequant_row,
// quant.rs:102-359, for the types with kernels).
__device__ __forceinline__ float embed_elem(const uint8_t *row, uint32_t type, uint32_t e) {
    float v = 0.0f;
    if (type == PI_TYPE_F32) {
        memcpy(&v, row + 4 * (uint64_t)e, 4);
    } else if (type == PI_TYPE_Q4_K) {
        const uint8_t *b = row + (uint64_t)(e / 256) * 144;
        const uint32_t j = e % 256, g = j / 64, hi = (j % 64) >= 32, l = j % 32, is = 2 * g + hi;
        const float dd = h2f((uint32_t)b[0] | ((uint32_t)b[1] << 8)), dm = h2f((uint32_t)b[2] | ((uint32_t)b[3] << 8));
        const uint8_t *sc = b + 4;
        uint32_t s, m;
        if (is < 4) {
            s = sc[is] & 63u;
            m = sc[is + 4] & 63u;
        } else {
            s = (sc[is + 4] & 0xFu) | ((sc[is - 4] >> 6) << 4);
            m = (sc[is + 4] >> 4) | ((sc[is] >> 6) << 4);
        }
        const uint32_t qv = hi ? (b[16 + g * 32 + l] >> 4) : (b[16 + g * 32 + l] & 0xFu);
        const float d1 = dd * (float)s, m1 = dm * (float)m;
        v = d1 * (float)qv - m1;
    } else if (type == PI_TYPE_Q6_K) {
        const uint8_t *b = row + (uint64_t)(e / 256) * 210;
        const uint32_t j = e % 256, hf = j / 128, r = j % 128, s4 = r / 32, l = r % 32;
        uint32_t qlv = b[hf * 64 + l + (s4 & 1u) * 32];
        qlv = (s4 >= 2) ? (qlv >> 4) : (qlv & 0xFu);
        const uint32_t qhv = (b[128 + hf * 32 + l] >> (2 * s4)) & 3u;
        const int qq = (int)(qlv | (qhv << 4)) - 32;
        const float dd = h2f((uint32_t)b[208] | ((uint32_t)b[209] << 8));
        const float scv = (float)(int8_t)b[192 + hf * 8 + l / 16 + 2 * s4];
        v = dd * scv * (float)qq;
    } else if (type == PI_TYPE_Q4_0) {
        const uint8_t *b = row + (uint64_t)(e / 32) * 18;
        const uint32_t j = e % 32;
        const uint32_t qv = j < 16 ? (b[2 + j] & 0xFu) : (b[2 + j - 16] >> 4);
        v = ((float)qv - 8.0f) * h2f((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    } else if (type == PI_TYPE_Q8_0) {
        const uint8_t *b = row + (uint64_t)(e / 32) * 34;
        v = (float)(int8_t)b[2 + e % 32] * h2f((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    }
    return v;
}

}  // namespace pig
