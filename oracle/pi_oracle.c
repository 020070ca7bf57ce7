/*
 * pi_oracle.c -- CPU oracle for the pocketinfer decode path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE: the checker that tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg compare the HIP
 * library against.  Nothing in the product links or calls this file.
 *
 * What it restates (reference paths relative to rust/pocketinfer/src/):
 *   - Q8Act::prepare                quant_int.rs:17-56 (bit-exact rule)
 *   - dp::* single-lane int8 dots   quant_int.rs:97-253
 *   - lanes::* multi-lane int8 dots quant_int.rs:271-419
 *   - dequant_row / dot_row_scalar / row_dot_multi   quant.rs:102-476
 *   - f16 <-> f32                   util.rs:76-138
 *   - Pool::matmul                  model.rs:139-350
 *   - KvCache / Scratch / rope      model.rs:352-461
 *   - Engine::rmsnorm, forward_inner, forward_layers  model.rs:777-1172
 *   - Engine::generate              model.rs:1235-1352
 *   - Rng / sample                  sampler.rs:1-92
 *
 * The oracle is the reference as built for aarch64, its only build with the
 * int8 matmul (quant_int.rs:64-80): at batch 1 RMSNorm uses f32_sum_sq
 * (two 4-lane FMA accumulators) and attention scores use f32_dot (two 4-lane
 * accumulators), both with the pairwise vaddvq reduction (simd.rs:17-64);
 * batches of more than one token use the scalar loops; attention values use
 * f32_axpy and skip zero weights (model.rs:1047-1075).  exp / pow / cos / sin
 * are the deterministic double-precision definitions of po_detmath.h, since
 * the reference's libm results are not pinned.  Compiled with
 * -ffp-contract=off: Rust evaluates a*b+c as two rounded operations unless it
 * calls an FMA explicitly (vfmaq_f32, fmaf here).
 */
#define _GNU_SOURCE
#include "pi_oracle.h"
#include "po_detmath.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#if defined(__x86_64__)
#include <immintrin.h>
#endif

#define MAX_BATCH 64

/* ------------------------------------------------------------------------ */
/* util.rs:76-100                                                            */
float po_f16_to_f32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u, exp = (h >> 10) & 0x1Fu, mant = h & 0x3FFu, bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else {
            uint32_t m = mant;
            int shifts = 0;
            while ((m & 0x400u) == 0) { m <<= 1; shifts++; }
            m &= 0x3FFu;
            bits = (sign << 31) | ((uint32_t)(113 - shifts) << 23) | (m << 13);
        }
    } else if (exp == 0x1F) {
        bits = (sign << 31) | (0xFFu << 23) | (mant << 13);
    } else {
        bits = (sign << 31) | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* util.rs:102-138 (round to nearest even) */
uint16_t po_f32_to_f16(float v) {
    uint32_t bits;
    memcpy(&bits, &v, 4);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    int32_t exp = (int32_t)((bits >> 23) & 0xFFu);
    uint32_t mant = bits & 0x7FFFFFu;
    if (exp == 0xFF) {
        uint16_t payload = mant ? (uint16_t)(0x200u | (mant >> 13)) : 0;
        return sign | 0x7C00u | payload;
    }
    int32_t e = exp - 127 + 15;
    if (e >= 0x1F) return sign | 0x7C00u;
    if (e <= 0) {
        if (e < -10) return sign;
        uint32_t m = mant | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint16_t half = (uint16_t)(m >> shift);
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half_bit = 1u << (shift - 1);
        if (rem > half_bit || (rem == half_bit && (half & 1u))) half++;
        return sign | half;
    }
    uint16_t half = (uint16_t)(((uint32_t)e << 10) | (mant >> 13));
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) {
        half++;
        if ((half & 0x7C00u) == 0x7C00u) return sign | 0x7C00u;
    }
    return sign | half;
}

static inline float f16_at(const uint8_t *p) { return po_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }
static inline float bf16_at(const uint8_t *p) {
    uint32_t b = (uint32_t)(p[0] | (p[1] << 8)) << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}
static inline float f32_at(const uint8_t *p) { float f; memcpy(&f, p, 4); return f; }
static inline uint32_t u32_at(const uint8_t *p) { uint32_t v; memcpy(&v, p, 4); return v; }

/* quant.rs:19-37 */
int po_type_block(uint32_t t, size_t *be, size_t *bb) {
    size_t e, b;
    switch (t) {
    case PO_F32: e = 1; b = 4; break;
    case PO_F16: case PO_BF16: e = 1; b = 2; break;
    case PO_Q4_0: e = 32; b = 18; break;
    case PO_Q4_1: e = 32; b = 20; break;
    case PO_Q5_0: e = 32; b = 22; break;
    case PO_Q5_1: e = 32; b = 24; break;
    case PO_Q8_0: e = 32; b = 34; break;
    case PO_Q8_1: e = 32; b = 36; break;
    case PO_Q2_K: e = 256; b = 84; break;
    case PO_Q3_K: e = 256; b = 110; break;
    case PO_Q4_K: e = 256; b = 144; break;
    case PO_Q5_K: e = 256; b = 176; break;
    case PO_Q6_K: e = 256; b = 210; break;
    case PO_Q8_K: e = 256; b = 292; break;
    default: return 0;
    }
    if (be) *be = e;
    if (bb) *bb = b;
    return 1;
}

/* quant.rs:60-72 */
int po_tensor_nbytes(uint32_t t, uint64_t ne0, uint64_t ne1, size_t *out) {
    size_t be, bb;
    if (!po_type_block(t, &be, &bb)) return -1;
    if (ne0 % be != 0) return -1;
    unsigned __int128 n = (unsigned __int128)ne0 * ne1;
    if (n >> 64) return -1;
    unsigned __int128 bytes = (n / be) * bb;
    if (bytes >> 63) return -1;
    *out = (size_t)bytes;
    return 0;
}

/* quant.rs:79-86 (also quant_int.rs:245-252) */
static inline void scale_min_k4(size_t j, const uint8_t *q, uint8_t *s, uint8_t *m) {
    if (j < 4) {
        *s = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *s = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* ------------------------------------------------------------------------ */
/* quant_int.rs:17-56 -- scalar rule; simd_q8.rs:8-51 is bit-identical.      */
void po_q8_prepare(const float *x, size_t k, size_t b, int8_t *q, float *d, int32_t *sum) {
    size_t nb = k / 32;
    for (size_t bi = 0; bi < b; bi++) {
        for (size_t blk = 0; blk < nb; blk++) {
            size_t base = blk * 32;
            float amax = 0.0f;
            for (size_t j = 0; j < 32; j++) {
                float v = fabsf(x[(base + j) * b + bi]);
                if (v > amax) amax = v;
            }
            float dd = amax / 127.0f;
            float inv = dd > 0.0f ? 1.0f / dd : 0.0f;
            int32_t s = 0;
            size_t qbase = bi * k + base;
            for (size_t j = 0; j < 32; j++) {
                /* f32::round is half away from zero; clamp keeps NaN, and
                 * `as i32` maps NaN to 0. */
                float r = roundf(x[(base + j) * b + bi] * inv);
                if (r < -127.0f) r = -127.0f;
                if (r > 127.0f) r = 127.0f;
                int32_t v = (r != r) ? 0 : (int32_t)r;
                q[qbase + j] = (int8_t)v;
                s += v;
            }
            d[bi * nb + blk] = dd;
            sum[bi * nb + blk] = s;
        }
    }
}

/* Integer dot of n int8 pairs (what vdotq_s32 + vaddvq_s32 compute). */
static inline int32_t idot(const int8_t *a, const int8_t *w, int n) {
    int32_t s = 0;
    for (int i = 0; i < n; i++) s += (int32_t)a[i] * (int32_t)w[i];
    return s;
}

/* Q6_K block -> we[8][32] int8 (quant_int.rs:383-395). */
static inline void unpack_q6k(const uint8_t *blk, int8_t we[8][32]) {
    for (int half = 0; half < 2; half++) {
        const uint8_t *qlb = blk + half * 64, *qhb = blk + 128 + half * 32;
        for (int i = 0; i < 32; i++) {
            uint8_t b0 = qlb[i], b1 = qlb[i + 32], hb = qhb[i];
            we[4 * half + 0][i] = (int8_t)((int)((b0 & 0xF) | ((hb & 3) << 4)) - 32);
            we[4 * half + 1][i] = (int8_t)((int)((b1 & 0xF) | (((hb >> 2) & 3) << 4)) - 32);
            we[4 * half + 2][i] = (int8_t)((int)(((b0 >> 4) & 0xF) | (((hb >> 4) & 3) << 4)) - 32);
            we[4 * half + 3][i] = (int8_t)((int)(((b1 >> 4) & 0xF) | (((hb >> 6) & 3) << 4)) - 32);
        }
    }
}

/* Q4_K block -> we[256] int8: low nibble of qs[g*32+i] is element 64g+i,
 * high nibble is element 64g+32+i (quant_int.rs:340-353). */
static inline void unpack_q4k(const uint8_t *blk, int8_t we[256]) {
    for (int g = 0; g < 4; g++) {
        const uint8_t *q = blk + 16 + g * 32;
        for (int i = 0; i < 32; i++) {
            we[2 * g * 32 + i] = (int8_t)(q[i] & 0x0F);
            we[(2 * g + 1) * 32 + i] = (int8_t)(q[i] >> 4);
        }
    }
}

/* quant_int.rs:82-253: dp::q8_0, dp::q4_0, dp::q4_k, dp::q6_k. */
float po_dot_row_q8(uint32_t t, const uint8_t *w, size_t k, const po_q8act *act, size_t lane) {
    float acc = 0.0f;
    switch (t) {
    case PO_Q8_0: {
        size_t nb = k / 32;
        for (size_t blk = 0; blk < nb; blk++) {
            const uint8_t *p = w + blk * 34;
            float d = f16_at(p);
            int32_t s = idot(act->q + lane * act->k + blk * 32, (const int8_t *)(p + 2), 32);
            acc += d * act->d[lane * nb + blk] * (float)s;
        }
        return acc;
    }
    case PO_Q4_0: {
        size_t nb = k / 32;
        for (size_t blk = 0; blk < nb; blk++) {
            const uint8_t *p = w + blk * 18;
            float d = f16_at(p);
            int8_t we[32];
            for (int i = 0; i < 16; i++) { we[i] = (int8_t)(p[2 + i] & 0xF); we[16 + i] = (int8_t)(p[2 + i] >> 4); }
            int32_t s = idot(act->q + lane * act->k + blk * 32, we, 32);
            float dq = act->d[lane * nb + blk];
            int32_t sq = act->sum[lane * nb + blk];
            acc += d * dq * ((float)s - 8.0f * (float)sq);
        }
        return acc;
    }
    case PO_Q4_K: {
        size_t nb = k / 256;
        for (size_t blk = 0; blk < nb; blk++) {
            const uint8_t *p = w + blk * 144;
            float d = f16_at(p), dmin = f16_at(p + 2);
            const uint8_t *scales = p + 4;
            int8_t we[256];
            unpack_q4k(p, we);
            size_t abl = lane * act->nb + blk * 8;
            const int8_t *a = act->q + lane * act->k + blk * 256;
            for (size_t g = 0; g < 4; g++) {
                uint8_t s1, m1, s2, m2;
                scale_min_k4(2 * g, scales, &s1, &m1);
                scale_min_k4(2 * g + 1, scales, &s2, &m2);
                float s_lo = (float)idot(a + g * 64, we + 2 * g * 32, 32);
                float s_hi = (float)idot(a + g * 64 + 32, we + (2 * g + 1) * 32, 32);
                float da = act->d[abl + 2 * g], db = act->d[abl + 2 * g + 1];
                int32_t sa = act->sum[abl + 2 * g], sb = act->sum[abl + 2 * g + 1];
                acc += d * da * (float)s1 * s_lo - da * dmin * (float)m1 * (float)sa;
                acc += d * db * (float)s2 * s_hi - db * dmin * (float)m2 * (float)sb;
            }
        }
        return acc;
    }
    case PO_Q6_K: {
        size_t nb = k / 256;
        for (size_t blk = 0; blk < nb; blk++) {
            const uint8_t *p = w + blk * 210;
            float d = f16_at(p + 208);
            int8_t we[8][32];
            unpack_q6k(p, we);
            const int8_t *sc = (const int8_t *)(p + 192);
            size_t abl = lane * act->nb + blk * 8;
            const int8_t *a = act->q + lane * act->k + blk * 256;
            for (size_t half = 0; half < 2; half++) {
                for (size_t g = 0; g < 2; g++) {
                    for (size_t s = 0; s < 4; s++) {
                        float dd = (float)idot(a + (4 * half + s) * 32 + g * 16, &we[4 * half + s][g * 16], 16);
                        float scale = (float)sc[half * 8 + g + 2 * s];
                        float da = act->d[abl + 4 * half + s];
                        acc += d * scale * da * dd;
                    }
                }
            }
        }
        return acc;
    }
    default:
        return 0.0f;
    }
}

/* quant_int.rs:255-419 (lanes::*).  The per-lane float order is the same
 * as the single-lane form, which the reference proves bitwise
 * (tests/quant_layout.rs:327-357). */
void po_dot_row_q8_lanes(uint32_t t, const uint8_t *w, size_t k, const po_q8act *act, float *out, size_t b) {
    float acc[MAX_BATCH];
    for (size_t l = 0; l < b; l++) acc[l] = 0.0f;
    switch (t) {
    case PO_Q8_0: {
        size_t nb = k / 32;
        for (size_t blk = 0; blk < nb; blk++) {
            const uint8_t *p = w + blk * 34;
            float d = f16_at(p);
            for (size_t lane = 0; lane < b; lane++) {
                int32_t s = idot(act->q + lane * act->k + blk * 32, (const int8_t *)(p + 2), 32);
                acc[lane] += d * act->d[lane * nb + blk] * (float)s;
            }
        }
        break;
    }
    case PO_Q4_0: {
        size_t nb = k / 32;
        for (size_t blk = 0; blk < nb; blk++) {
            const uint8_t *p = w + blk * 18;
            float d = f16_at(p);
            int8_t we[32];
            for (int i = 0; i < 16; i++) { we[i] = (int8_t)(p[2 + i] & 0xF); we[16 + i] = (int8_t)(p[2 + i] >> 4); }
            for (size_t lane = 0; lane < b; lane++) {
                int32_t s = idot(act->q + lane * act->k + blk * 32, we, 32);
                float dq = act->d[lane * nb + blk];
                int32_t sq = act->sum[lane * nb + blk];
                acc[lane] += d * dq * ((float)s - 8.0f * (float)sq);
            }
        }
        break;
    }
    case PO_Q4_K: {
        size_t nb = k / 256;
        int8_t we[256];
        for (size_t blk = 0; blk < nb; blk++) {
            const uint8_t *p = w + blk * 144;
            float d = f16_at(p), dmin = f16_at(p + 2);
            const uint8_t *scales = p + 4;
            unpack_q4k(p, we);
            for (size_t lane = 0; lane < b; lane++) {
                size_t abl = lane * act->nb + blk * 8;
                for (size_t sb = 0; sb < 8; sb++) {
                    uint8_t s, m;
                    scale_min_k4(sb, scales, &s, &m);
                    const int8_t *a = act->q + lane * act->k + blk * 256 + sb * 32;
                    float qd = (float)idot(a, we + sb * 32, 32);
                    float da = act->d[abl + sb];
                    int32_t sa = act->sum[abl + sb];
                    acc[lane] += d * da * (float)s * qd - da * dmin * (float)m * (float)sa;
                }
            }
        }
        break;
    }
    case PO_Q6_K: {
        size_t nb = k / 256;
        int8_t we[8][32];
        for (size_t blk = 0; blk < nb; blk++) {
            const uint8_t *p = w + blk * 210;
            float d = f16_at(p + 208);
            unpack_q6k(p, we);
            const int8_t *sc = (const int8_t *)(p + 192);
            for (size_t lane = 0; lane < b; lane++) {
                size_t abl = lane * act->nb + blk * 8;
                for (size_t half = 0; half < 2; half++)
                    for (size_t g = 0; g < 2; g++)
                        for (size_t s = 0; s < 4; s++) {
                            float da = act->d[abl + 4 * half + s];
                            const int8_t *a = act->q + lane * act->k + blk * 256 + (4 * half + s) * 32 + g * 16;
                            float qd = (float)idot(a, &we[4 * half + s][g * 16], 16);
                            float scale = (float)sc[half * 8 + g + 2 * s];
                            acc[lane] += d * scale * da * qd;
                        }
            }
        }
        break;
    }
    default:
        for (size_t lane = 0; lane < b; lane++) out[lane] += po_dot_row_q8(t, w, k, act, lane);
        return;
    }
    for (size_t lane = 0; lane < b; lane++) out[lane] += acc[lane];
}

long po_block_sums(uint32_t t, const uint8_t *w, size_t k, const po_q8act *act, size_t lane, int32_t *sums) {
    const int8_t *a = act->q + lane * act->k;
    long n = 0;
    switch (t) {
    case PO_Q8_0:
        for (size_t blk = 0; blk < k / 32; blk++)
            sums[n++] = idot(a + blk * 32, (const int8_t *)(w + blk * 34 + 2), 32);
        return n;
    case PO_Q4_0:
        for (size_t blk = 0; blk < k / 32; blk++) {
            const uint8_t *p = w + blk * 18;
            int8_t we[32];
            for (int i = 0; i < 16; i++) { we[i] = (int8_t)(p[2 + i] & 0xF); we[16 + i] = (int8_t)(p[2 + i] >> 4); }
            sums[n++] = idot(a + blk * 32, we, 32);
        }
        return n;
    case PO_Q4_K:
        for (size_t blk = 0; blk < k / 256; blk++) {
            int8_t we[256];
            unpack_q4k(w + blk * 144, we);
            for (size_t sb = 0; sb < 8; sb++) sums[n++] = idot(a + blk * 256 + sb * 32, we + sb * 32, 32);
        }
        return n;
    case PO_Q6_K:
        /* the visiting order of q6_k_lanes: half, g, s */
        for (size_t blk = 0; blk < k / 256; blk++) {
            int8_t we[8][32];
            unpack_q6k(w + blk * 210, we);
            for (size_t half = 0; half < 2; half++)
                for (size_t g = 0; g < 2; g++)
                    for (size_t s = 0; s < 4; s++)
                        sums[n++] = idot(a + blk * 256 + (4 * half + s) * 32 + g * 16, &we[4 * half + s][g * 16], 16);
        }
        return n;
    default:
        return -1;
    }
}

/* ------------------------------------------------------------------------ */
/* quant.rs:102-359                                                          */
void po_dequant_row(uint32_t t, const uint8_t *data, size_t k, float *out) {
    size_t done = 0, off = 0;
    switch (t) {
    case PO_F32: for (size_t i = 0; i < k; i++) out[i] = f32_at(data + i * 4); return;
    case PO_F16: for (size_t i = 0; i < k; i++) out[i] = f16_at(data + i * 2); return;
    case PO_BF16: for (size_t i = 0; i < k; i++) out[i] = bf16_at(data + i * 2); return;
    default: break;
    }
    while (done < k) {
        const uint8_t *p = data + off;
        switch (t) {
        case PO_Q4_0: {
            float d = f16_at(p);
            for (int j = 0; j < 16; j++) {
                uint8_t v = p[2 + j];
                out[done + j] = ((float)(v & 0x0F) - 8.0f) * d;
                out[done + j + 16] = ((float)(v >> 4) - 8.0f) * d;
            }
            off += 18; done += 32;
            break;
        }
        case PO_Q4_1: {
            float d = f16_at(p), m = f16_at(p + 2);
            for (int j = 0; j < 16; j++) {
                uint8_t v = p[4 + j];
                out[done + j] = (float)(v & 0x0F) * d + m;
                out[done + j + 16] = (float)(v >> 4) * d + m;
            }
            off += 20; done += 32;
            break;
        }
        case PO_Q5_0: {
            float d = f16_at(p);
            uint32_t qh = u32_at(p + 2);
            for (int j = 0; j < 16; j++) {
                uint32_t xh0 = ((qh >> j) << 4) & 0x10u, xh1 = (qh >> (j + 12)) & 0x10u;
                uint8_t v = p[6 + j];
                out[done + j] = ((float)((uint32_t)(v & 0x0F) | xh0) - 16.0f) * d;
                out[done + j + 16] = ((float)((uint32_t)(v >> 4) | xh1) - 16.0f) * d;
            }
            off += 22; done += 32;
            break;
        }
        case PO_Q5_1: {
            float d = f16_at(p), m = f16_at(p + 2);
            uint32_t qh = u32_at(p + 4);
            for (int j = 0; j < 16; j++) {
                uint32_t xh0 = ((qh >> j) << 4) & 0x10u, xh1 = (qh >> (j + 12)) & 0x10u;
                uint8_t v = p[8 + j];
                out[done + j] = (float)((uint32_t)(v & 0x0F) | xh0) * d + m;
                out[done + j + 16] = (float)((uint32_t)(v >> 4) | xh1) * d + m;
            }
            off += 24; done += 32;
            break;
        }
        case PO_Q8_0: case PO_Q8_1: {
            float d = f16_at(p);
            const uint8_t *qs = p + (t == PO_Q8_0 ? 2 : 4);
            for (int j = 0; j < 32; j++) out[done + j] = (float)(int8_t)qs[j] * d;
            off += (t == PO_Q8_0) ? 34 : 36; done += 32;
            break;
        }
        case PO_Q2_K: {
            /* quant.rs:185-217 advances qp by 32 in every one of the four
             * shifts, so its third shift indexes qs[64..] of a 64-byte slice
             * and panics: the reference has no output for Q2_K.  This follows
             * the GGUF format's layout instead (qs advances 32 bytes per 128
             * elements, ggml's dequantize_row_q2_K) with the reference's float
             * expressions. */
            float d = f16_at(p + 80), dmin = f16_at(p + 82);
            const uint8_t *scales = p, *qs = p + 16;
            size_t is = 0, n = 0, qp = 0;
            while (n < 256) {
                unsigned shift = 0;
                for (int r = 0; r < 4; r++) {
                    uint8_t sc = scales[is++];
                    float dl = d * (float)(sc & 0xF), ml = dmin * (float)(sc >> 4);
                    for (int l = 0; l < 16; l++) out[done + n + l] = dl * (float)((qs[qp + l] >> shift) & 3) - ml;
                    sc = scales[is++];
                    dl = d * (float)(sc & 0xF); ml = dmin * (float)(sc >> 4);
                    for (int l = 0; l < 16; l++) out[done + n + 16 + l] = dl * (float)((qs[qp + 16 + l] >> shift) & 3) - ml;
                    shift += 2; n += 32;
                }
                qp += 32;
            }
            off += 84; done += 256;
            break;
        }
        case PO_Q3_K: {
            /* quant.rs:218-259 indexes hm[qp + l] with qp advancing 32 per
             * shift, past the 32-byte hmask slice from the second shift on,
             * and panics.  This follows the GGUF format's layout (hmask
             * indexed by l alone, bit m of it per shift; qs advancing 32 bytes
             * per 128 elements, ggml's dequantize_row_q3_K) with the
             * reference's float expressions. */
            float d_all = f16_at(p + 108);
            const uint8_t *qs = p + 32, *hm = p;
            uint32_t aux[4];
            for (int i = 0; i < 3; i++) aux[i] = u32_at(p + 96 + i * 4);
            uint32_t tmp = aux[2];
            aux[2] = ((aux[0] >> 4) & 0x0f0f0f0fu) | (((tmp >> 4) & 0x03030303u) << 4);
            aux[3] = ((aux[1] >> 4) & 0x0f0f0f0fu) | (((tmp >> 6) & 0x03030303u) << 4);
            aux[0] = (aux[0] & 0x0f0f0f0fu) | (((tmp >> 0) & 0x03030303u) << 4);
            aux[1] = (aux[1] & 0x0f0f0f0fu) | (((tmp >> 2) & 0x03030303u) << 4);
            uint8_t scales[16];
            memcpy(scales, aux, 16); /* little-endian byte view, as the reference */
            size_t is = 0, n = 0, qp = 0;
            uint8_t m = 1;
            while (n < 256) {
                unsigned shift = 0;
                for (int r = 0; r < 4; r++) {
                    float dl = d_all * ((float)(int8_t)scales[is++] - 32.0f);
                    for (int l = 0; l < 16; l++) {
                        int hi = (hm[l] & m) ? 0 : 4;
                        out[done + n + l] = dl * (float)((int8_t)((qs[qp + l] >> shift) & 3) - hi);
                    }
                    dl = d_all * ((float)(int8_t)scales[is++] - 32.0f);
                    for (int l = 0; l < 16; l++) {
                        int hi = (hm[16 + l] & m) ? 0 : 4;
                        out[done + n + 16 + l] = dl * (float)((int8_t)((qs[qp + 16 + l] >> shift) & 3) - hi);
                    }
                    shift += 2; m = (uint8_t)(m << 1); n += 32;
                }
                qp += 32;
            }
            off += 110; done += 256;
            break;
        }
        case PO_Q4_K: {
            float d = f16_at(p), dmin = f16_at(p + 2);
            const uint8_t *scales = p + 4, *qs = p + 16;
            size_t is = 0, n = 0, qp = 0;
            while (n < 256) {
                uint8_t sc, m;
                scale_min_k4(is, scales, &sc, &m);
                float d1 = d * (float)sc, m1 = dmin * (float)m;
                scale_min_k4(is + 1, scales, &sc, &m);
                float d2 = d * (float)sc, m2 = dmin * (float)m;
                for (int l = 0; l < 32; l++) out[done + n + l] = d1 * (float)(qs[qp + l] & 0x0F) - m1;
                for (int l = 0; l < 32; l++) out[done + n + 32 + l] = d2 * (float)(qs[qp + l] >> 4) - m2;
                qp += 32; n += 64; is += 2;
            }
            off += 144; done += 256;
            break;
        }
        case PO_Q5_K: {
            /* quant.rs:285-319 indexes qh[qp + l] with qp advancing 32 per
             * 64 elements, past the 32-byte qh slice from the second pair of
             * sub-blocks on, and panics.  This follows the GGUF format's
             * layout (qh indexed by l alone, bits u1/u2 moving by two per
             * pair, ggml's dequantize_row_q5_K) with the reference's float
             * expressions. */
            float d = f16_at(p), dmin = f16_at(p + 2);
            const uint8_t *scales = p + 4, *qh = p + 16, *ql = p + 48;
            size_t is = 0, n = 0, qp = 0;
            uint8_t u1 = 1, u2 = 2;
            while (n < 256) {
                uint8_t sc, m;
                scale_min_k4(is, scales, &sc, &m);
                float d1 = d * (float)sc, m1 = dmin * (float)m;
                scale_min_k4(is + 1, scales, &sc, &m);
                float d2 = d * (float)sc, m2 = dmin * (float)m;
                for (int l = 0; l < 32; l++) {
                    uint8_t q = (uint8_t)((ql[qp + l] & 0x0F) + ((qh[l] & u1) ? 16 : 0));
                    out[done + n + l] = d1 * (float)q - m1;
                }
                for (int l = 0; l < 32; l++) {
                    uint8_t q = (uint8_t)((ql[qp + l] >> 4) + ((qh[l] & u2) ? 16 : 0));
                    out[done + n + 32 + l] = d2 * (float)q - m2;
                }
                qp += 32; n += 64; is += 2;
                u1 = (uint8_t)(u1 << 2); u2 = (uint8_t)(u2 << 2);
            }
            off += 176; done += 256;
            break;
        }
        case PO_Q6_K: {
            float d = f16_at(p + 208);
            const uint8_t *ql = p, *qh = p + 128;
            const int8_t *sc = (const int8_t *)(p + 192);
            for (int half = 0; half < 2; half++) {
                int qlb = half * 64, qhb = half * 32, scb = half * 8;
                for (int l = 0; l < 32; l++) {
                    int is = l / 16;
                    int q1 = (int)((ql[qlb + l] & 0xF) | (((qh[qhb + l] >> 0) & 3) << 4)) - 32;
                    int q2 = (int)((ql[qlb + l + 32] & 0xF) | (((qh[qhb + l] >> 2) & 3) << 4)) - 32;
                    int q3 = (int)((ql[qlb + l] >> 4) | (((qh[qhb + l] >> 4) & 3) << 4)) - 32;
                    int q4 = (int)((ql[qlb + l + 32] >> 4) | (((qh[qhb + l] >> 6) & 3) << 4)) - 32;
                    size_t base = done + (size_t)half * 128;
                    out[base + l] = d * (float)sc[scb + is] * (float)q1;
                    out[base + 32 + l] = d * (float)sc[scb + is + 2] * (float)q2;
                    out[base + 64 + l] = d * (float)sc[scb + is + 4] * (float)q3;
                    out[base + 96 + l] = d * (float)sc[scb + is + 6] * (float)q4;
                }
            }
            off += 210; done += 256;
            break;
        }
        case PO_Q8_K: {
            float d = f32_at(p);
            for (int j = 0; j < 256; j++) out[done + j] = (float)(int8_t)p[4 + j] * d;
            off += 292; done += 256;
            break;
        }
        default:
            return;
        }
    }
}

/* quant.rs:377-441 (what quant::dot_row executes on x86, quant.rs:361-375) */
float po_dot_row_scalar(uint32_t t, const uint8_t *data, size_t k, const float *x) {
    float sum = 0.0f;
    switch (t) {
    case PO_F32: for (size_t i = 0; i < k; i++) sum += f32_at(data + i * 4) * x[i]; return sum;
    case PO_F16: for (size_t i = 0; i < k; i++) sum += f16_at(data + i * 2) * x[i]; return sum;
    case PO_BF16: for (size_t i = 0; i < k; i++) sum += bf16_at(data + i * 2) * x[i]; return sum;
    case PO_Q6_K: {
        size_t nb = k / 256;
        float acc = 0.0f;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t *p = data + b * 210;
            float d = f16_at(p + 208);
            const uint8_t *ql = p, *qh = p + 128;
            const int8_t *sc = (const int8_t *)(p + 192);
            const float *xb = x + b * 256;
            for (int half = 0; half < 2; half++) {
                int qlb = half * 64, qhb = half * 32, scb = half * 8;
                for (int l = 0; l < 32; l++) {
                    int is = l / 16;
                    int q1 = (int)((ql[qlb + l] & 0xF) | (((qh[qhb + l] >> 0) & 3) << 4)) - 32;
                    int q2 = (int)((ql[qlb + l + 32] & 0xF) | (((qh[qhb + l] >> 2) & 3) << 4)) - 32;
                    int q3 = (int)((ql[qlb + l] >> 4) | (((qh[qhb + l] >> 4) & 3) << 4)) - 32;
                    int q4 = (int)((ql[qlb + l + 32] >> 4) | (((qh[qhb + l] >> 6) & 3) << 4)) - 32;
                    int o = half * 128;
                    acc += d * (float)sc[scb + is] * (float)q1 * xb[o + l];
                    acc += d * (float)sc[scb + is + 2] * (float)q2 * xb[o + 32 + l];
                    acc += d * (float)sc[scb + is + 4] * (float)q3 * xb[o + 64 + l];
                    acc += d * (float)sc[scb + is + 6] * (float)q4 * xb[o + 96 + l];
                }
            }
        }
        return acc;
    }
    default: {
        size_t be, bb;
        if (!po_type_block(t, &be, &bb)) return 0.0f;
        size_t nb = k / be;
        float tmp[256];
        for (size_t i = 0; i < nb; i++) {
            po_dequant_row(t, data + i * bb, be, tmp);
            for (size_t j = 0; j < be; j++) sum += tmp[j] * x[i * be + j];
        }
        return sum;
    }
    }
}

/* quant.rs:443-476 (x86 branch) */
void po_row_dot_multi(uint32_t t, const uint8_t *row, size_t k, const float *xt, size_t b, float *out) {
    if (b == 1) {
        out[0] = po_dot_row_scalar(t, row, k, xt);
        return;
    }
    size_t be, bb;
    if (!po_type_block(t, &be, &bb)) {
        for (size_t i = 0; i < b; i++) out[i] = 0.0f;
        return;
    }
    size_t nb = k / be;
    float tmp[256];
    for (size_t i = 0; i < nb; i++) {
        po_dequant_row(t, row + i * bb, be, tmp);
        size_t obase = i * be * b;
        for (size_t j = 0; j < be; j++) {
            float w = tmp[j];
            const float *xp = xt + obase + j * b;
            for (size_t bi = 0; bi < b; bi++) out[bi] += w * xp[bi];
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Pool (model.rs:139-350): n-1 workers spin 20000 times then park; the     */
/* caller also steals chunks of ceil(rows/(4n)) rows.  Every row is owned by */
/* one thread, so results do not depend on the thread count.                 */
typedef struct {
    size_t n_rows, chunk, row_bytes, k, b;
    uint32_t t;
    const uint8_t *w;
    const float *xt;
    float *out;
    const po_q8act *act;
} po_job;

struct po_pool {
    int n;
    pthread_t *workers;
    _Atomic size_t gen, done, next;
    _Atomic int shutdown;
    pthread_mutex_t mu;
    pthread_cond_t cv;
    po_job job;
};

static inline void cpu_relax(void) {
#if defined(__x86_64__)
    _mm_pause();
#endif
}

static void run_rows(const po_job *j, size_t start, size_t end) {
    for (size_t r = start; r < end; r++) {
        const uint8_t *row = j->w + r * j->row_bytes;
        float *dst = j->out + r * j->b;
        if (j->act) po_dot_row_q8_lanes(j->t, row, j->k, j->act, dst, j->b);
        else po_row_dot_multi(j->t, row, j->k, j->xt, j->b, dst);
    }
}

static void steal(po_pool *p) {
    const po_job *j = &p->job;
    for (;;) {
        size_t start = atomic_fetch_add_explicit(&p->next, j->chunk, memory_order_relaxed);
        if (start >= j->n_rows) break;
        size_t end = start + j->chunk < j->n_rows ? start + j->chunk : j->n_rows;
        run_rows(j, start, end);
    }
}

static void *worker_main(void *arg) {
    po_pool *p = (po_pool *)arg;
    size_t local = 0;
    for (;;) {
        if (atomic_load_explicit(&p->shutdown, memory_order_acquire)) return NULL;
        unsigned spins = 0;
        while (atomic_load_explicit(&p->gen, memory_order_acquire) == local) {
            if (++spins > 20000) {
                pthread_mutex_lock(&p->mu);
                while (atomic_load_explicit(&p->gen, memory_order_acquire) == local &&
                       !atomic_load_explicit(&p->shutdown, memory_order_acquire))
                    pthread_cond_wait(&p->cv, &p->mu);
                pthread_mutex_unlock(&p->mu);
                spins = 0;
            } else {
                cpu_relax();
            }
        }
        local = atomic_load_explicit(&p->gen, memory_order_acquire);
        if (atomic_load_explicit(&p->shutdown, memory_order_acquire)) return NULL;
        steal(p);
        atomic_fetch_add_explicit(&p->done, 1, memory_order_release);
    }
}

po_pool *po_pool_new(int threads) {
    po_pool *p = (po_pool *)calloc(1, sizeof(po_pool));
    if (!p) return NULL;
    p->n = threads < 1 ? 1 : threads;
    pthread_mutex_init(&p->mu, NULL);
    pthread_cond_init(&p->cv, NULL);
    p->workers = (pthread_t *)calloc((size_t)p->n, sizeof(pthread_t));
    for (int i = 0; i < p->n - 1; i++) pthread_create(&p->workers[i], NULL, worker_main, p);
    return p;
}

void po_pool_free(po_pool *p) {
    if (!p) return;
    pthread_mutex_lock(&p->mu);
    atomic_store_explicit(&p->shutdown, 1, memory_order_release);
    atomic_fetch_add_explicit(&p->gen, 1, memory_order_release);
    pthread_cond_broadcast(&p->cv);
    pthread_mutex_unlock(&p->mu);
    for (int i = 0; i < p->n - 1; i++) pthread_join(p->workers[i], NULL);
    pthread_mutex_destroy(&p->mu);
    pthread_cond_destroy(&p->cv);
    free(p->workers);
    free(p);
}

void po_pool_matmul(po_pool *p, uint32_t t, const uint8_t *w, size_t row_bytes, size_t k,
                    const float *xt, size_t b, float *out, size_t rows, const po_q8act *act) {
    for (size_t i = 0; i < rows * b; i++) out[i] = 0.0f;
    po_job j = {rows, 1, row_bytes, k, b, t, w, xt, out, act};
    if (p->n == 1) {
        run_rows(&j, 0, rows);
        return;
    }
    size_t n4 = (size_t)p->n * 4;
    j.chunk = (rows + n4 - 1) / n4;
    if (j.chunk < 1) j.chunk = 1;
    p->job = j;
    atomic_store_explicit(&p->next, 0, memory_order_relaxed);
    atomic_store_explicit(&p->done, 0, memory_order_relaxed);
    pthread_mutex_lock(&p->mu);
    atomic_fetch_add_explicit(&p->gen, 1, memory_order_release);
    pthread_cond_broadcast(&p->cv);
    pthread_mutex_unlock(&p->mu);
    steal(p);
    while (atomic_load_explicit(&p->done, memory_order_acquire) < (size_t)(p->n - 1)) cpu_relax();
}

/* ------------------------------------------------------------------------ */
/* sampler.rs:1-19 (SplitMix64)                                              */
void po_rng_init(po_rng *r, uint64_t seed) { r->s = seed + 0x9E3779B97F4A7C15ull; }
uint64_t po_rng_next_u64(po_rng *r) {
    uint64_t z = r->s + 0x9E3779B97F4A7C15ull;
    r->s = z;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
float po_rng_next_f32(po_rng *r) { return (float)(po_rng_next_u64(r) >> 40) / (float)(1u << 24); }

/* Descending by probability; equal keys keep index order.  The reference
 * uses an unstable sort (sampler.rs:54-59), so the order of exactly tied
 * probabilities is not pinned by it. */
static const float *g_sort_keys;
static int cmp_desc(const void *a, const void *b) {
    uint32_t ia = *(const uint32_t *)a, ib = *(const uint32_t *)b;
    float va = g_sort_keys[ia], vb = g_sort_keys[ib];
    if (va > vb) return -1;
    if (va < vb) return 1;
    return ia < ib ? -1 : (ia > ib);
}

/* sampler.rs:21-92 */
uint32_t po_sample(float *logits, size_t n, float temp, float top_p, po_rng *rng) {
    if (n == 0) return 0;
    if (temp <= 0.0f) {
        size_t best = 0;
        float bv = -INFINITY;
        for (size_t i = 0; i < n; i++)
            if (logits[i] > bv) { bv = logits[i]; best = i; }
        return (uint32_t)best;
    }
    float inv = 1.0f / temp, max = -INFINITY;
    for (size_t i = 0; i < n; i++) if (logits[i] > max) max = logits[i];
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float e = po_expf((logits[i] - max) * inv);
        logits[i] = e;
        sum += e;
    }
    if (!(sum > 0.0f)) return 0;
    if (top_p > 0.0f && top_p < 1.0f) {
        uint32_t *idx = (uint32_t *)malloc(n * sizeof(uint32_t));
        for (size_t i = 0; i < n; i++) idx[i] = (uint32_t)i;
        g_sort_keys = logits;
        qsort(idx, n, sizeof(uint32_t), cmp_desc);
        float acc = 0.0f;
        size_t cut = n;
        for (size_t kk = 0; kk < n; kk++) {
            acc += logits[idx[kk]] / sum;
            if (acc >= top_p) { cut = kk + 1; break; }
        }
        unsigned char *keep = (unsigned char *)calloc(n, 1);
        for (size_t kk = 0; kk < cut; kk++) keep[idx[kk]] = 1;
        float new_sum = 0.0f;
        for (size_t i = 0; i < n; i++) {
            if (!keep[i]) logits[i] = 0.0f;
            else new_sum += logits[i];
        }
        sum = new_sum;
        free(keep);
        free(idx);
    }
    float r = po_rng_next_f32(rng) * sum;
    float acc = 0.0f;
    for (size_t i = 0; i < n; i++) {
        acc += logits[i];
        if (acc >= r) return (uint32_t)i;
    }
    return (uint32_t)(n - 1);
}

/* ------------------------------------------------------------------------ */
/* util.rs:274-282                                                           */
static _Atomic int g_stop;
void po_request_stop(void) { atomic_store(&g_stop, 1); }
void po_clear_stop(void) { atomic_store(&g_stop, 0); }
static int stop_requested(void) { return atomic_load_explicit(&g_stop, memory_order_relaxed); }

/* ------------------------------------------------------------------------ */
/* Engine (model.rs:678-1352)                                                */
struct po_engine {
    po_model m;
    po_layer *layers;
    uint32_t *eos;
    size_t n_ctx;
    po_pool *pool;
    float *kv_k, *kv_v;            /* [layer][kv_head][n_ctx][head_dim] */
    /* Scratch (model.rs:389-461) */
    float *x, *x2, *q, *k, *v, *attn, *proj, *gate, *up, *row, *scores, *logits;
    size_t n_logits;
    float *rope_cos, *rope_sin, *rope_inv;
    size_t rope_upto, rope_half;
    /* Q8Act storage */
    int8_t *q8q; float *q8d; int32_t *q8s;
    int int8_enabled, kv_int8_enabled;
    uint32_t *kv_tokens;
    size_t kv_len, cached_prefill_len;
    char err[256];
};

static void set_err(po_engine *e, const char *msg) { snprintf(e->err, sizeof e->err, "%s", msg); }
const char *po_last_error(const po_engine *e) { return e->err; }

static size_t row_bytes_of(const po_tensor *t) {
    size_t rb = 0;
    po_tensor_nbytes(t->type, t->ne0, 1, &rb);
    return rb;
}

static int check_shape(const po_tensor *t, size_t cols, size_t rows) { return t->ne0 == cols && t->ne1 == rows; }

static int int8_supported(uint32_t t) {
    /* quant_int.rs:75-80 with int8_available() true (the aarch64 semantics) */
    return t == PO_Q4_K || t == PO_Q6_K || t == PO_Q4_0 || t == PO_Q8_0;
}

po_engine *po_engine_create(const po_model *m, size_t n_ctx, int threads, char *err, size_t errlen) {
#define FAIL(msg) do { if (err) snprintf(err, errlen, "%s", msg); po_engine_destroy(e); return NULL; } while (0)
    po_engine *e = (po_engine *)calloc(1, sizeof(po_engine));
    if (!e) return NULL;
    e->m = *m;
    e->layers = (po_layer *)malloc(sizeof(po_layer) * (m->n_layer ? m->n_layer : 1));
    memcpy(e->layers, m->layers, sizeof(po_layer) * m->n_layer);
    e->m.layers = e->layers;
    e->eos = (uint32_t *)malloc(sizeof(uint32_t) * (m->n_eos + 1));
    if (m->n_eos) memcpy(e->eos, m->eos_ids, sizeof(uint32_t) * m->n_eos);
    e->m.eos_ids = e->eos;
    /* Model::finish (model.rs:571-601) */
    size_t vocab = m->token_embd.ne1, ne = m->n_embd;
    size_t qdim = m->n_head * m->head_dim, kdim = m->n_head_kv * m->head_dim;
    if (m->n_layer == 0 || ne == 0 || m->n_ff == 0 || m->n_head == 0) FAIL("invalid model configuration");
    if (m->head_dim == 0 || m->n_head_kv == 0 || m->n_head % m->n_head_kv) FAIL("invalid GQA configuration");
    if (m->n_rot == 0 || m->n_rot > m->head_dim || m->n_rot % 2) FAIL("invalid RoPE / RMSNorm configuration");
    if (vocab == 0 || m->token_embd.ne0 != ne || (m->n_vocab && m->n_vocab != vocab))
        FAIL("embedding / metadata / tokenizer vocab dimensions disagree");
    if (!check_shape(&m->output, ne, vocab) || !check_shape(&m->output_norm, ne, 1)) FAIL("bad output shape");
    for (size_t l = 0; l < m->n_layer; l++) {
        const po_layer *L = &m->layers[l];
        if (!check_shape(&L->attn_norm, ne, 1) || !check_shape(&L->ffn_norm, ne, 1) ||
            !check_shape(&L->attn_q, ne, qdim) || !check_shape(&L->attn_k, ne, kdim) ||
            !check_shape(&L->attn_v, ne, kdim) || !check_shape(&L->attn_o, qdim, ne) ||
            !check_shape(&L->ffn_gate, ne, m->n_ff) || !check_shape(&L->ffn_up, ne, m->n_ff) ||
            !check_shape(&L->ffn_down, m->n_ff, ne))
            FAIL("layer tensor shape mismatch");
    }
    e->n_ctx = n_ctx;
    size_t nkv = m->n_layer * m->n_head_kv * n_ctx * m->head_dim;
    e->kv_k = (float *)calloc(nkv, sizeof(float));
    e->kv_v = (float *)calloc(nkv, sizeof(float));
    if (!e->kv_k || !e->kv_v) FAIL("cannot allocate KV cache");
    size_t nb = MAX_BATCH;
    size_t big = ne > m->n_ff ? ne : m->n_ff;
    e->x = calloc(ne * nb, 4); e->x2 = calloc(ne * nb, 4);
    e->q = calloc(qdim * nb, 4); e->k = calloc(kdim * nb, 4); e->v = calloc(kdim * nb, 4);
    e->attn = calloc(qdim * nb, 4); e->proj = calloc(ne * nb, 4);
    e->gate = calloc(m->n_ff * nb, 4); e->up = calloc(m->n_ff * nb, 4);
    e->row = calloc(big, 4); e->scores = calloc(n_ctx, 4);
    e->n_logits = (m->n_vocab ? m->n_vocab : 1);
    if (e->n_logits < m->output.ne1) e->n_logits = m->output.ne1;
    e->logits = calloc(e->n_logits, 4);
    size_t half = m->n_rot / 2;
    e->rope_half = half ? half : 1;
    e->rope_inv = calloc(e->rope_half, 4);
    for (size_t i = 0; i < half; i++)
        e->rope_inv[i] = 1.0f / po_powf(m->rope_theta, 2.0f * (float)i / (float)m->n_rot);
    e->rope_cos = calloc(n_ctx * half + 1, 4);
    e->rope_sin = calloc(n_ctx * half + 1, 4);
    e->q8q = malloc(big * nb); e->q8d = malloc(big / 32 * nb * 4 + 4); e->q8s = malloc(big / 32 * nb * 4 + 4);
    e->kv_tokens = calloc(n_ctx + 1, 4);
    e->int8_enabled = e->kv_int8_enabled = 1;
    e->pool = po_pool_new(threads);
    if (!e->x || !e->logits || !e->pool || !e->q8q) FAIL("out of memory");
    return e;
#undef FAIL
}

void po_engine_destroy(po_engine *e) {
    if (!e) return;
    if (e->pool) po_pool_free(e->pool);
    free(e->layers); free(e->eos); free(e->kv_k); free(e->kv_v);
    free(e->x); free(e->x2); free(e->q); free(e->k); free(e->v); free(e->attn); free(e->proj);
    free(e->gate); free(e->up); free(e->row); free(e->scores); free(e->logits);
    free(e->rope_cos); free(e->rope_sin); free(e->rope_inv);
    free(e->q8q); free(e->q8d); free(e->q8s); free(e->kv_tokens);
    free(e);
}

void po_engine_set_int8(po_engine *e, int enabled) { e->int8_enabled = enabled; }
const float *po_logits(const po_engine *e) { return e->logits; }
size_t po_n_logits(const po_engine *e) { return e->n_logits; }
float *po_kv_k(po_engine *e) { return e->kv_k; }
float *po_kv_v(po_engine *e) { return e->kv_v; }
size_t po_kv_index(const po_engine *e, size_t l, size_t h, size_t pos, size_t d) {
    return ((l * e->m.n_head_kv + h) * e->n_ctx + pos) * e->m.head_dim + d;
}

/* Scratch::ensure_rope (model.rs:445-460) */
static void ensure_rope(po_engine *e, size_t upto) {
    size_t half = e->rope_half;
    size_t cap = (e->n_ctx * (e->m.n_rot / 2)) / half;
    size_t n = upto < cap ? upto : cap;
    if (n <= e->rope_upto) return;
    for (size_t pos = e->rope_upto; pos < n; pos++)
        for (size_t i = 0; i < half; i++) {
            float a = (float)pos * e->rope_inv[i];
            e->rope_cos[pos * half + i] = po_cosf(a);
            e->rope_sin[pos * half + i] = po_sinf(a);
        }
    e->rope_upto = n;
}

/* Engine::matmul (model.rs:725-756) without a GPU backend */
static void engine_matmul(po_engine *e, const po_tensor *w, const float *x, size_t b, float *out) {
    size_t rb = row_bytes_of(w);
    if (e->int8_enabled && int8_supported(w->type)) {
        po_q8_prepare(x, w->ne0, b, e->q8q, e->q8d, e->q8s);
        po_q8act act = {e->q8q, e->q8d, e->q8s, w->ne0, b, w->ne0 / 32};
        po_pool_matmul(e->pool, w->type, w->data, rb, w->ne0, x, b, out, w->ne1, &act);
        return;
    }
    po_pool_matmul(e->pool, w->type, w->data, rb, w->ne0, x, b, out, w->ne1, NULL);
}

/* simd::f32_sum_sq (simd.rs:45-64): two 4-lane FMA accumulators over steps
 * of 8, lane-wise add, vaddvq_f32 = (t0 + t1) + (t2 + t3), scalar tail. */
static float neon_sum_sq(const float *x, size_t n) {
    float a0[4] = {0, 0, 0, 0}, a1[4] = {0, 0, 0, 0}, t[4];
    size_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int j = 0; j < 4; j++) {
            a0[j] = fmaf(x[i + j], x[i + j], a0[j]);
            a1[j] = fmaf(x[i + 4 + j], x[i + 4 + j], a1[j]);
        }
    for (int j = 0; j < 4; j++) t[j] = a0[j] + a1[j];
    float s = (t[0] + t[1]) + (t[2] + t[3]);
    for (; i < n; i++) s += x[i] * x[i];
    return s;
}

/* simd::f32_dot (simd.rs:17-43): two 4-lane accumulators of products (no
 * FMA), s = vaddvq(acc0), s += vaddvq(acc1), scalar tail. */
static float neon_dot(const float *a, const float *b, size_t n) {
    float a0[4] = {0, 0, 0, 0}, a1[4] = {0, 0, 0, 0};
    size_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int j = 0; j < 4; j++) {
            a0[j] = a0[j] + a[i + j] * b[i + j];
            a1[j] = a1[j] + a[i + 4 + j] * b[i + 4 + j];
        }
    float s = (a0[0] + a0[1]) + (a0[2] + a0[3]);
    s += (a1[0] + a1[1]) + (a1[2] + a1[3]);
    for (; i < n; i++) s += a[i] * b[i];
    return s;
}

/* Engine::rmsnorm (model.rs:777-823) as built for aarch64: b == 1 uses
 * f32_sum_sq then f32_rms_apply (out = x*s*w); b > 1 the scalar loop. */
static void engine_rmsnorm(po_engine *e, const float *x, const po_tensor *w, size_t b, float *out) {
    size_t ne = e->m.n_embd;
    float eps = e->m.rms_eps;
    const float *wp;
    float *wbuf = NULL;
    if (w->type == PO_F32 && ((uintptr_t)w->data % 4) == 0) {
        wp = (const float *)w->data;
    } else {
        wbuf = (float *)malloc(ne * 4);
        po_dequant_row(w->type, w->data, ne, wbuf);
        wp = wbuf;
    }
    if (b == 1) {
        float ss = neon_sum_sq(x, ne);
        float s = 1.0f / sqrtf(ss / (float)ne + eps);
        for (size_t i = 0; i < ne; i++) out[i] = x[i] * s * wp[i];
        free(wbuf);
        return;
    }
    for (size_t bi = 0; bi < b; bi++) {
        float ss = 0.0f;
        for (size_t i = 0; i < ne; i++) { float v = x[i * b + bi]; ss += v * v; }
        float s = 1.0f / sqrtf(ss / (float)ne + eps);
        for (size_t i = 0; i < ne; i++) out[i * b + bi] = x[i * b + bi] * s * wp[i];
    }
    free(wbuf);
}

/* Engine::forward_inner + forward_layers (model.rs:833-1172) */
static int forward_inner(po_engine *e, const uint32_t *ids, const size_t *positions, size_t b,
                         int want_logits, int cancellable) {
    const po_model *m = &e->m;
    if (b == 0 || b > MAX_BATCH) { set_err(e, "invalid batch"); return -1; }
    size_t ne = m->n_embd, dh = m->head_dim;
    size_t vocab = m->token_embd.ne1, maxpos = 0;
    for (size_t i = 0; i < b; i++) {
        if (positions[i] >= e->n_ctx) { set_err(e, "context full"); return -1; }
        if (ids[i] >= vocab) { set_err(e, "token out of vocab"); return -1; }
        if (positions[i] > maxpos) maxpos = positions[i];
    }
    ensure_rope(e, maxpos + 1);
    size_t tok_bytes = row_bytes_of(&m->token_embd);
    for (size_t bi = 0; bi < b; bi++) {
        po_dequant_row(m->token_embd.type, m->token_embd.data + (size_t)ids[bi] * tok_bytes, ne, e->row);
        for (size_t i = 0; i < ne; i++) e->x[i * b + bi] = e->row[i];
    }
    size_t n_head = m->n_head, n_kv = m->n_head_kv, group = n_head / n_kv;
    float scale = 1.0f / sqrtf((float)dh);
    float *x = e->x, *x2 = e->x2, *q = e->q, *k = e->k, *v = e->v, *attn = e->attn, *proj = e->proj;
    for (size_t l = 0; l < m->n_layer; l++) {
        const po_layer *L = &m->layers[l];
        if (cancellable && stop_requested()) { set_err(e, "generation stopped"); return -1; }
        engine_rmsnorm(e, x, &L->attn_norm, b, x2);
        engine_matmul(e, &L->attn_q, x2, b, q);
        engine_matmul(e, &L->attn_k, x2, b, k);
        engine_matmul(e, &L->attn_v, x2, b, v);
        size_t half = m->n_rot / 2;
        for (size_t bi = 0; bi < b; bi++) {
            const float *cb = e->rope_cos + positions[bi] * half, *sb = e->rope_sin + positions[bi] * half;
            for (size_t h = 0; h < n_head; h++)
                for (size_t i = 0; i < half; i++) {
                    size_t i0 = (h * dh + 2 * i) * b + bi, i1 = (h * dh + 2 * i + 1) * b + bi;
                    float x0 = q[i0], x1 = q[i1];
                    q[i0] = x0 * cb[i] - x1 * sb[i];
                    q[i1] = x0 * sb[i] + x1 * cb[i];
                }
            for (size_t h = 0; h < n_kv; h++)
                for (size_t i = 0; i < half; i++) {
                    size_t i0 = (h * dh + 2 * i) * b + bi, i1 = (h * dh + 2 * i + 1) * b + bi;
                    float x0 = k[i0], x1 = k[i1];
                    k[i0] = x0 * cb[i] - x1 * sb[i];
                    k[i1] = x0 * sb[i] + x1 * cb[i];
                }
        }
        for (size_t bi = 0; bi < b; bi++)
            for (size_t h = 0; h < n_kv; h++) {
                size_t base = po_kv_index(e, l, h, positions[bi], 0);
                for (size_t d = 0; d < dh; d++) {
                    e->kv_k[base + d] = k[(h * dh + d) * b + bi];
                    e->kv_v[base + d] = v[(h * dh + d) * b + bi];
                }
            }
        /* attention (model.rs:993-1087), aarch64 build: scores by f32_dot at
         * b == 1 and by the scalar loop at b > 1; values by f32_axpy, skipping
         * zero weights, into a zeroed row scaled by 1/sum afterwards. */
        float *orow = e->row;
        for (size_t bi = 0; bi < b; bi++) {
            size_t pos = positions[bi];
            for (size_t h = 0; h < n_head; h++) {
                size_t kh = h / group, qbase = (h * dh) * b + bi;
                float maxs = -INFINITY;
                for (size_t p = 0; p <= pos; p++) {
                    const float *kr = e->kv_k + po_kv_index(e, l, kh, p, 0);
                    float s;
                    if (b == 1) {
                        s = neon_dot(q + qbase, kr, dh);
                    } else {
                        s = 0.0f;
                        for (size_t d = 0; d < dh; d++) s += q[qbase + d * b] * kr[d];
                    }
                    s = s * scale;
                    e->scores[p] = s;
                    if (s > maxs) maxs = s;
                }
                float sum = 0.0f;
                for (size_t p = 0; p <= pos; p++) {
                    float ex = po_expf(e->scores[p] - maxs);
                    e->scores[p] = ex;
                    sum += ex;
                }
                float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
                for (size_t d = 0; d < dh; d++) orow[d] = 0.0f;
                for (size_t p = 0; p <= pos; p++) {
                    float s = e->scores[p];
                    if (s != 0.0f) {
                        const float *vr = e->kv_v + po_kv_index(e, l, kh, p, 0);
                        for (size_t d = 0; d < dh; d++) orow[d] = orow[d] + s * vr[d];
                    }
                }
                for (size_t d = 0; d < dh; d++) attn[(h * dh + d) * b + bi] = orow[d] * inv;
            }
        }
        engine_matmul(e, &L->attn_o, attn, b, proj);
        for (size_t i = 0; i < ne * b; i++) x[i] += proj[i];
        engine_rmsnorm(e, x, &L->ffn_norm, b, x2);
        engine_matmul(e, &L->ffn_gate, x2, b, e->gate);
        engine_matmul(e, &L->ffn_up, x2, b, e->up);
        for (size_t i = 0; i < m->n_ff * b; i++) {
            float g = e->gate[i];
            float s = g / (1.0f + po_expf(-g));
            e->gate[i] = s * e->up[i];
        }
        engine_matmul(e, &L->ffn_down, e->gate, b, proj);
        for (size_t i = 0; i < ne * b; i++) x[i] += proj[i];
    }
    if (want_logits) {
        if (cancellable && stop_requested()) { set_err(e, "generation stopped"); return -1; }
        size_t last = b - 1;
        float *last_x = (float *)malloc(ne * 4), *normed = (float *)malloc(ne * 4);
        for (size_t i = 0; i < ne; i++) last_x[i] = x[i * b + last];
        engine_rmsnorm(e, last_x, &m->output_norm, 1, normed);
        const po_tensor *out = &m->output;
        size_t n_rows = out->ne1;
        if (e->n_logits < n_rows) {
            e->logits = realloc(e->logits, n_rows * 4);
            e->n_logits = n_rows;
        }
        if (e->int8_enabled && int8_supported(out->type)) {
            po_q8_prepare(normed, out->ne0, 1, e->q8q, e->q8d, e->q8s);
            po_q8act act = {e->q8q, e->q8d, e->q8s, out->ne0, 1, out->ne0 / 32};
            po_pool_matmul(e->pool, out->type, out->data, row_bytes_of(out), out->ne0, normed, 1, e->logits, n_rows, &act);
        } else {
            po_pool_matmul(e->pool, out->type, out->data, row_bytes_of(out), out->ne0, normed, 1, e->logits, n_rows, NULL);
        }
        free(last_x);
        free(normed);
    }
    return 0;
}

/* Engine::forward (model.rs:825-831) */
int po_forward(po_engine *e, const uint32_t *ids, const size_t *pos, size_t b, int want_logits) {
    e->kv_len = 0;
    e->cached_prefill_len = 0;
    return forward_inner(e, ids, pos, b, want_logits, 0);
}

static double now_ms(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e3 + ts.tv_nsec / 1e6;
}

static int is_eog(const po_engine *e, uint32_t tok) {
    for (size_t i = 0; i < e->m.n_eos; i++) if (e->eos[i] == tok) return 1;
    return 0;
}

/* Engine::generate (model.rs:1235-1352).  The reference's CPU-only engine
 * keeps prefix reuse across calls; this oracle has no GPU backend. */
int po_generate(po_engine *e, const uint32_t *prompt, size_t n, const po_genopts *o, po_genstats *st,
                uint32_t *gen_ids) {
    memset(st, 0, sizeof *st);
    snprintf(st->stop, sizeof st->stop, "max_tokens");
    po_rng rng;
    po_rng_init(&rng, o->seed);
    if (n == 0) { set_err(e, "empty prompt"); return -1; }
    double t0 = now_ms();
    const size_t chunk = 32;
    if (e->kv_int8_enabled != e->int8_enabled) { e->kv_len = 0; e->cached_prefill_len = 0; }
    e->kv_int8_enabled = e->int8_enabled;
    size_t common = 0;
    while (common < e->kv_len && common < n && e->kv_tokens[common] == prompt[common]) common++;
    size_t reused = common;
    if (reused > e->cached_prefill_len) reused = e->cached_prefill_len;
    if (reused > n - 1) reused = n - 1;
    reused = reused / chunk * chunk;
    e->kv_len = reused;
    e->cached_prefill_len = 0;
    st->prefill_cached_tokens = reused;
    size_t off = reused;
    size_t positions[32];
    while (off < n) {
        if (stop_requested()) { snprintf(st->stop, sizeof st->stop, "user_stop"); break; }
        size_t cnt = n - off < chunk ? n - off : chunk;
        for (size_t i = 0; i < cnt; i++) positions[i] = off + i;
        int last = off + cnt >= n;
        if (forward_inner(e, prompt + off, positions, cnt, last, 1) != 0) {
            e->kv_len = 0;
            if (stop_requested()) { snprintf(st->stop, sizeof st->stop, "user_stop"); break; }
            return -1;
        }
        if (e->kv_len + cnt <= e->n_ctx) memcpy(e->kv_tokens + e->kv_len, prompt + off, cnt * 4);
        e->kv_len += cnt;
        off += cnt;
    }
    st->prefill_tokens = off - reused;
    st->prefill_ms = now_ms() - t0;
    if (strcmp(st->stop, "user_stop") == 0) { e->kv_len = 0; return 0; }
    e->cached_prefill_len = n;
    size_t pos = n;
    double g0 = now_ms();
    size_t nvocab = e->m.token_embd.ne1 < e->n_logits ? e->m.token_embd.ne1 : e->n_logits;
    for (size_t i = 0; i < o->max_tokens; i++) {
        if (stop_requested()) { snprintf(st->stop, sizeof st->stop, "user_stop"); break; }
        uint32_t tok = po_sample(e->logits, nvocab, o->temp, o->top_p, &rng);
        if (is_eog(e, tok)) { snprintf(st->stop, sizeof st->stop, "eog"); break; }
        gen_ids[st->gen_tokens++] = tok;
        if (i + 1 == o->max_tokens) break;
        if (pos >= e->n_ctx) { snprintf(st->stop, sizeof st->stop, "context_full"); break; }
        size_t p1 = pos;
        if (forward_inner(e, &tok, &p1, 1, 1, 1) != 0) {
            e->kv_len = 0;
            e->cached_prefill_len = 0;
            if (stop_requested()) { snprintf(st->stop, sizeof st->stop, "user_stop"); break; }
            return -1;
        }
        if (e->kv_len < e->n_ctx) e->kv_tokens[e->kv_len] = tok;
        e->kv_len++;
        pos++;
    }
    if (strcmp(st->stop, "user_stop") == 0) { e->kv_len = 0; e->cached_prefill_len = 0; }
    st->gen_ms = now_ms() - g0;
    return 0;
}

/* Exported views of po_detmath.h for tests. */
float po_det_expf(float x) { return po_expf(x); }
float po_det_cosf(float x) { return po_cosf(x); }
float po_det_sinf(float x) { return po_sinf(x); }
float po_det_powf(float x, float y) { return po_powf(x, y); }
