// Shared definitions of the pocketinfer HIP backend: type table, f16
// conversion and the tiled weight layout.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>

#include "../../include/pocketinfer_hip.h"

#if defined(__HIPCC__)
#define PI_HD __host__ __device__
#else
#define PI_HD
#endif

// quant.rs:19-37: elements and bytes per block.
inline size_t pi_type_block_elems(uint32_t t) {
    switch (t) {
    case PI_TYPE_F32: case PI_TYPE_F16: case PI_TYPE_BF16: return 1;
    case PI_TYPE_Q4_0: case PI_TYPE_Q4_1: case PI_TYPE_Q5_0: case PI_TYPE_Q5_1: case PI_TYPE_Q8_0: case PI_TYPE_Q8_1:
        return 32;
    case PI_TYPE_Q2_K: case PI_TYPE_Q3_K: case PI_TYPE_Q4_K: case PI_TYPE_Q5_K: case PI_TYPE_Q6_K: case PI_TYPE_Q8_K:
        return 256;
    default: return 0;
    }
}
inline size_t pi_type_block_bytes(uint32_t t) {
    switch (t) {
    case PI_TYPE_F32: return 4;
    case PI_TYPE_F16: case PI_TYPE_BF16: return 2;
    case PI_TYPE_Q4_0: return 18;
    case PI_TYPE_Q4_1: return 20;
    case PI_TYPE_Q5_0: return 22;
    case PI_TYPE_Q5_1: return 24;
    case PI_TYPE_Q8_0: return 34;
    case PI_TYPE_Q8_1: return 36;
    case PI_TYPE_Q2_K: return 84;
    case PI_TYPE_Q3_K: return 110;
    case PI_TYPE_Q4_K: return 144;
    case PI_TYPE_Q5_K: return 176;
    case PI_TYPE_Q6_K: return 210;
    case PI_TYPE_Q8_K: return 292;
    default: return 0;
    }
}
// Row bytes (quant.rs:60-72 for one row); 0 when unsupported or k not divisible.
inline size_t pi_row_bytes(uint32_t t, size_t k) {
    size_t be = pi_type_block_elems(t);
    if (be == 0 || k % be) return 0;
    return k / be * pi_type_block_bytes(t);
}
// Types with the int8 path (quant_int.rs:75-80): tiled layout, Q8 activations.
inline bool pi_gemv_type(uint32_t t) {
    return t == PI_TYPE_Q4_K || t == PI_TYPE_Q6_K || t == PI_TYPE_Q4_0 || t == PI_TYPE_Q8_0;
}
// Types the reference evaluates on its f32 path (quant.rs:377-441) that have a
// row kernel here (GGUF row layout; BF16 rows of a multiple of 32 elements).
inline bool pi_row_type(uint32_t t) {
    switch (t) {
    case PI_TYPE_Q4_1: case PI_TYPE_Q5_0: case PI_TYPE_Q5_1: case PI_TYPE_Q8_1: case PI_TYPE_Q2_K: case PI_TYPE_Q3_K:
    case PI_TYPE_Q5_K: case PI_TYPE_Q8_K: case PI_TYPE_BF16:
        return true;
    default: return false;
    }
}

// util.rs:76-100: exact half -> single, subnormals included.
PI_HD inline float pi_f16_to_f32(uint16_t h) {
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
        bits = (sign << 31) | ((exp + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// util.rs:102-138: single -> half, round to nearest even.
inline uint16_t pi_f32_to_f16(float v) {
    uint32_t bits;
    memcpy(&bits, &v, 4);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    int32_t exp = (int32_t)((bits >> 23) & 0xFFu);
    uint32_t mant = bits & 0x7FFFFFu;
    if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant ? (0x200u | (mant >> 13)) : 0u));
    int32_t e = exp - 127 + 15;
    if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return sign;
        uint32_t m = mant | 0x800000u, shift = (uint32_t)(14 - e);
        uint16_t half = (uint16_t)(m >> shift);
        uint32_t rem = m & ((1u << shift) - 1u), hb = 1u << (shift - 1);
        if (rem > hb || (rem == hb && (half & 1u))) half++;
        return (uint16_t)(sign | half);
    }
    uint16_t half = (uint16_t)(((uint32_t)e << 10) | (mant >> 13));
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) {
        half++;
        if ((half & 0x7C00u) == 0x7C00u) return (uint16_t)(sign | 0x7C00u);
    }
    return (uint16_t)(sign | half);
}

// ---------------------------------------------------------------------------
// Tiled weight layout ("lane-interleaved units").
//
// A row of k elements is cut into `upr` units of `g` base blocks (a base
// block is one 256-element super-block for Q4_K/Q6_K, one 32-element block
// for Q4_0/Q8_0).  One wavefront tile holds `rpw` whole rows, i.e.
// lpt = rpw*upr units, one unit per lane; lane l of tile t owns unit
// (row t*rpw + l/upr, unit l%upr).  Inside a tile of `lanes` units:
//   Q plane: chunk j (16 bytes) of lane l at  (j*lanes + l)*16
//   D plane: f16 field f of lane l at          lanes*qc*16 + (f*lanes + l)*2
//            (plane padded to 16 bytes)
// so every load instruction of a wavefront reads one contiguous span.
// Unit contents per base block (b = 0..g-1):
//   Q4_K: 9 chunks = the native 144-byte block (d, dmin, scales | qs[128])
//   Q6_K: 13 chunks = ql[128] | qh[64] | scales[16]; D field = d
//   Q4_0: 1 chunk  = qs[16];                          D field = d
//   Q8_0: 2 chunks = qs[32];                          D field = d
// Tiles are stored back to back; all tiles but the last are full.
// ---------------------------------------------------------------------------
struct pi_layout {
    uint32_t type, k, rows;
    uint32_t g;        // base blocks per unit
    uint32_t upr;      // units per row
    uint32_t rpw;      // rows per tile
    uint32_t lpt;      // lanes (units) per full tile
    uint32_t qc;       // 16-byte chunks per unit
    uint32_t dg;       // f16 fields per unit
    uint32_t ntiles;
    uint64_t tile_bytes;   // bytes of a full tile
    uint64_t bytes;        // total bytes
};

inline uint32_t pi_base_elems(uint32_t t) { return (t == PI_TYPE_Q4_K || t == PI_TYPE_Q6_K) ? 256u : 32u; }
inline uint32_t pi_base_chunks(uint32_t t) {
    switch (t) {
    case PI_TYPE_Q4_K: return 9;
    case PI_TYPE_Q6_K: return 13;
    case PI_TYPE_Q4_0: return 1;
    case PI_TYPE_Q8_0: return 2;
    default: return 0;
    }
}
inline uint32_t pi_base_dfields(uint32_t t) { return t == PI_TYPE_Q4_K ? 0u : 1u; }
PI_HD inline uint64_t pi_tile_bytes(uint32_t lanes, uint32_t qc, uint32_t dg) {
    return (uint64_t)lanes * qc * 16u + (((uint64_t)lanes * dg * 2u + 15u) & ~(uint64_t)15u);
}

// Units per row: the smallest g (most units per row, at most 64) whose tiles
// keep at least 55 of 64 lanes busy, else the g with the most busy lanes.
// g is limited to the instantiated kernels: 1 for K-quants, {1,2,3,4,6,8}
// for 32-element blocks.
inline bool pi_make_layout(uint32_t type, uint32_t rows, uint32_t k, pi_layout *L) {
    if (!pi_gemv_type(type) || rows == 0 || k == 0) return false;
    uint32_t be = pi_base_elems(type);
    if (k % be) return false;
    uint32_t nbr = k / be;
    static const uint32_t gk[] = {1};
    static const uint32_t g32[] = {1, 2, 3, 4, 6, 8};
    const uint32_t *gs = (be == 256) ? gk : g32;
    uint32_t ng = (be == 256) ? 1u : 6u;
    uint32_t pick = 0, best_lanes = 0;
    for (uint32_t i = 0; i < ng; i++) {
        uint32_t g = gs[i];
        if (nbr % g || nbr / g > 64) continue;
        uint32_t upr = nbr / g, lanes = (64 / upr) * upr;
        if (lanes >= 55) { pick = g; break; }
        if (lanes > best_lanes) { best_lanes = lanes; pick = g; }
    }
    if (!pick) return false;
    L->type = type; L->k = k; L->rows = rows; L->g = pick;
    L->upr = nbr / pick;
    L->rpw = 64 / L->upr;
    L->lpt = L->rpw * L->upr;
    L->qc = pi_base_chunks(type) * pick;
    L->dg = pi_base_dfields(type) * pick;
    L->ntiles = (rows + L->rpw - 1) / L->rpw;
    L->tile_bytes = pi_tile_bytes(L->lpt, L->qc, L->dg);
    uint32_t last_rows = rows - (L->ntiles - 1) * L->rpw;
    L->bytes = (uint64_t)(L->ntiles - 1) * L->tile_bytes + pi_tile_bytes(last_rows * L->upr, L->qc, L->dg);
    return true;
}
