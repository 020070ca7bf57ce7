// Batched prefill for gfx950: up to PI_PF_MAX_TOK consecutive prompt tokens per pass.
//
// The projections run on int8 MFMA: v_mfma_i32_16x16x32_i8 forms, for a tile
// of 16 weight rows x 16 tokens, the exact int32 dot product of one
// 32-element group (Q4_K sub-block, Q4_0/Q8_0 block; Q6_K 16-element group
// with the other half of the operand zeroed).  Each (row, token) then takes
// the reference's float epilogue term by term in block order
// (quant_int.rs:281-419), so every output equals the lanes path bit for bit:
// the lanes path gives each token the same result as a batch of one
// (tests/quant_layout.rs:327-357).  The epilogue, one term per 32 weights per
// token with its own scales, is VALU work and bounds these kernels; the
// MFMA part is a small share of their time.
//
// Norms and attention follow the reference's orders for a batch of more
// than one token: scalar sum of squares (model.rs:812-822) and scalar dot
// products for the scores (1028-1038), with the value accumulation of
// simd::f32_axpy (1056-1074).
#include <hip/hip_runtime.h>

#include "pi_gemv.h"
#include "pi_prefill.h"

using namespace pig;

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ long pack2(uint32_t lo, uint32_t hi) { return (long)(((uint64_t)hi << 32) | lo); }
__device__ __forceinline__ uint32_t byte16(const uint4 &v, int i) {
    const uint32_t w = i < 4 ? v.x : (i < 8 ? v.y : (i < 12 ? v.z : v.w));
    return (w >> (8 * (i & 3))) & 0xFFu;
}

// Device view of a tiled matrix.
struct WV {
    const uint8_t *w;
    uint32_t rows, upr, rpw, lpt, g, qc, ntiles;
    uint32_t gmag;        // ceil(2^32 / g) for g > 1: u / g == umulhi(u, gmag) for u < 2^16
    uint64_t tile_bytes;
};
__device__ __forceinline__ uint32_t div_g(const WV &W, uint32_t u) { return W.g == 1 ? u : __umulhi(u, W.gmag); }

__device__ __forceinline__ uint4 ld16(const uint8_t *p) { return *gld(reinterpret_cast<const uint4 *>(p)); }

__device__ __forceinline__ v4i mfma16(long a, long b) {
    v4i c = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// GEMM.  A workgroup of four wavefronts owns 16 rows of one matrix and 64
// tokens of the pass; wavefront w serves tokens 16w..16w+15 of them.  Every
// (row, token) output is 0 + t_0 + t_1 + ... in the reference's term order
// (one term per 32-element group; Q6_K one per 16-element group in
// (half, g, s) order).  Each term is one int8 MFMA (lane l: A row
// r0 + l%16 with group elements 8*(l/16)..+7; B token l%16; D rows
// 4*(l/16)+i) and the float term per pair, added at once to the pair's sum
// in a register: a lane keeps the sums of rows 4*(l/16)..+3 for its token.
// The weight chunks of a phase of 16 terms are staged into LDS by the whole
// workgroup (whole 16-byte chunks, one phase ahead, two buffers: one barrier
// per phase) and read by all four wavefronts; the activation operands of the
// next kPfActDepth terms are in flight in registers; the per-row constants
// of the terms (f16 scales, 6-bit sub-block scales/mins, Q6_K d*scale) are
// decoded once into LDS.
// ---------------------------------------------------------------------------
constexpr uint32_t kPfRows = 16;
constexpr uint32_t kPfThreads = 256;
constexpr uint32_t kPfPhase = 16;                   // terms per row per phase
constexpr uint32_t kPfTokWg = 64;                   // tokens per workgroup
constexpr uint32_t kPfActDepth = 8;                 // terms whose activation operands are in flight
constexpr uint32_t kPfMaxSeg = 3;
static_assert(kPfPhase % kPfActDepth == 0, "the operand ring index is static within a phase");

// Row r of a tiled matrix: its tile, the tile's lane count and the lane of
// the row's first unit.
struct RowPos {
    const uint8_t *tile;
    uint32_t lanes, ln0;
};
__device__ __forceinline__ RowPos row_pos(const WV &W, uint32_t r) {
    const uint32_t t = r / W.rpw, rt = r - t * W.rpw;
    RowPos p;
    p.tile = W.w + (uint64_t)t * W.tile_bytes;
    p.lanes = (t == W.ntiles - 1) ? (W.rows - t * W.rpw) * W.upr : W.lpt;
    p.ln0 = rt * W.upr;
    return p;
}

struct PfSegs {
    WV W[kPfMaxSeg];
    float *out[kPfMaxSeg];
    uint32_t wg_end[kPfMaxSeg];   // cumulative workgroup counts
    uint32_t mode[kPfMaxSeg];     // pi_pf_out
    uint32_t nseg;
    pi_pf_rope rope;
};

// Offset of the 8 quants 8*ka..+7 of group G of token t in a prefill Q8 buffer.
__device__ __forceinline__ uint64_t pfq_off(uint32_t G, uint32_t ka, uint32_t t) {
    return (((uint64_t)G * 4 + ka) * PI_PF_MAX_TOK + t) * 8;
}
// Stores the Q8 of half hh of block b of token t (q8_pair_core results).
__device__ __forceinline__ void pf_store_pair(pi_pf_q8 o, uint32_t t, uint32_t b, uint32_t hh, const uint32_t (&w4)[4],
                                              float dd, int sum) {
    *reinterpret_cast<uint2 *>(o.q + pfq_off(b, 2 * hh, t)) = make_uint2(w4[0], w4[1]);
    *reinterpret_cast<uint2 *>(o.q + pfq_off(b, 2 * hh + 1, t)) = make_uint2(w4[2], w4[3]);
    if (hh == 0) {
        o.d[b * PI_PF_MAX_TOK + t] = dd;
        o.s[b * PI_PF_MAX_TOK + t] = sum;
    }
}
__device__ __forceinline__ float f4(const float4 &v, int i) { return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w)); }

template <uint32_t T>
struct PfLds;
// Q4_K: d, dmin per (block, row); s, m per (block, sub-block, row).
template <>
struct PfLds<PI_TYPE_Q4_K> {
    static constexpr uint32_t floats_per_block = 16 * 2 + 8 * 16 * 2;
};
// Q6_K: d * scale per (block, 16-group, row).
template <>
struct PfLds<PI_TYPE_Q6_K> {
    static constexpr uint32_t floats_per_block = 16 * 16;
};
// Q4_0 / Q8_0: d per (block, row).
template <>
struct PfLds<PI_TYPE_Q4_0> {
    static constexpr uint32_t floats_per_block = 16;
};
template <>
struct PfLds<PI_TYPE_Q8_0> {
    static constexpr uint32_t floats_per_block = 16;
};

// Decodes the epilogue constants of rows r0..r0+15 into cst (all loads of a
// round are issued before any is used).
template <uint32_t T>
__device__ __forceinline__ void decode_consts(const WV &W, uint32_t r0, uint32_t nb, float *cst) {
    constexpr uint32_t R = (T == PI_TYPE_Q4_K || T == PI_TYPE_Q6_K) ? 2u : 12u;   // entries per thread per round
    const uint32_t tid = threadIdx.x, ne = nb * kPfRows;
    for (uint32_t base = 0; base < ne; base += kPfThreads * R) {
        if constexpr (T == PI_TYPE_Q4_K || T == PI_TYPE_Q6_K) {
            uint4 h[R];
            float dv[R];
#pragma unroll
            for (uint32_t j = 0; j < R; j++) {
                const uint32_t p = min(base + tid + kPfThreads * j, ne - 1), i = p % kPfRows, u = p / kPfRows;
                const RowPos rp = row_pos(W, min(r0 + i, W.rows - 1));
                if constexpr (T == PI_TYPE_Q4_K) {
                    h[j] = ld16(rp.tile + (uint64_t)(rp.ln0 + u) * 16u);
                } else {
                    h[j] = ld16(rp.tile + (uint64_t)(12u * rp.lanes + rp.ln0 + u) * 16u);
                    dv[j] = h2f(*gld(reinterpret_cast<const uint16_t *>(rp.tile + (uint64_t)rp.lanes * W.qc * 16u +
                                                                        (uint64_t)(rp.ln0 + u) * 2u)));
                }
            }
#pragma unroll
            for (uint32_t j = 0; j < R; j++) {
                const uint32_t p = base + tid + kPfThreads * j;
                if (p >= ne) break;
                const uint32_t i = p % kPfRows, u = p / kPfRows;
                float *c = cst + (uint64_t)u * PfLds<T>::floats_per_block;
                if constexpr (T == PI_TYPE_Q4_K) {
                    c[i] = h2f(h[j].x);
                    c[16 + i] = h2f(h[j].x >> 16);
#pragma unroll
                    for (int sb = 0; sb < 8; sb++) {
                        uint32_t sv, mv;   // get_scale_min_k4 on the 12 scale bytes (bytes 4..15)
                        if (sb < 4) {
                            sv = byte16(h[j], 4 + sb) & 63u;
                            mv = byte16(h[j], 4 + sb + 4) & 63u;
                        } else {
                            sv = (byte16(h[j], 4 + sb + 4) & 0xFu) | ((byte16(h[j], 4 + sb - 4) >> 6) << 4);
                            mv = (byte16(h[j], 4 + sb + 4) >> 4) | ((byte16(h[j], 4 + sb) >> 6) << 4);
                        }
                        c[32 + sb * 16 + i] = (float)sv;
                        c[32 + 128 + sb * 16 + i] = (float)mv;
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < 16; q++) c[q * 16 + i] = dv[j] * (float)(int8_t)byte16(h[j], q);
                }
            }
        } else {
            uint32_t hv[R];
#pragma unroll
            for (uint32_t j = 0; j < R; j++) {
                const uint32_t p = min(base + tid + kPfThreads * j, ne - 1), i = p % kPfRows, u = p / kPfRows;
                const RowPos rp = row_pos(W, min(r0 + i, W.rows - 1));
                const uint32_t unit = div_g(W, u), b = u - unit * W.g;
                hv[j] = *gld(reinterpret_cast<const uint16_t *>(rp.tile + (uint64_t)rp.lanes * W.qc * 16u +
                                                                (uint64_t)(b * rp.lanes + rp.ln0 + unit) * 2u));
            }
#pragma unroll
            for (uint32_t j = 0; j < R; j++) {
                const uint32_t p = base + tid + kPfThreads * j;
                if (p >= ne) break;
                cst[(p / kPfRows) * PfLds<T>::floats_per_block + p % kPfRows] = h2f(hv[j]);
            }
        }
    }
}

// Runs use(buffer, i) for i = 0..n-1 in order with the loads of the next
// P - 1 steps in flight: P buffers in registers, the inner loop unrolled so
// each keeps its registers; loads past the end repeat step n - 1.  middle()
// runs after the first P loads are issued; its false return ends the run.
template <int P, typename L, typename U, typename M>
__device__ __forceinline__ void ring_run(uint32_t n, L &&load, U &&use, M &&middle) {
    using Buf = decltype(load(0u));
    Buf R[P];
#pragma unroll
    for (int k = 0; k < P; k++) R[k] = load(min((uint32_t)k, n - 1));
    if (!middle()) return;
    for (uint32_t i0 = 0; i0 < n; i0 += P) {
#pragma unroll
        for (int k = 0; k < P; k++) {
            if (i0 + k < n) {
                use(R[k], i0 + k);
                R[k] = load(min(i0 + k + P, n - 1));
            }
        }
    }
}

// Weight chunks staged per phase (16-byte pieces): blocks per phase, pieces
// per row and the LDS row stride in pieces (odd multiples of 4 dwords keep
// the 16 rows of an MFMA read on distinct banks).
template <uint32_t T> struct PfStage;
template <> struct PfStage<PI_TYPE_Q4_K> { static constexpr uint32_t PB = 2, PPR = 16, WS = 17; };   // qs chunks 1..8
template <> struct PfStage<PI_TYPE_Q6_K> { static constexpr uint32_t PB = 1, PPR = 12, WS = 13; };   // ql, qh chunks 0..11
template <> struct PfStage<PI_TYPE_Q8_0> { static constexpr uint32_t PB = 16, PPR = 32, WS = 33; };
template <> struct PfStage<PI_TYPE_Q4_0> { static constexpr uint32_t PB = 16, PPR = 16, WS = 17; };

// Activation operands of one term for one lane.
struct TermAct {
    uint2 b;   // 8 activation quants
    float da;
    int as;
};

template <uint32_t T>
__global__ __launch_bounds__(kPfThreads) __attribute__((amdgpu_waves_per_eu(4))) void k_pf_gemm(PfSegs S, const int8_t *__restrict__ aq,
                                                         const float *__restrict__ ad, const int32_t *__restrict__ as,
                                                         uint32_t k, uint32_t ntok, int resid) {
    using ST = PfStage<T>;
    constexpr uint32_t PIECES = kPfRows * ST::PPR;                       // per phase
    constexpr uint32_t PPT = (PIECES + kPfThreads - 1) / kPfThreads;    // pieces per thread
    extern __shared__ __align__(16) float lds[];
    const uint32_t wg = blockIdx.x;
    const uint32_t seg = (S.nseg > 1 && wg >= S.wg_end[0]) ? ((S.nseg > 2 && wg >= S.wg_end[1]) ? 2u : 1u) : 0u;
    const WV W = seg == 0 ? S.W[0] : (seg == 1 ? S.W[1] : S.W[2]);
    float *const out = seg == 0 ? S.out[0] : (seg == 1 ? S.out[1] : S.out[2]);
    const uint32_t mode = seg == 0 ? S.mode[0] : (seg == 1 ? S.mode[1] : S.mode[2]);
    const uint32_t wg0 = seg == 0 ? 0u : (seg == 1 ? S.wg_end[0] : S.wg_end[1]);
    const uint32_t ntb = (ntok + kPfTokWg - 1) / kPfTokWg;
    const uint32_t rg = (wg - wg0) / ntb, tb = (wg - wg0) - rg * ntb;
    const uint32_t r0 = rg * kPfRows;
    const uint32_t tid = threadIdx.x, w = tid >> 6, lane = tid & 63u;
    const uint32_t ka = lane >> 4, li = lane & 15u;
    constexpr bool KQ = T == PI_TYPE_Q4_K || T == PI_TYPE_Q6_K;
    const uint32_t nb = k / (KQ ? 256u : 32u);
    const uint32_t tpr = T == PI_TYPE_Q6_K ? 16 * nb : (T == PI_TYPE_Q4_K ? 8 * nb : nb);   // terms per row
    const uint32_t nph = (tpr + kPfPhase - 1) / kPfPhase;
    float *cst = lds;
    uint4 *wb0 = reinterpret_cast<uint4 *>(lds + (((uint64_t)nb * PfLds<T>::floats_per_block + 3) & ~3ull));
    uint4 *wb1 = wb0 + kPfRows * ST::WS;

    // ---- staging: this thread's pieces -----------------------------------
    struct Piece {
        const uint8_t *tile;
        uint32_t lanes, ln0, q;   // q: piece index within a phase (PIECES: none)
    };
    Piece pc[PPT];
#pragma unroll
    for (uint32_t j = 0; j < PPT; j++) {
        const uint32_t q = tid + kPfThreads * j;
        const uint32_t i = min(q / ST::PPR, kPfRows - 1);
        const RowPos rp = row_pos(W, min(r0 + i, W.rows - 1));
        pc[j] = Piece{rp.tile, rp.lanes, rp.ln0, q < PIECES ? q : PIECES};
    }
    struct Staged {
        uint4 v[PPT];
    };
    auto load_pieces = [&](uint32_t ph) {
        Staged R;
#pragma unroll
        for (uint32_t j = 0; j < PPT; j++) {
            const Piece &P = pc[j];
            const uint32_t q = min(P.q, PIECES - 1), r = q % ST::PPR;
            uint64_t off;
            if constexpr (T == PI_TYPE_Q4_K) {
                const uint32_t c = r >> 1, v = r & 1u, u = min(ph * ST::PB + v, nb - 1);
                off = (uint64_t)((1u + c) * P.lanes + P.ln0 + u) * 16u;
            } else if constexpr (T == PI_TYPE_Q6_K) {
                off = (uint64_t)(r * P.lanes + P.ln0 + min(ph * ST::PB, nb - 1)) * 16u;
            } else {
                constexpr uint32_t BC = T == PI_TYPE_Q8_0 ? 2u : 1u;
                const uint32_t v = r / BC, jc = r - v * BC, u = min(ph * ST::PB + v, nb - 1);
                const uint32_t unit = div_g(W, u), b = u - unit * W.g;
                off = (uint64_t)((b * BC + jc) * P.lanes + P.ln0 + unit) * 16u;
            }
            R.v[j] = *gld(reinterpret_cast<const uint4 *>(P.tile + off));
        }
        return R;
    };
    auto store_pieces = [&](const Staged &R, uint4 *wb) {
#pragma unroll
        for (uint32_t j = 0; j < PPT; j++)
            if (pc[j].q < PIECES) wb[(pc[j].q / ST::PPR) * ST::WS + pc[j].q % ST::PPR] = R.v[j];
    };

    // ---- activation operands -----------------------------------------------
    // this lane's MFMA token; lanes past the pass read the last token's operands
    const uint32_t n = tb * kPfTokWg + w * 16 + li, nc = min(n, ntok - 1);
    auto act_group = [&](uint32_t tg) -> uint32_t {
        if constexpr (T == PI_TYPE_Q6_K) return (tg >> 4) * 8 + 4 * ((tg >> 3) & 1u) + (tg & 3u);
        else return tg;
    };
    auto load_act = [&](uint32_t tg) {
        const uint32_t a = act_group(min(tg, tpr - 1));
        TermAct X;
        X.b = *gld(reinterpret_cast<const uint2 *>(aq + pfq_off(a, ka, nc)));
        X.da = *gld(ad + a * PI_PF_MAX_TOK + nc);
        X.as = 0;
        if constexpr (T == PI_TYPE_Q4_K || T == PI_TYPE_Q4_0) X.as = *gld(as + a * PI_PF_MAX_TOK + nc);
        return X;
    };

    // the 4 terms of rows 4*ka..4*ka+3 for this lane's token
    auto term4 = [&](const TermAct &X, const uint4 *wb, uint32_t ph, uint32_t tg, float (&t)[4]) {
        const long B = pack2(X.b.x, X.b.y);
        const uint8_t *wrow = reinterpret_cast<const uint8_t *>(wb + li * ST::WS) + 8u * (ka & 1u);
        if constexpr (T == PI_TYPE_Q4_K) {
            const uint32_t u = tg >> 3, sb = tg & 7u, v = u - ph * ST::PB;
            const uint2 a = *reinterpret_cast<const uint2 *>(wrow + ((2u * (sb >> 1) + (ka >> 1)) * 2u + v) * 16u);
            const uint32_t sh = (sb & 1u) * 4u;
            const v4i cc = mfma16(pack2((a.x >> sh) & 0x0F0F0F0Fu, (a.y >> sh) & 0x0F0F0F0Fu), B);
            const float *c = cst + (uint64_t)u * PfLds<T>::floats_per_block;
            const float4 d4 = reinterpret_cast<const float4 *>(c)[ka];
            const float4 dm4 = reinterpret_cast<const float4 *>(c + 16)[ka];
            const float4 s4 = reinterpret_cast<const float4 *>(c + 32 + sb * 16)[ka];
            const float4 m4 = reinterpret_cast<const float4 *>(c + 160 + sb * 16)[ka];
            const float asf = (float)X.as;
#pragma unroll
            for (int i = 0; i < 4; i++)
                t[i] = f4(d4, i) * X.da * f4(s4, i) * (float)cc[i] - X.da * f4(dm4, i) * f4(m4, i) * asf;
        } else if constexpr (T == PI_TYPE_Q6_K) {
            const uint32_t u = tg >> 4, half = (tg >> 3) & 1u, g = (tg >> 2) & 1u, s = tg & 3u;
            const uint2 ql = *reinterpret_cast<const uint2 *>(wrow + (half * 4 + 2 * (s & 1u) + (ka >> 1)) * 16u);
            const uint2 qh = *reinterpret_cast<const uint2 *>(wrow + (8 + half * 2 + (ka >> 1)) * 16u);
            const bool mine = (ka >> 1) == g;   // this lane's 8 elements are in 16-group g
            uint32_t w6[2];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const uint32_t l4 = e ? ql.y : ql.x, h2 = e ? qh.y : qh.x;
                const uint32_t nib = s < 2 ? (l4 & 0x0F0F0F0Fu) : ((l4 >> 4) & 0x0F0F0F0Fu);
                const uint32_t q = nib | (((h2 >> (2 * s)) & 0x03030303u) << 4);   // 0..63 per byte
                const uint32_t x = q ^ 0x20202020u;                               // q - 32 in 6 bits
                w6[e] = x | ((x & 0x20202020u) * 6u);                              // sign-extend to 8
            }
            const v4i cc = mfma16(mine ? pack2(w6[0], w6[1]) : 0L, B);
            const float4 ds4 =
                reinterpret_cast<const float4 *>(cst + (uint64_t)u * PfLds<T>::floats_per_block + (half * 8 + g + 2 * s) * 16)[ka];
#pragma unroll
            for (int i = 0; i < 4; i++) t[i] = f4(ds4, i) * X.da * (float)cc[i];
        } else {
            const uint32_t v = tg - ph * ST::PB;
            long A;
            if constexpr (T == PI_TYPE_Q8_0) {
                const uint2 a = *reinterpret_cast<const uint2 *>(wrow + (v * 2u + (ka >> 1)) * 16u);
                A = pack2(a.x, a.y);
            } else {
                const uint2 a = *reinterpret_cast<const uint2 *>(wrow + v * 16u);
                const uint32_t sh = (ka >> 1) * 4u;
                A = pack2((a.x >> sh) & 0x0F0F0F0Fu, (a.y >> sh) & 0x0F0F0F0Fu);
            }
            const v4i cc = mfma16(A, B);
            const float4 d4 = reinterpret_cast<const float4 *>(cst + (uint64_t)tg * PfLds<T>::floats_per_block)[ka];
            if constexpr (T == PI_TYPE_Q8_0) {
#pragma unroll
                for (int i = 0; i < 4; i++) t[i] = f4(d4, i) * X.da * (float)cc[i];
            } else {
                const float asf = (float)X.as;
#pragma unroll
                for (int i = 0; i < 4; i++) t[i] = f4(d4, i) * X.da * ((float)cc[i] - 8.0f * asf);
            }
        }
    };

    // ---- phases ---------------------------------------------------------------
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    TermAct R[kPfActDepth];
    Staged SW = load_pieces(0);
#pragma unroll
    for (uint32_t j = 0; j < kPfActDepth; j++) R[j] = load_act(j);
    decode_consts<T>(W, r0, nb, cst);
    store_pieces(SW, wb0);
    SW = load_pieces(min(1u, nph - 1));
    __syncthreads();
    auto step = [&](const uint4 *wb, uint32_t ph, uint32_t tg, TermAct &X) {
        float t[4];
        term4(X, wb, ph, tg, t);
        X = load_act(tg + kPfActDepth);
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = acc[i] + t[i];
        // Q6_K, Q8_0: the sums are pinned after each term, which keeps the
        // compiler from forming all 16 MFMAs of a phase ahead of their terms
        // (more wavefronts per SIMD fit); Q4_K and Q4_0 run faster with them
        // formed ahead within the 128-register budget (measured).
        if constexpr (T != PI_TYPE_Q4_K && T != PI_TYPE_Q4_0) asm volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]));
    };
    for (uint32_t ph = 0; ph < nph; ph++) {
        const uint4 *wb = (ph & 1u) ? wb1 : wb0;
        const uint32_t tg0 = ph * kPfPhase;
        if (tg0 + kPfPhase <= tpr) {
#pragma unroll
            for (uint32_t j = 0; j < kPfPhase; j++) step(wb, ph, tg0 + j, R[j % kPfActDepth]);
        } else {
#pragma unroll
            for (uint32_t j = 0; j < kPfPhase; j++)
                if (tg0 + j < tpr) step(wb, ph, tg0 + j, R[j % kPfActDepth]);
        }
        if (ph + 1 < nph) store_pieces(SW, (ph & 1u) ? wb0 : wb1);
        SW = load_pieces(min(ph + 2, nph - 1));
        __syncthreads();
    }
    if (n >= ntok) return;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = 0.0f + acc[i];
    if (mode == PI_PF_STORE) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t r = r0 + 4 * ka + i;
            if (r < W.rows) {
                float *o = out + (uint64_t)n * W.rows + r;
                *o = resid ? *o + v[i] : v[i];
            }
        }
        return;
    }
    // Rows of 64-dimension heads (rows a multiple of 64): this lane holds
    // dimensions d..d+3 of head rr / 64 for token n at position pos.
    const uint32_t rr = r0 + 4 * ka, d = rr % 64, pos = S.rope.pos0 + n;
    if (mode != PI_PF_CACHE) {
        // RoPE of the pairs (d, d+1), (d+2, d+3) (model.rs:953-979)
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const uint32_t p = d / 2 + q;
            if (p < S.rope.half) {
                const float c = S.rope.cos_tab[(uint64_t)pos * S.rope.half + p];
                const float sn = S.rope.sin_tab[(uint64_t)pos * S.rope.half + p];
                const float x0 = v[2 * q], x1 = v[2 * q + 1];
                v[2 * q] = x0 * c - x1 * sn;
                v[2 * q + 1] = x0 * sn + x1 * c;
            }
        }
    }
    float *o = mode == PI_PF_ROPE ? out + (uint64_t)n * W.rows + rr
                                  : out + ((uint64_t)(rr / 64) * S.rope.n_ctx + pos) * 64 + d;   // cache row (984-992)
    *reinterpret_cast<float4 *>(o) = make_float4(v[0], v[1], v[2], v[3]);
}

// ---------------------------------------------------------------------------
// Embedding rows of the pass.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_pf_embed(const uint8_t *__restrict__ E, uint32_t etype, uint64_t row_bytes,
                                                  const uint32_t *__restrict__ ids, uint32_t ne, float *__restrict__ X) {
    const uint32_t t = blockIdx.x;
    const uint8_t *row = E + (uint64_t)ids[t] * row_bytes;
    for (uint32_t e = threadIdx.x; e < ne; e += blockDim.x) X[(uint64_t)t * ne + e] = embed_elem(row, etype, e);
}

// ---------------------------------------------------------------------------
// RMSNorm (scalar order) + Q8 of up to four tokens per workgroup.  The rows
// and their squares are staged in LDS (the squares padded by floats the chain
// reads ahead); lane 0 of wavefront j adds token j's squares in order, so the
// tokens' add chains run on different SIMDs instead of queueing on one; pairs
// of lanes then quantize half a block each.
// ---------------------------------------------------------------------------
constexpr uint32_t kNormPad = 128;   // floats the chain reads past the row (2 x 16 float4)
__host__ __device__ constexpr uint32_t pf_norm_region(uint32_t ne) { return 2 * ne + 2 * kNormPad; }

__global__ __launch_bounds__(256) void k_pf_norm_q8(const float *__restrict__ X, const float *__restrict__ w,
                                                    uint32_t ne, float eps, uint32_t ntok, uint32_t tpb, pi_pf_q8 o) {
    extern __shared__ __align__(16) float xs[];
    __shared__ float sv[4];
    const uint32_t tid = threadIdx.x, nb = ne / 32, t0 = blockIdx.x * tpb, nt = min(tpb, ntok - t0);
    const uint32_t region = pf_norm_region(ne), n4 = ne / 4;
    // rows of tokens t0 .. t0 + nt - 1: a thread's 8 loads are issued before its stores
    for (uint32_t base = 0; base < nt * n4; base += 256 * 8) {
        float4 v[8];
#pragma unroll
        for (uint32_t i = 0; i < 8; i++) {
            const uint32_t q = min(base + tid + 256 * i, nt * n4 - 1), j = q / n4;
            v[i] = reinterpret_cast<const float4 *>(X + (uint64_t)(t0 + j) * ne)[q - j * n4];
        }
#pragma unroll
        for (uint32_t i = 0; i < 8; i++) {
            const uint32_t q = base + tid + 256 * i, j = q / n4;
            if (q < nt * n4) {
                float *r = xs + j * region;
                reinterpret_cast<float4 *>(r)[q - j * n4] = v[i];
                reinterpret_cast<float4 *>(r + ne + kNormPad)[q - j * n4] =
                    make_float4(v[i].x * v[i].x, v[i].y * v[i].y, v[i].z * v[i].z, v[i].w * v[i].w);
            }
        }
    }
    for (uint32_t i = tid; i < nt * kNormPad; i += 256) xs[(i / kNormPad) * region + 2 * ne + kNormPad + i % kNormPad] = 0.0f;
    __syncthreads();
    const uint32_t wave = tid >> 6;
    if ((tid & 63u) == 0 && wave < nt) {
        // ss += v * v in order (model.rs:812-822): the products are formed above
        float ss = 0.0f;
        lds_chain4<16>(reinterpret_cast<const float4 *>(xs + wave * region + ne + kNormPad), n4, [&](const float4 &q) {
            ss += q.x;
            ss += q.y;
            ss += q.z;
            ss += q.w;
        });
        sv[wave] = 1.0f / sqrtf(ss / (float)ne + eps);
    }
    __syncthreads();
    for (uint32_t p = tid; p < nt * 2 * nb; p += blockDim.x) {   // pairs of lanes stay together
        const uint32_t j = p / (2 * nb), pp = p - j * 2 * nb, b = pp >> 1, hh = pp & 1u;
        const float sc = sv[j];
        const float4 *xv = reinterpret_cast<const float4 *>(xs + j * region + 16 * pp);
        const float4 *wv = reinterpret_cast<const float4 *>(w + 16 * pp);
        float v[16];
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            const float4 xx = xv[jj], ww = wv[jj];
            v[4 * jj + 0] = xx.x * sc * ww.x;
            v[4 * jj + 1] = xx.y * sc * ww.y;
            v[4 * jj + 2] = xx.z * sc * ww.z;
            v[4 * jj + 3] = xx.w * sc * ww.w;
        }
        uint32_t w4[4];
        float dd;
        int sum;
        q8_pair_core(v, w4, dd, sum);
        pf_store_pair(o, t0 + j, b, hh, w4, dd, sum);
    }
}

// ---------------------------------------------------------------------------
// h = silu(gate) * up, then Q8 of h: a lane per 4 elements, 8 consecutive
// lanes per 32-element block (the block's maximum and quant sum reduced over
// the 8 lanes with DPP; both are exact in any order).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_pf_swiglu_q8(const float *__restrict__ G, const float *__restrict__ U,
                                                      uint32_t n_ff, pi_pf_q8 o) {
    const uint32_t t = blockIdx.x, nq = n_ff / 4;
    const uint32_t q = blockIdx.y * blockDim.x + threadIdx.x;
    if (q >= nq) return;   // nq is a multiple of 8 and so is every workgroup: blocks stay whole
    const float4 gg = reinterpret_cast<const float4 *>(G + (uint64_t)t * n_ff)[q];
    const float4 uu = reinterpret_cast<const float4 *>(U + (uint64_t)t * n_ff)[q];
    const float ga[4] = {gg.x, gg.y, gg.z, gg.w}, ua[4] = {uu.x, uu.y, uu.z, uu.w};
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float sg = ga[e] / (1.0f + pi_expf(-ga[e]));
        v[e] = sg * ua[e];
    }
    // Q8 of the block (quant_int.rs:33-55): amax ignores NaN, d = amax / 127,
    // inv = 1 / d, roundf half away from zero, clamped
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    amax = fmaxf(amax, dpp<kDppXor1>(amax));
    amax = fmaxf(amax, dpp<kDppXor2>(amax));
    amax = fmaxf(amax, dpp<kDppHalfMirror>(amax));
    amax = fmaxf(amax, 0.0f);   // all-NaN block: 0
    const float dd = amax / 127.0f;
    const float inv = dd > 0.0f ? 1.0f / dd : 0.0f;
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) word |= ((uint32_t)q8_round_clamp(v[e] * inv) & 0xFFu) << (8 * e);
    int sum = sdot4((int)word, 0x01010101, 0);
    sum += dpp<kDppXor1>(sum);
    sum += dpp<kDppXor2>(sum);
    sum += dpp<kDppHalfMirror>(sum);
    const uint32_t b = q / 8, k = q % 8;   // block, quad within the block
    *reinterpret_cast<uint32_t *>(o.q + pfq_off(b, k / 2, t) + 4 * (k & 1u)) = word;
    if (k == 0) {
        o.d[b * PI_PF_MAX_TOK + t] = dd;
        o.s[b * PI_PF_MAX_TOK + t] = sum;
    }
}

// ---------------------------------------------------------------------------
// Attention: a workgroup serves 4 * TPW consecutive tokens of one head with 5
// wavefronts; wavefront w (0-3) serves tokens TPW*w..TPW*w+TPW-1 of them.
// K, then V, rows are staged through two LDS buffers 64 positions per step
// by wavefronts 0-3, each step's rows loaded into registers one step ahead
// (one barrier per step); every staged row feeds the chains of all the
// workgroup's tokens.  96 registers per lane and under 40 KB of LDS per
// workgroup keep five wavefronts per SIMD (four workgroups per CU), whose
// steps hide each other's load latency better than a second step in flight
// would.
// Pass 1, scores (model.rs:1028-1038, scalar dot in d order, * scale): lane
// = position, one chain per token of the wavefront, q of the wavefront's
// tokens in scalar registers (loaded from Q, so the LDS serves only K); each
// score goes to the token's row of a score scratch in global memory, and the
// maximum is kept.
// Pass 2, per step: the wavefront reads its tokens' scores back (loaded two
// steps ahead), forms e_p = exp(s_p - max) lane-parallel (into an LDS step
// buffer; a full step reads a quarter of its e_p from their lanes into
// scalar registers instead), then adds e_p * v_p[d] in position order
// (f32_axpy order, model.rs:1056-1074: products rounded, e_p == 0 skipped),
// lane = dimension, one chain per token, from the transposed V step; lane i
// of wavefront 4 adds sum += e_p of token i in position order, one step
// behind.  V is staged as blocks of 4 positions x 4 dimensions per thread,
// transposed in registers, so its LDS writes are 16 bytes wide and free of
// bank conflicts.
// Output acc * (1/sum), then Q8 of the head's 64 values.
// ---------------------------------------------------------------------------
constexpr uint32_t kAttStep = 64;               // positions per staged step
constexpr uint32_t kAttThreads = 320;
constexpr uint32_t kAttTpw = 2;                 // tokens per wavefront
constexpr uint32_t kAttTok = 4 * kAttTpw;       // tokens per workgroup
constexpr uint32_t kKRow = 68;                  // floats per staged K row
constexpr uint32_t kVRow = kAttStep + 4;        // floats per staged transposed V row
constexpr uint32_t kAttBuf = kAttStep * kKRow;  // floats per staging buffer (>= 64 * kVRow)
constexpr uint32_t kAttLaneE = 32;              // e of a full value step read from lanes (of TPW * 64)
static_assert(kAttBuf >= 64 * kVRow, "staging buffer holds a transposed V step");
static_assert(kAttTok <= 64, "wavefront 4 holds one token per lane");

// Parts per head in the attention's XCD assignment: 8 / gcd(n_head, 8).
__host__ __device__ constexpr uint32_t pf_att_parts(uint32_t n_head) {
    return (n_head % 8 == 0) ? 1u : (n_head % 4 == 0 ? 2u : (n_head % 2 == 0 ? 4u : 8u));
}

template <uint32_t TPW>
__global__ __launch_bounds__(kAttThreads) __attribute__((amdgpu_waves_per_eu(5))) void k_pf_attn(const float *__restrict__ Q, const float *__restrict__ kc,
                                                         const float *__restrict__ vc, uint32_t pos0, uint32_t ntok,
                                                         uint32_t n_head, uint32_t group, uint32_t n_ctx, float scale,
                                                         float *__restrict__ scr, int8_t *__restrict__ oq,
                                                         float *__restrict__ od, int32_t *__restrict__ os) {
    constexpr uint32_t DH = 64, TW = 4 * TPW;
    __shared__ __align__(16) float lds[2 * kAttBuf + 2 * TW * kAttStep];
    float *const buf0 = lds, *const buf1 = lds + kAttBuf;
    float *eb = lds + 2 * kAttBuf;              // [2][TW][64]: e of a step per token, two steps alternating
    // per-token sums and the non-finite-V flags live in the staging rows'
    // padding (column 64 of buf0's rows 0..7 and 8..8+TW), which no step reads
    // or writes
    static_assert(kKRow == kVRow && kKRow > 64 && 8 + TW <= kAttStep, "flags and sums fit the row padding");
    auto misc_at = [&](uint32_t i) -> float & { return buf0[(8u + i) * kKRow + 64u]; };
    auto vbad_at = [&](uint32_t i) -> uint32_t & { return reinterpret_cast<uint32_t *>(buf0)[i * kKRow + 64u]; };
    // Workgroup b runs on XCD b % 8 (round-robin dispatch).  The token groups
    // of a head are split into P interleaved parts (tg % P), P = 8 / gcd(n_head,
    // 8), so the n_head * P units (head, part) divide evenly over the 8 XCDs:
    // unit u goes to XCD u % 8, and a head's K/V rows are read into P L2s.
    // Within an XCD the units advance together, the last token groups (the
    // most positions) first, so the workgroups that start last are the short
    // ones.
    const uint32_t ntg = (ntok + TW - 1) / TW, xcd = blockIdx.x & 7u, r = blockIdx.x >> 3;
    const uint32_t P = pf_att_parts(n_head), nu = (n_head * P - xcd + 7) / 8;   // units of this XCD
    const uint32_t u = xcd + 8 * (r % nu), level = r / nu, part = u % P, h = u / P;
    const uint32_t cnt = (ntg - part + P - 1) / P;   // token groups part, part + P, ... below ntg
    if (level >= cnt) return;   // before any barrier: the whole workgroup leaves
    const uint32_t tg = part + P * (cnt - 1 - level);
    const uint32_t tid = threadIdx.x, w = tid >> 6, lane = tid & 63u;
    const bool stager = w < 4;
    const uint32_t t0 = tg * TW + (w & 3u) * TPW;   // first token of this wavefront
    const uint32_t n_all = pos0 + min(tg * TW + TW - 1, ntok - 1) + 1;
    const uint32_t nsteps = (n_all + kAttStep - 1) / kAttStep;
    const uint32_t kvh = h / group, qdim = n_head * DH;
    const float *kbase = kc + (uint64_t)kvh * n_ctx * DH, *vbase = vc + (uint64_t)kvh * n_ctx * DH;
    // tokens of this wavefront: valid ones are a prefix (consecutive tokens)
    uint32_t nv = 0;
    if (w < 4 && t0 < ntok) nv = min(TPW, ntok - t0);
    const uint32_t pos_last = pos0 + t0 + (nv ? nv - 1 : 0);   // position of the wavefront's last valid token
    // the tokens' scores; rows are whole 128-byte lines apart, so no other
    // wavefront touches a line of these rows
    auto srow = [&](uint32_t j) {
        return scr + ((uint64_t)min(t0 + j, ntok - 1) * n_head + h) * pi_pf_score_stride(n_ctx);
    };

    struct Rows {
        float4 v[4];
    };
    // K (wavefronts 0-3): row tid / 4 of the step, float4 columns 4*(tid%4)..+3.
    // V: positions 4*(tid%16)..+3, float4 column tid/16.  Rows of wavefront 4
    // are a clamped in-bounds copy of row 0 (never stored).
    auto load_k = [&](uint32_t c) -> Rows {
        const uint32_t p = stager ? min(c * kAttStep + (tid >> 2), n_all - 1) : 0u;
        const float4 *src = reinterpret_cast<const float4 *>(kbase + (uint64_t)p * DH) + (stager ? (tid & 3u) * 4u : 0u);
        Rows R;
#pragma unroll
        for (int j = 0; j < 4; j++) R.v[j] = src[j];
        return R;
    };
    auto load_v = [&](uint32_t c) -> Rows {
        const uint32_t rb = tid & 15u, cb = stager ? tid >> 4 : 0u;
        Rows R;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t p = stager ? min(c * kAttStep + 4 * rb + j, n_all - 1) : 0u;
            R.v[j] = reinterpret_cast<const float4 *>(vbase + (uint64_t)p * DH)[cb];
        }
        return R;
    };
    auto store_k = [&](const Rows R, float *bf) {
        if (!stager) return;
        const uint32_t srw = tid >> 2, sf = (tid & 3u) * 4u;
#pragma unroll
        for (int j = 0; j < 4; j++) reinterpret_cast<float4 *>(bf + srw * kKRow)[sf + j] = R.v[j];
    };
    auto store_vt = [&](const Rows R, float *bf) {
        if (!stager) return;
        const uint32_t rb = tid & 15u, cb = tid >> 4;
        float *d0 = bf + (4 * cb) * kVRow + 4 * rb;
        *reinterpret_cast<float4 *>(d0) = make_float4(R.v[0].x, R.v[1].x, R.v[2].x, R.v[3].x);
        *reinterpret_cast<float4 *>(d0 + kVRow) = make_float4(R.v[0].y, R.v[1].y, R.v[2].y, R.v[3].y);
        *reinterpret_cast<float4 *>(d0 + 2 * kVRow) = make_float4(R.v[0].z, R.v[1].z, R.v[2].z, R.v[3].z);
        *reinterpret_cast<float4 *>(d0 + 3 * kVRow) = make_float4(R.v[0].w, R.v[1].w, R.v[2].w, R.v[3].w);
        bool fin = true;
#pragma unroll
        for (int j = 0; j < 4; j++)
            fin = fin && __builtin_isfinite(R.v[j].x) && __builtin_isfinite(R.v[j].y) &&
                  __builtin_isfinite(R.v[j].z) && __builtin_isfinite(R.v[j].w);
        const bool bad = __ballot(!fin) != 0;
        if (lane == 0) vbad_at((bf == buf1 ? 4u : 0u) + w) = bad ? 1u : 0u;
    };
    // Runs body(c, buffer of step c, parity of c) for every step; the rows of
    // step c + 1 are in flight while step c is used and stored after it.
    auto stream = [&](auto transposed, auto &&body) {
        auto load = [&](uint32_t c) {
            if constexpr (decltype(transposed)::value) return load_v(c);
            else return load_k(c);
        };
        auto put = [&](const Rows R, float *bf) {
            if constexpr (decltype(transposed)::value) store_vt(R, bf);
            else store_k(R, bf);
        };
        Rows A = load(0);
        put(A, buf0);
        __syncthreads();
        A = load(min(1u, nsteps - 1));
        for (uint32_t c = 0; c < nsteps; c += 2) {
            body(c, buf0, std::integral_constant<uint32_t, 0>{});
            if (c + 1 < nsteps) put(A, buf1);
            __syncthreads();
            if (c + 1 >= nsteps) break;
            A = load(min(c + 2, nsteps - 1));
            body(c + 1, buf1, std::integral_constant<uint32_t, 1>{});
            if (c + 2 < nsteps) put(A, buf0);
            __syncthreads();
            A = load(min(c + 3, nsteps - 1));
        }
    };

    // ---- pass 1: scores and maxima -----------------------------------------
    float mx[TPW];
    // scores of this lane's positions in steps 0 and 1, kept for pass 2
    float sA[TPW], sB[TPW];
#pragma unroll
    for (uint32_t j = 0; j < TPW; j++) mx[j] = sA[j] = sB[j] = -INFINITY;
    stream(std::false_type{}, [&](uint32_t c, const float *cur, auto) {
        const uint32_t p = c * kAttStep + lane;
        if (nv && p <= pos_last) {
            const float4 *kr = reinterpret_cast<const float4 *>(cur + lane * kKRow);
            // q is the same in every lane: with a wavefront-uniform address
            // it is read into scalar registers, leaving the LDS to K
            const uint32_t wu = __builtin_amdgcn_readfirstlane(w & 3u);
            const float4 *qg[TPW];
#pragma unroll
            for (uint32_t j = 0; j < TPW; j++)
                qg[j] = reinterpret_cast<const float4 *>(Q + (uint64_t)min(tg * TW + wu * TPW + j, ntok - 1) * qdim +
                                                         h * DH);
            float sc[TPW];
#pragma unroll
            for (uint32_t j = 0; j < TPW; j++) sc[j] = 0.0f;
#pragma unroll 4
            for (int d4 = 0; d4 < 16; d4++) {
                const float4 kk = kr[d4];
#pragma unroll
                for (uint32_t j = 0; j < TPW; j++) {
                    const float4 qq = qg[j][d4];
                    sc[j] += qq.x * kk.x;
                    sc[j] += qq.y * kk.y;
                    sc[j] += qq.z * kk.z;
                    sc[j] += qq.w * kk.w;
                }
            }
#pragma unroll
            for (uint32_t j = 0; j < TPW; j++) {
                if (j < nv && p <= pos0 + t0 + j) {
                    const float sv = sc[j] * scale;
                    srow(j)[p] = sv;
                    mx[j] = fmaxf(mx[j], sv);
                    if (c == 0) sA[j] = sv;
                    if (c == 1) sB[j] = sv;
                }
            }
        }
    });
#pragma unroll
    for (uint32_t j = 0; j < TPW; j++)
#pragma unroll
        for (int off = 32; off; off >>= 1) mx[j] = fmaxf(mx[j], __shfl_xor(mx[j], off, 64));

    // ---- pass 2: e, then the sums in position order --------------------------
    float acc[TPW], sum = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < TPW; j++) acc[j] = 0.0f;
    const uint32_t st_t = tg * TW + lane;   // wavefront 4: lane = token
    auto add_sums = [&](uint32_t c, uint32_t par) {   // wavefront 4: the e of step c
        const uint32_t p0 = c * kAttStep;
        if (lane < TW && st_t < ntok && pos0 + st_t >= p0) {
            const uint32_t lim = min(kAttStep, pos0 + st_t + 1 - p0);
            const float *e = eb + (par * TW + lane) * kAttStep;
            uint32_t r = 0;
            for (; r + 4 <= lim; r += 4) {
                const float4 e4 = *reinterpret_cast<const float4 *>(e + r);
                sum += e4.x;
                sum += e4.y;
                sum += e4.z;
                sum += e4.w;
            }
            for (; r < lim; r++) sum += e[r];
        }
    };
    stream(std::true_type{}, [&](uint32_t c, const float *cur, auto parity) {
        constexpr uint32_t par = decltype(parity)::value;
        const uint32_t p0 = c * kAttStep;
        if (w < 4) {
            if (nv == 0 || pos_last < p0) return;
            const uint32_t p = p0 + lane;
            float *const e0 = eb + (par * TW + (w & 3u) * TPW) * kAttStep;   // [TPW][64]
            // Skipping a position with e_p == 0 leaves the sum as adding
            // e_p * v = +-0 would (the sum starts at +0, so it is never -0),
            // unless v is infinite or NaN: the skip is taken only in a step
            // whose staged V holds such a value.
            bool zero = false, full = true;
            float evs[TPW];
#pragma unroll
            for (uint32_t j = 0; j < TPW; j++) {
                const uint32_t pj = pos0 + t0 + j;
                const float sv = par ? sB[j] : sA[j];
                const bool in = j < nv && p <= pj;
                const float ev = in ? pi_expf(sv - mx[j]) : 0.0f;
                evs[j] = ev;
                e0[j * kAttStep + lane] = ev;
                zero |= __ballot(in && ev == 0.0f) != 0;
                full &= j < nv && pj >= p0 + kAttStep - 1;
                const float sn = j < nv ? srow(j)[min(p + 2 * kAttStep, pj)] : 0.0f;   // scores of step c + 2
                if (par) sB[j] = sn;
                else sA[j] = sn;
            }
            const bool skip = zero && (vbad_at(par * 4u) | vbad_at(par * 4u + 1u) | vbad_at(par * 4u + 2u) |
                                       vbad_at(par * 4u + 3u)) != 0u;
            const float *vr = cur + lane * kVRow;
            if (full && !skip) {
                // e of the first kAttLaneE (token, position) pairs of the step
                // comes from its lane (v_readlane, VALU work), the rest from
                // the LDS step buffer (16-byte broadcast reads): the split
                // that balances the two (measured: a quarter read from lanes
                // ran faster than none, a half, three quarters or all)
#pragma unroll
                for (uint32_t q = 0; q < kAttStep; q += 4) {
                    const float4 v4 = *reinterpret_cast<const float4 *>(vr + q);
#pragma unroll
                    for (uint32_t j = 0; j < TPW; j++) {
                        const int ei = __float_as_int(evs[j]);
                        auto lane_e = [&](uint32_t i) { return __int_as_float(__builtin_amdgcn_readlane(ei, q + i)); };
                        const float4 e4 = (j * kAttStep + q) < kAttLaneE
                                              ? make_float4(lane_e(0), lane_e(1), lane_e(2), lane_e(3))
                                              : *reinterpret_cast<const float4 *>(e0 + j * kAttStep + q);
                        acc[j] = acc[j] + e4.x * v4.x;
                        acc[j] = acc[j] + e4.y * v4.y;
                        acc[j] = acc[j] + e4.z * v4.z;
                        acc[j] = acc[j] + e4.w * v4.w;
                    }
                }
            } else {
#pragma unroll
                for (uint32_t j = 0; j < TPW; j++) {
                    const uint32_t pj = pos0 + t0 + j;
                    if (j >= nv || pj < p0) continue;
                    const uint32_t lim = min(kAttStep, pj + 1 - p0);
                    const float *e = e0 + j * kAttStep;
                    uint32_t r = 0;
                    if (!skip) {
                        for (; r + 4 <= lim; r += 4) {
                            const float4 e4 = *reinterpret_cast<const float4 *>(e + r);
                            const float4 v4 = *reinterpret_cast<const float4 *>(vr + r);
                            acc[j] = acc[j] + e4.x * v4.x;
                            acc[j] = acc[j] + e4.y * v4.y;
                            acc[j] = acc[j] + e4.z * v4.z;
                            acc[j] = acc[j] + e4.w * v4.w;
                        }
                        for (; r < lim; r++) acc[j] = acc[j] + e[r] * vr[r];
                    } else {
                        for (; r < lim; r++) {
                            const float ee = e[r];
                            acc[j] = acc[j] + (ee != 0.0f ? ee * vr[r] : -0.0f);   // x + (-0) == x: a skipped position
                        }
                    }
                }
            }
        } else if (c > 0) {
            add_sums(c - 1, par ^ 1u);
        }
    });
    if (w == 4) {
        add_sums(nsteps - 1, (nsteps - 1) & 1u);
        if (lane < TW) misc_at(lane) = sum;
    }
    __syncthreads();
    if (w < 4) {
#pragma unroll
        for (uint32_t j = 0; j < TPW; j++) {
            const float tot = misc_at((w & 3u) * TPW + j);
            const float inv = tot > 0.0f ? 1.0f / tot : 0.0f;
            const float o = acc[j] * inv;
            const uint32_t blk = h * 2 + lane / 32, jj = lane % 32, t = t0 + j;
            float dd;
            int bsum;
            const int iv = q8_block32_core(o, dd, bsum);
            if (j < nv) {
                oq[pfq_off(blk, jj / 8, t) + jj % 8] = (int8_t)iv;
                if (jj == 0) {
                    od[blk * PI_PF_MAX_TOK + t] = dd;
                    os[blk * PI_PF_MAX_TOK + t] = bsum;
                }
            }
        }
    }
}

WV to_wv(const pi_pf_mat &M) {
    WV W;
    W.w = M.w;
    W.rows = M.L.rows;
    W.upr = M.L.upr;
    W.rpw = M.L.rpw;
    W.lpt = M.L.lpt;
    W.g = M.L.g;
    W.gmag = M.L.g > 1 ? (uint32_t)((((uint64_t)1 << 32) + M.L.g - 1) / M.L.g) : 0u;
    W.qc = M.L.qc;
    W.ntiles = M.L.ntiles;
    W.tile_bytes = M.L.tile_bytes;
    return W;
}

}  // namespace

hipError_t pi_pf_embed(const uint8_t *embd, uint32_t etype, uint64_t row_bytes, const uint32_t *ids, uint32_t ntok,
                       uint32_t ne, float *X, hipStream_t s) {
    if (ntok == 0 || ntok > PI_PF_MAX_TOK) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_pf_embed, dim3(ntok), dim3(256), 0, s, embd, etype, row_bytes, ids, ne, X);
    return hipGetLastError();
}

hipError_t pi_pf_norm_q8(const float *X, const float *w, uint32_t ne, float eps, uint32_t ntok, pi_pf_q8 o,
                         hipStream_t s) {
    if (ntok == 0 || ntok > PI_PF_MAX_TOK || ne % 32 || ne > 16384) return hipErrorInvalidValue;
    // tokens per workgroup: one while every token can have a CU of its own,
    // else two or four (while their LDS regions fit 128 KB), so that the chains
    // of the tokens sharing a CU run on different SIMDs
    const size_t region = (size_t)pf_norm_region(ne) * 4;
    const uint32_t want = ntok <= 256 ? 1u : (ntok <= 512 ? 2u : 4u);
    uint32_t tpb = want;
    while (tpb > 1 && region * tpb > (128u << 10)) tpb /= 2;
    const size_t lds = region * tpb;
    hipError_t e = hipFuncSetAttribute((const void *)k_pf_norm_q8, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_pf_norm_q8, dim3((ntok + tpb - 1) / tpb), dim3(256), lds, s, X, w, ne, eps, ntok, tpb, o);
    return hipGetLastError();
}

hipError_t pi_pf_gemm_multi(const pi_pf_mat *M, float *const *out, const uint32_t *mode, uint32_t nseg, pi_pf_q8 a,
                             uint32_t ntok, bool resid, const pi_pf_rope *rope, hipStream_t s) {
    if (ntok == 0 || ntok > PI_PF_MAX_TOK || nseg == 0 || nseg > kPfMaxSeg) return hipErrorInvalidValue;
    const uint32_t t = M[0].L.type, k = M[0].L.k;
    PfSegs S{};
    if (rope) S.rope = *rope;
    uint32_t wgs = 0;
    for (uint32_t i = 0; i < nseg; i++) {
        if (M[i].L.type != t || M[i].L.k != k || M[i].L.rows == 0) return hipErrorInvalidValue;
        S.mode[i] = mode ? mode[i] : PI_PF_STORE;
        if (S.mode[i] > PI_PF_CACHE) return hipErrorInvalidValue;
        if (S.mode[i] != PI_PF_STORE &&
            (resid || !rope || M[i].L.rows % 64 || rope->half > 32 || rope->pos0 + ntok > rope->n_ctx))
            return hipErrorInvalidValue;
        S.W[i] = to_wv(M[i]);
        S.out[i] = out[i];
        wgs += (M[i].L.rows + kPfRows - 1) / kPfRows * ((ntok + kPfTokWg - 1) / kPfTokWg);
        S.wg_end[i] = wgs;
    }
    S.nseg = nseg;
    const uint32_t nb = k / pi_base_elems(t);
    size_t cfl = 0;
    switch (t) {
    case PI_TYPE_Q4_K: cfl = (size_t)nb * PfLds<PI_TYPE_Q4_K>::floats_per_block; break;
    case PI_TYPE_Q6_K: cfl = (size_t)nb * PfLds<PI_TYPE_Q6_K>::floats_per_block; break;
    case PI_TYPE_Q4_0:
    case PI_TYPE_Q8_0:
        cfl = (size_t)nb * PfLds<PI_TYPE_Q8_0>::floats_per_block;
        static_assert(PfLds<PI_TYPE_Q8_0>::floats_per_block == PfLds<PI_TYPE_Q4_0>::floats_per_block, "");
        break;
    default: return hipErrorInvalidValue;
    }
    uint32_t ws = 0;
    switch (t) {
    case PI_TYPE_Q4_K: ws = PfStage<PI_TYPE_Q4_K>::WS; break;
    case PI_TYPE_Q6_K: ws = PfStage<PI_TYPE_Q6_K>::WS; break;
    case PI_TYPE_Q8_0: ws = PfStage<PI_TYPE_Q8_0>::WS; break;
    default: ws = PfStage<PI_TYPE_Q4_0>::WS; break;
    }
    const size_t lds = ((cfl + 3) & ~(size_t)3) * 4 + 2 * (size_t)kPfRows * ws * 16;
    if (lds > 64 * 1024 || nb > 65535) return hipErrorInvalidValue;
    const dim3 grid(wgs), block(kPfThreads);
    auto launch = [&](auto kern) {
        hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(kern, grid, block, lds, s, S, a.q, a.d, a.s, k, ntok, (int)resid);
        return hipGetLastError();
    };
    switch (t) {
    case PI_TYPE_Q4_K: return launch(k_pf_gemm<PI_TYPE_Q4_K>);
    case PI_TYPE_Q6_K: return launch(k_pf_gemm<PI_TYPE_Q6_K>);
    case PI_TYPE_Q8_0: return launch(k_pf_gemm<PI_TYPE_Q8_0>);
    default: return launch(k_pf_gemm<PI_TYPE_Q4_0>);
    }
}

hipError_t pi_pf_gemm(const pi_pf_mat &M, pi_pf_q8 a, uint32_t ntok, float *out, bool resid, hipStream_t s) {
    return pi_pf_gemm_multi(&M, &out, nullptr, 1, a, ntok, resid, nullptr, s);
}

hipError_t pi_pf_attn(const float *Q, const float *kc, const float *vc, uint32_t pos0, uint32_t ntok, uint32_t n_head,
                      uint32_t n_kv, uint32_t n_ctx, float scale, float *scores, pi_pf_q8 o, hipStream_t s) {
    if (ntok == 0 || ntok > PI_PF_MAX_TOK || pos0 + ntok > n_ctx || n_kv == 0 || n_head % n_kv) return hipErrorInvalidValue;
    const uint32_t P = pf_att_parts(n_head), ntg = (ntok + kAttTok - 1) / kAttTok;
    const uint32_t blocks = 8 * ((n_head * P + 7) / 8) * ((ntg + P - 1) / P);   // XCD 0 has the most units
    hipLaunchKernelGGL(k_pf_attn<kAttTpw>, dim3(blocks), dim3(kAttThreads), 0, s, Q, kc, vc, pos0, ntok, n_head, n_head / n_kv,
                       n_ctx, scale, scores, o.q, o.d, o.s);
    return hipGetLastError();
}

hipError_t pi_pf_swiglu_q8(const float *G, const float *U, uint32_t ntok, uint32_t n_ff, pi_pf_q8 o, hipStream_t s) {
    if (ntok == 0 || ntok > PI_PF_MAX_TOK || n_ff % 32) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_pf_swiglu_q8, dim3(ntok, (n_ff / 4 + 255) / 256), dim3(256), 0, s, G, U, n_ff, o);
    return hipGetLastError();
}
