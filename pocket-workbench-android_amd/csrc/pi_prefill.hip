// Batched prefill for gfx950: a chunk of up to 32 prompt tokens per pass.
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

// Device view of a tiled matrix and the byte offset of chunk j of base
// block u of row r (bc chunks per base block), or of its f16 field.
struct WV {
    const uint8_t *w;
    uint32_t rows, upr, rpw, lpt, g, qc, ntiles;
    uint64_t tile_bytes;
};

__device__ __forceinline__ void tile_pos(const WV &W, uint32_t r, uint32_t u, uint64_t &tbase, uint32_t &lanes,
                                         uint32_t &ln, uint32_t &b) {
    const uint32_t t = r / W.rpw, rt = r - t * W.rpw;
    lanes = (t == W.ntiles - 1) ? (W.rows - t * W.rpw) * W.upr : W.lpt;
    const uint32_t unit = u / W.g;
    b = u - unit * W.g;
    ln = rt * W.upr + unit;
    tbase = (uint64_t)t * W.tile_bytes;
}
__device__ __forceinline__ const uint8_t *chunk_at(const WV &W, uint32_t r, uint32_t u, uint32_t j, uint32_t bc) {
    uint64_t tb;
    uint32_t lanes, ln, b;
    tile_pos(W, r, u, tb, lanes, ln, b);
    return W.w + tb + ((uint64_t)(b * bc + j) * lanes + ln) * 16u;
}
__device__ __forceinline__ float dfield_at(const WV &W, uint32_t r, uint32_t u) {
    uint64_t tb;
    uint32_t lanes, ln, b;
    tile_pos(W, r, u, tb, lanes, ln, b);
    const PI_GLOBAL uint16_t *p =
        gld(reinterpret_cast<const uint16_t *>(W.w + tb + (uint64_t)lanes * W.qc * 16u + ((uint64_t)b * lanes + ln) * 2u));
    return h2f(*p);
}
__device__ __forceinline__ uint2 ld8(const uint8_t *p) { return *gld(reinterpret_cast<const uint2 *>(p)); }
__device__ __forceinline__ uint4 ld16(const uint8_t *p) { return *gld(reinterpret_cast<const uint4 *>(p)); }

__device__ __forceinline__ v4i mfma16(long a, long b) {
    v4i c = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// GEMM: a wavefront owns 16 rows x 16 tokens.  Lane l: A row r0 + l%16 with
// group elements 8*(l/16)..+7; B (and D) token 16*th + l%16; D rows
// r0 + 4*(l/16) + i, i = 0..3.
// ---------------------------------------------------------------------------
template <uint32_t T>
__global__ __launch_bounds__(256) void k_pf_gemm(WV W, const int8_t *__restrict__ aq, const float *__restrict__ ad,
                                                 const int32_t *__restrict__ as, uint32_t k, uint32_t ntok,
                                                 float *__restrict__ out, uint32_t ld, int resid) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wv = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t r0 = (wv >> 1) * 16, th = wv & 1u;
    if (r0 >= W.rows || th * 16 >= ntok) return;
    const uint32_t ka = lane >> 4, li = lane & 15u;
    const uint32_t ra = min(r0 + li, W.rows - 1);
    const uint32_t n = th * 16 + li;
    const bool n_ok = n < ntok;
    const uint32_t nn = n_ok ? n : 0u;
    const uint32_t nb32 = k / 32;
    const int8_t *arow = aq + (uint64_t)nn * k;
    const PI_GLOBAL float *adr = gld(ad + (uint64_t)nn * nb32);
    const PI_GLOBAL int32_t *asr = gld(as + (uint64_t)nn * nb32);
    uint32_t rd[4];
#pragma unroll
    for (int i = 0; i < 4; i++) rd[i] = min(r0 + 4 * ka + (uint32_t)i, W.rows - 1);
    float acc[4] = {0.f, 0.f, 0.f, 0.f};

    if constexpr (T == PI_TYPE_Q4_K) {
        const uint32_t nblk = k / 256;
        for (uint32_t u = 0; u < nblk; u++) {
            uint4 hdr[4];
#pragma unroll
            for (int i = 0; i < 4; i++) hdr[i] = ld16(chunk_at(W, rd[i], u, 0, 9));
            uint2 qa[4];
#pragma unroll
            for (int g = 0; g < 4; g++) qa[g] = ld8(chunk_at(W, ra, u, 1 + 2 * g + (ka >> 1), 9) + 8 * (ka & 1));
            long bq[8];
#pragma unroll
            for (int sb = 0; sb < 8; sb++) bq[sb] = *gld(reinterpret_cast<const long *>(arow + u * 256 + sb * 32 + 8 * ka));
#pragma unroll
            for (int sb = 0; sb < 8; sb++) {
                const int g = sb >> 1, h = sb & 1;
                const uint32_t lo = h ? (qa[g].x >> 4) & 0x0F0F0F0Fu : qa[g].x & 0x0F0F0F0Fu;
                const uint32_t hi = h ? (qa[g].y >> 4) & 0x0F0F0F0Fu : qa[g].y & 0x0F0F0F0Fu;
                const v4i c = mfma16(pack2(lo, hi), bq[sb]);
                const float da = adr[u * 8 + sb];
                const float asf = (float)asr[u * 8 + sb];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float d = h2f(hdr[i].x), dmin = h2f(hdr[i].x >> 16);
                    uint32_t s, m;  // get_scale_min_k4 on the 12 scale bytes (bytes 4..15)
                    if (sb < 4) {
                        s = byte16(hdr[i], 4 + sb) & 63u;
                        m = byte16(hdr[i], 4 + sb + 4) & 63u;
                    } else {
                        s = (byte16(hdr[i], 4 + sb + 4) & 0xFu) | ((byte16(hdr[i], 4 + sb - 4) >> 6) << 4);
                        m = (byte16(hdr[i], 4 + sb + 4) >> 4) | ((byte16(hdr[i], 4 + sb) >> 6) << 4);
                    }
                    const float term = d * da * (float)s * (float)c[i] - da * dmin * (float)m * asf;
                    acc[i] += term;
                }
            }
        }
    } else if constexpr (T == PI_TYPE_Q6_K) {
        const uint32_t nblk = k / 256;
        for (uint32_t u = 0; u < nblk; u++) {
            uint4 sc4[4];
            float d6[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sc4[i] = ld16(chunk_at(W, rd[i], u, 12, 13));
                d6[i] = dfield_at(W, rd[i], u);
            }
            long bq[8];
#pragma unroll
            for (int j = 0; j < 8; j++) bq[j] = *gld(reinterpret_cast<const long *>(arow + u * 256 + j * 32 + 8 * ka));
#pragma unroll
            for (int half = 0; half < 2; half++) {
                const uint2 ql0 = ld8(chunk_at(W, ra, u, half * 4 + (ka >> 1), 13) + 8 * (ka & 1));
                const uint2 ql1 = ld8(chunk_at(W, ra, u, half * 4 + 2 + (ka >> 1), 13) + 8 * (ka & 1));
                const uint2 qh = ld8(chunk_at(W, ra, u, 8 + half * 2 + (ka >> 1), 13) + 8 * (ka & 1));
#pragma unroll
                for (int g = 0; g < 2; g++) {
                    const bool mine = (ka >> 1) == (uint32_t)g;   // this lane's 8 elements are in group g
#pragma unroll
                    for (int s = 0; s < 4; s++) {
                        const uint2 qlw = (s & 1) ? ql1 : ql0;
                        uint32_t w6[2];
#pragma unroll
                        for (int c = 0; c < 2; c++) {
                            const uint32_t l4 = c ? qlw.y : qlw.x, h2 = c ? qh.y : qh.x;
                            const uint32_t nib = s < 2 ? (l4 & 0x0F0F0F0Fu) : ((l4 >> 4) & 0x0F0F0F0Fu);
                            const uint32_t q = nib | (((h2 >> (2 * s)) & 0x03030303u) << 4);   // 0..63 per byte
                            const uint32_t x = q ^ 0x20202020u;                               // q - 32 in 6 bits
                            w6[c] = x | ((x & 0x20202020u) * 6u);                              // sign-extend to 8
                        }
                        const long A = mine ? pack2(w6[0], w6[1]) : 0L;
                        const v4i c = mfma16(A, bq[4 * half + s]);
                        const float da = adr[u * 8 + 4 * half + s];
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const float scale = (float)(int8_t)byte16(sc4[i], half * 8 + g + 2 * s);
                            const float term = d6[i] * scale * da * (float)c[i];
                            acc[i] += term;
                        }
                    }
                }
            }
        }
    } else if constexpr (T == PI_TYPE_Q8_0) {
        const uint32_t nblk = k / 32;
        for (uint32_t u = 0; u < nblk; u++) {
            const uint2 w8 = ld8(chunk_at(W, ra, u, ka >> 1, 2) + 8 * (ka & 1));
            const long bq = *gld(reinterpret_cast<const long *>(arow + u * 32 + 8 * ka));
            const v4i c = mfma16(pack2(w8.x, w8.y), bq);
            const float da = adr[u];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float term = dfield_at(W, rd[i], u) * da * (float)c[i];
                acc[i] += term;
            }
        }
    } else {  // Q4_0: lo nibbles -> elements 0..15, hi -> 16..31
        const uint32_t nblk = k / 32;
        for (uint32_t u = 0; u < nblk; u++) {
            const uint2 raw = ld8(chunk_at(W, ra, u, 0, 1) + 8 * (ka & 1));
            const uint32_t sh = (ka >> 1) * 4;
            const long A = pack2((raw.x >> sh) & 0x0F0F0F0Fu, (raw.y >> sh) & 0x0F0F0F0Fu);
            const long bq = *gld(reinterpret_cast<const long *>(arow + u * 32 + 8 * ka));
            const v4i c = mfma16(A, bq);
            const float da = adr[u];
            const float asf = (float)asr[u];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float term = dfield_at(W, rd[i], u) * da * ((float)c[i] - 8.0f * asf);
                acc[i] += term;
            }
        }
    }
    if (n_ok) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t r = r0 + 4 * ka + (uint32_t)i;
            if (r < W.rows) {
                float *o = out + (uint64_t)n * ld + r;
                const float v = 0.0f + acc[i];
                *o = resid ? *o + v : v;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Embedding rows of the chunk.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_pf_embed(const uint8_t *__restrict__ E, uint32_t etype, uint64_t row_bytes,
                                                  const uint32_t *__restrict__ ids, uint32_t ne, float *__restrict__ X) {
    const uint32_t t = blockIdx.x;
    const uint8_t *row = E + (uint64_t)ids[t] * row_bytes;
    for (uint32_t e = threadIdx.x; e < ne; e += blockDim.x) X[(uint64_t)t * ne + e] = embed_elem(row, etype, e);
}

// ---------------------------------------------------------------------------
// RMSNorm (scalar order) + Q8 of one token per workgroup.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_pf_norm_q8(const float *__restrict__ X, const float *__restrict__ w,
                                                    uint32_t ne, float eps, int8_t *__restrict__ q,
                                                    float *__restrict__ d, int32_t *__restrict__ s) {
    extern __shared__ __align__(16) float xs[];
    __shared__ float sv;
    const uint32_t t = blockIdx.x, tid = threadIdx.x, nb = ne / 32;
    const float4 *x4 = reinterpret_cast<const float4 *>(X + (uint64_t)t * ne);
    for (uint32_t i = tid; i < ne / 4; i += blockDim.x) reinterpret_cast<float4 *>(xs)[i] = x4[i];
    __syncthreads();
    if (tid == 0) {
        float ss = 0.0f;
        lds_fold4<6>(reinterpret_cast<const float4 *>(xs), ne / 4, [&](const float4 &v) {
            ss += v.x * v.x;
            ss += v.y * v.y;
            ss += v.z * v.z;
            ss += v.w * v.w;
        });
        sv = 1.0f / sqrtf(ss / (float)ne + eps);
    }
    __syncthreads();
    const float sc = sv;
    for (uint32_t b = tid; b < nb; b += blockDim.x) {
        float v[32];
#pragma unroll
        for (int j = 0; j < 32; j++) v[j] = xs[32 * b + j] * sc * w[32 * b + j];
        q8_lane(v, reinterpret_cast<uint32_t *>(q + (uint64_t)t * ne) + 8 * b, d + (uint64_t)t * nb + b,
                s + (uint64_t)t * nb + b);
    }
}

// ---------------------------------------------------------------------------
// h = silu(gate) * up, then Q8 of h (one token per workgroup).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_pf_swiglu_q8(const float *__restrict__ G, const float *__restrict__ U,
                                                      uint32_t n_ff, int8_t *__restrict__ q, float *__restrict__ d,
                                                      int32_t *__restrict__ s) {
    const uint32_t t = blockIdx.x, nb = n_ff / 32;
    for (uint32_t b = threadIdx.x; b < nb; b += blockDim.x) {
        float v[32];
        const float *g = G + (uint64_t)t * n_ff + 32 * b, *u = U + (uint64_t)t * n_ff + 32 * b;
#pragma unroll
        for (int j = 0; j < 32; j++) {
            const float gg = g[j];
            const float sg = gg / (1.0f + pi_expf(-gg));
            v[j] = sg * u[j];
        }
        q8_lane(v, reinterpret_cast<uint32_t *>(q + (uint64_t)t * n_ff) + 8 * b, d + (uint64_t)t * nb + b,
                s + (uint64_t)t * nb + b);
    }
}

// ---------------------------------------------------------------------------
// RoPE + KV rows (one token per workgroup).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_pf_rope_kv(float *__restrict__ Q, const float *__restrict__ K,
                                                    const float *__restrict__ V, const float *__restrict__ cos_tab,
                                                    const float *__restrict__ sin_tab, uint32_t pos0,
                                                    uint32_t n_head, uint32_t n_kv, uint32_t half,
                                                    float *__restrict__ kc, float *__restrict__ vc, uint32_t n_ctx) {
    constexpr uint32_t DH = 64;
    const uint32_t t = blockIdx.x, pos = pos0 + t;
    const float *cb = cos_tab + (uint64_t)pos * half, *sb = sin_tab + (uint64_t)pos * half;
    const uint32_t qdim = n_head * DH, kdim = n_kv * DH;
    for (uint32_t i = threadIdx.x; i < n_head * (DH / 2); i += blockDim.x) {
        const uint32_t h = i / (DH / 2), p = i % (DH / 2);
        if (p < half) {
            float *x = Q + (uint64_t)t * qdim + h * DH + 2 * p;
            const float x0 = x[0], x1 = x[1], c = cb[p], s = sb[p];
            x[0] = x0 * c - x1 * s;
            x[1] = x0 * s + x1 * c;
        }
    }
    for (uint32_t i = threadIdx.x; i < n_kv * (DH / 2); i += blockDim.x) {
        const uint32_t h = i / (DH / 2), p = i % (DH / 2);
        const float *x = K + (uint64_t)t * kdim + h * DH + 2 * p;
        float y0 = x[0], y1 = x[1];
        if (p < half) {
            const float c = cb[p], s = sb[p];
            const float r0 = y0 * c - y1 * s, r1 = y0 * s + y1 * c;
            y0 = r0;
            y1 = r1;
        }
        float *dst = kc + ((uint64_t)h * n_ctx + pos) * DH + 2 * p;
        dst[0] = y0;
        dst[1] = y1;
    }
    for (uint32_t i = threadIdx.x; i < kdim; i += blockDim.x) {
        const uint32_t h = i / DH, dd = i % DH;
        vc[((uint64_t)h * n_ctx + pos) * DH + dd] = V[(uint64_t)t * kdim + i];
    }
}

// ---------------------------------------------------------------------------
// Attention: a workgroup serves 4 tokens (one per wavefront) of one head and
// stages 64 K, then V rows at a time through LDS for all four.
// Scores: lane = position, scalar dot in d order, * scale.  Values: lane =
// dimension, in position order: sum += e_p; acc += e_p * v_p[d] unless
// e_p == 0.  Output acc * (1/sum), then Q8 of the head's 64 values.
// ---------------------------------------------------------------------------
constexpr uint32_t kKvPad = 65;

__global__ __launch_bounds__(256) void k_pf_attn(const float *__restrict__ Q, const float *__restrict__ kc,
                                                 const float *__restrict__ vc, uint32_t pos0, uint32_t ntok,
                                                 uint32_t n_head, uint32_t group, uint32_t n_ctx, float scale,
                                                 int8_t *__restrict__ oq, float *__restrict__ od,
                                                 int32_t *__restrict__ os) {
    constexpr uint32_t DH = 64;
    extern __shared__ __align__(16) float lds[];
    float *kv = lds;                          // 64 x 65
    float *qs = kv + 64 * kKvPad;             // 4 x 64
    float *sc = qs + 4 * DH;                  // 4 x n_ctx
    const uint32_t h = blockIdx.x % n_head, tg = blockIdx.x / n_head;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u, tid = threadIdx.x;
    const uint32_t t = 4 * tg + wave;
    const bool valid = t < ntok;
    const uint32_t pos_t = pos0 + t;          // positions 0..pos_t (valid tokens)
    const uint32_t n_all = pos0 + min(4 * tg + 3, ntok - 1) + 1;
    const uint32_t kvh = h / group, qdim = n_head * DH;
    const float *kbase = kc + (uint64_t)kvh * n_ctx * DH, *vbase = vc + (uint64_t)kvh * n_ctx * DH;
    float *scw = sc + (uint64_t)wave * n_ctx;
    qs[wave * DH + lane] = valid ? Q[(uint64_t)t * qdim + h * DH + lane] : 0.0f;
    float mx = -INFINITY;
    auto stage = [&](const float *base, uint32_t c0, uint32_t rows) {
        for (uint32_t i = tid; i < rows * 16; i += 256) {
            const uint32_t p = i / 16, f = i % 16;
            const float4 v = reinterpret_cast<const float4 *>(base + (uint64_t)(c0 + p) * DH)[f];
            float *dst = kv + p * kKvPad + 4 * f;
            dst[0] = v.x;
            dst[1] = v.y;
            dst[2] = v.z;
            dst[3] = v.w;
        }
    };
    for (uint32_t c0 = 0; c0 < n_all; c0 += 64) {
        const uint32_t rows = min(64u, n_all - c0);
        __syncthreads();
        stage(kbase, c0, rows);
        __syncthreads();
        const uint32_t p = c0 + lane;
        if (valid && lane < rows && p <= pos_t) {
            float s = 0.0f;
            const float *kr = kv + lane * kKvPad, *qv = qs + wave * DH;
#pragma unroll 16
            for (uint32_t dd = 0; dd < DH; dd++) s += qv[dd] * kr[dd];
            s = s * scale;
            scw[p] = s;
            mx = fmaxf(mx, s);
        }
    }
#pragma unroll
    for (int off = 32; off; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    if (valid)
        for (uint32_t p = lane; p <= pos_t; p += 64) scw[p] = pi_expf(scw[p] - mx);
    float acc = 0.0f, sum = 0.0f;
    for (uint32_t c0 = 0; c0 < n_all; c0 += 64) {
        const uint32_t rows = min(64u, n_all - c0);
        __syncthreads();
        stage(vbase, c0, rows);
        __syncthreads();
        if (valid && pos_t >= c0) {
            const uint32_t lim = min(rows, pos_t + 1 - c0);
            for (uint32_t r = 0; r < lim; r++) {
                const float e = scw[c0 + r];
                sum += e;
                const float v = kv[r * kKvPad + lane];
                acc = (e != 0.0f) ? acc + e * v : acc;
            }
        }
    }
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    const float o = acc * inv;
    const uint32_t nb = qdim / 32, blk = h * 2 + lane / 32;
    q8_block32(o, (int)(lane % 32), oq + (uint64_t)t * qdim + blk * 32, od + (uint64_t)t * nb + blk,
               os + (uint64_t)t * nb + blk, valid);
}

WV to_wv(const pi_pf_mat &M) {
    WV W;
    W.w = M.w;
    W.rows = M.L.rows;
    W.upr = M.L.upr;
    W.rpw = M.L.rpw;
    W.lpt = M.L.lpt;
    W.g = M.L.g;
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
    if (ntok == 0 || ntok > PI_PF_MAX_TOK || ne % 32 || ne / 32 > 256) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_pf_norm_q8, dim3(ntok), dim3(256), ne * 4, s, X, w, ne, eps, o.q, o.d, o.s);
    return hipGetLastError();
}

hipError_t pi_pf_gemm(const pi_pf_mat &M, pi_pf_q8 a, uint32_t ntok, float *out, bool resid, hipStream_t s) {
    if (ntok == 0 || ntok > PI_PF_MAX_TOK || M.L.rows == 0) return hipErrorInvalidValue;
    const WV W = to_wv(M);
    const uint32_t waves = (M.L.rows + 15) / 16 * 2, blocks = (waves + 3) / 4;
    switch (M.L.type) {
    case PI_TYPE_Q4_K:
        hipLaunchKernelGGL(k_pf_gemm<PI_TYPE_Q4_K>, dim3(blocks), dim3(256), 0, s, W, a.q, a.d, a.s, M.L.k, ntok, out,
                           M.L.rows, (int)resid);
        break;
    case PI_TYPE_Q6_K:
        hipLaunchKernelGGL(k_pf_gemm<PI_TYPE_Q6_K>, dim3(blocks), dim3(256), 0, s, W, a.q, a.d, a.s, M.L.k, ntok, out,
                           M.L.rows, (int)resid);
        break;
    case PI_TYPE_Q8_0:
        hipLaunchKernelGGL(k_pf_gemm<PI_TYPE_Q8_0>, dim3(blocks), dim3(256), 0, s, W, a.q, a.d, a.s, M.L.k, ntok, out,
                           M.L.rows, (int)resid);
        break;
    case PI_TYPE_Q4_0:
        hipLaunchKernelGGL(k_pf_gemm<PI_TYPE_Q4_0>, dim3(blocks), dim3(256), 0, s, W, a.q, a.d, a.s, M.L.k, ntok, out,
                           M.L.rows, (int)resid);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t pi_pf_rope_kv(float *Q, const float *K, const float *V, const float *cos_tab, const float *sin_tab,
                         uint32_t pos0, uint32_t ntok, uint32_t n_head, uint32_t n_kv, uint32_t half, float *kc,
                         float *vc, uint32_t n_ctx, hipStream_t s) {
    if (ntok == 0 || ntok > PI_PF_MAX_TOK || pos0 + ntok > n_ctx || half > 32) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_pf_rope_kv, dim3(ntok), dim3(256), 0, s, Q, K, V, cos_tab, sin_tab, pos0, n_head, n_kv, half,
                       kc, vc, n_ctx);
    return hipGetLastError();
}

size_t pi_pf_attn_lds_bytes(uint32_t n_ctx) { return (size_t)(64 * kKvPad + 4 * 64 + 4 * (size_t)n_ctx) * 4; }

hipError_t pi_pf_attn(const float *Q, const float *kc, const float *vc, uint32_t pos0, uint32_t ntok, uint32_t n_head,
                      uint32_t n_kv, uint32_t n_ctx, float scale, pi_pf_q8 o, hipStream_t s) {
    if (ntok == 0 || ntok > PI_PF_MAX_TOK || pos0 + ntok > n_ctx || n_kv == 0 || n_head % n_kv) return hipErrorInvalidValue;
    const size_t lds = pi_pf_attn_lds_bytes(n_ctx);
    hipError_t e = hipFuncSetAttribute((const void *)k_pf_attn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    const uint32_t blocks = n_head * ((ntok + 3) / 4);
    hipLaunchKernelGGL(k_pf_attn, dim3(blocks), dim3(256), lds, s, Q, kc, vc, pos0, ntok, n_head, n_head / n_kv, n_ctx,
                       scale, o.q, o.d, o.s);
    return hipGetLastError();
}

hipError_t pi_pf_swiglu_q8(const float *G, const float *U, uint32_t ntok, uint32_t n_ff, pi_pf_q8 o, hipStream_t s) {
    if (ntok == 0 || ntok > PI_PF_MAX_TOK || n_ff % 32) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_pf_swiglu_q8, dim3(ntok), dim3(256), 0, s, G, U, n_ff, o.q, o.d, o.s);
    return hipGetLastError();
}
