// Fused kernels of one decode token on gfx950 (batch 1, or one token of a
// prefill chunk evaluated in the batch order).
//
// Per layer (model.rs:905-1127):
//   k_norm_gemv      RMSNorm + Q8 of x into LDS (every workgroup), then the
//                    Q/K/V GEMVs                              -> q, k, v (f32)
//   k_attn           RoPE of q and k, KV write, attention over positions
//                    0..pos, Q8 of the output                 -> Q8 act
//   k_gemv_res       O GEMV on that Q8 activation, x += proj
//   k_norm_gemv      RMSNorm + Q8, gate/up GEMVs; a wavefront owns a gate
//                    tile and the matching up tile and writes
//                    silu(gate)*up for its rows              -> h (f32)
//   k_q8_gemv_res    Q8 of h into LDS, down GEMV, x += proj
// After the last layer k_norm_gemv runs output_norm + the head GEMV with a
// per-workgroup argmax partial, and k_step reduces the partials, records the
// greedy id, advances the position and embeds the next token.
//
// Every float expression keeps the reference's operation order (the file is
// built with -ffp-contract=off; the only fused multiply-adds are the explicit
// ones of simd::f32_sum_sq), so a forward is bit-identical to the CPU path.
#include <hip/hip_runtime.h>

#include "pi_decode.h"
#include "pi_gemv.h"

using namespace pig;

namespace {

constexpr uint32_t kThreads = 256;  // threads of a fused workgroup (4 wavefronts)
constexpr uint32_t kGemvThreads = 256;   // standalone GEMV: 4 single-tile wavefronts per workgroup

__host__ __device__ constexpr uint32_t pad32(uint32_t i) { return i + (i >> 5); }
// floats of the padded staging copy of x, rounded to 16 bytes
__host__ __device__ constexpr uint32_t xs_floats(uint32_t ne) { return (pad32(ne) + 4) & ~3u; }

// LDS of a prologue: the Q8 activation of the whole input vector.
struct ActLds {
    uint32_t *qw;  // k/4 words of quants
    float *d;      // k/32 block scales
    int32_t *s;    // k/32 block sums
};

__device__ __forceinline__ ActLds carve_act(unsigned char *base, uint32_t k) {
    ActLds a;
    a.qw = reinterpret_cast<uint32_t *>(base);
    a.d = reinterpret_cast<float *>(base + k);
    a.s = reinterpret_cast<int32_t *>(base + k + (k / 32) * 4);
    return a;
}
__host__ __device__ constexpr uint32_t act_lds_bytes(uint32_t k) { return k + (k / 32) * 8; }

// Engine::rmsnorm (model.rs:777-823) of one column, then Q8Act::prepare
// (quant_int.rs:17-56) of the result into LDS.  NEON: f32_sum_sq of the
// aarch64 build at batch 1 (simd.rs:45-64): eight FMA chains over stride-8
// elements, a0 + a1 lane-wise, (t0 + t1) + (t2 + t3), scalar tail; else the
// scalar loop used for batches of more than one token.  out = (x*s)*w.
template <bool NEON>
__device__ void pro_norm_q8(const float *__restrict__ x, const float *__restrict__ w, uint32_t ne, float eps,
                            float *xs, float *red, ActLds A) {
    const uint32_t tid = threadIdx.x;
    for (uint32_t i = tid; i < ne; i += blockDim.x) xs[pad32(i)] = x[i];
    __syncthreads();
    if constexpr (NEON) {
        if (tid < 8) {
            float acc = 0.0f;
            const uint32_t n8 = ne / 8;
#pragma unroll 8
            for (uint32_t i = 0; i < n8; i++) {
                const float v = xs[pad32(8 * i + tid)];
                acc = __builtin_fmaf(v, v, acc);
            }
            red[tid] = acc;
        }
        wave_sync();
        if (tid == 0) {
            const float t0 = red[0] + red[4], t1 = red[1] + red[5], t2 = red[2] + red[6], t3 = red[3] + red[7];
            float ss = (t0 + t1) + (t2 + t3);
            for (uint32_t i = ne / 8 * 8; i < ne; i++) ss += xs[pad32(i)] * xs[pad32(i)];
            red[8] = 1.0f / sqrtf(ss / (float)ne + eps);
        }
    } else {
        if (tid == 0) {
            float ss = 0.0f;
#pragma unroll 8
            for (uint32_t i = 0; i < ne; i++) {
                const float v = xs[pad32(i)];
                ss += v * v;
            }
            red[8] = 1.0f / sqrtf(ss / (float)ne + eps);
        }
    }
    __syncthreads();
    const float s = red[8];
    for (uint32_t b = tid; b < ne / 32; b += blockDim.x) {
        float v[32];
        const float4 *w4 = reinterpret_cast<const float4 *>(w + 32 * b);
#pragma unroll
        for (int j4 = 0; j4 < 8; j4++) {
            const float4 ww = w4[j4];
            v[4 * j4 + 0] = xs[pad32(32 * b + 4 * j4 + 0)] * s * ww.x;
            v[4 * j4 + 1] = xs[pad32(32 * b + 4 * j4 + 1)] * s * ww.y;
            v[4 * j4 + 2] = xs[pad32(32 * b + 4 * j4 + 2)] * s * ww.z;
            v[4 * j4 + 3] = xs[pad32(32 * b + 4 * j4 + 3)] * s * ww.w;
        }
        q8_lane(v, A.qw + 8 * b, A.d + b, A.s + b);
    }
    __syncthreads();
}

// Q8Act::prepare of a vector already in HBM (the SwiGLU output) into LDS.
__device__ void pro_q8(const float *__restrict__ x, uint32_t k, ActLds A) {
    for (uint32_t b = threadIdx.x; b < k / 32; b += blockDim.x) {
        float v[32];
        const float4 *x4 = reinterpret_cast<const float4 *>(x + 32 * b);
#pragma unroll
        for (int j4 = 0; j4 < 8; j4++) {
            const float4 t = x4[j4];
            v[4 * j4 + 0] = t.x;
            v[4 * j4 + 1] = t.y;
            v[4 * j4 + 2] = t.z;
            v[4 * j4 + 3] = t.w;
        }
        q8_lane(v, A.qw + 8 * b, A.d + b, A.s + b);
    }
    __syncthreads();
}

__device__ __forceinline__ void amax_merge(float &bv, uint32_t &bi, float v, uint32_t i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

// ---------------------------------------------------------------------------
// RMSNorm + GEMVs.  Segment A (type TA) and optional segment B (type TB) share
// the normalized activation (both have 256-element units when TB != TA).
// EPI_OUT: y = value.  EPI_SWIGLU: segment A holds gate and up with equal
// tile counts; a wavefront runs gate tile i then up tile i and stores
// h = silu(g)*u (model.rs:1111-1115).  EPI_ARGMAX: y = value plus the
// workgroup's (max, first index) pair.
// ---------------------------------------------------------------------------
template <bool NEON, uint32_t TA, uint32_t TB, int EPI>
__global__ __launch_bounds__(kThreads) void k_norm_gemv(const float *__restrict__ x, const float *__restrict__ nw,
                                                        uint32_t ne, float eps, MatSet SA, MatSet SB,
                                                        float *__restrict__ h, float *__restrict__ pv,
                                                        uint32_t *__restrict__ pidx) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int TPUA = QT<TA>::TPB, TPUB = QT<TB>::TPB;
    constexpr int TPU = TPUA > TPUB ? TPUA : TPUB;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    float *strip = reinterpret_cast<float *>(smem) + wave * 64 * TPU;
    float *red = reinterpret_cast<float *>(smem) + (kThreads / 64) * 64 * TPU;
    float *xs = red + 16;
    ActLds A = carve_act(reinterpret_cast<unsigned char *>(xs + xs_floats(ne)), ne);

    const uint32_t gw = blockIdx.x * (kThreads / 64) + wave, nw_all = gridDim.x * (kThreads / 64);
    const uint32_t ntA = SA.tile0[3];
    float best_v = -INFINITY;
    uint32_t best_i = 0xFFFFFFFFu;

    if constexpr (EPI == PI_EPI_SWIGLU) {
        // pairs (gate tile i, up tile i); one pair per step
        const uint32_t npair = SA.tile0[1];
        const uint32_t p0 = gw < npair ? gw : npair - 1;
        Unit<TA, 1> Ug, Uu;
        TileRef Rg = tile_ref(SA, p0), Ru = tile_ref(SA, SA.tile0[1] + p0);
        Ug.load(Rg.base, Rg.lanes, min(lane, Rg.lanes - 1));
        Uu.load(Ru.base, Ru.lanes, min(lane, Ru.lanes - 1));
        pro_norm_q8<NEON>(x, nw, ne, eps, xs, red, A);
        Slice<TA, 1> S;
        S.load(reinterpret_cast<const int8_t *>(A.qw), A.d, A.s, lane % SA.upr);
        const uint32_t per_row = SA.upr * TPUA;
        for (uint32_t p = gw; p < npair; p += nw_all) {
            if (p != p0) {
                Rg = tile_ref(SA, p);
                Ru = tile_ref(SA, SA.tile0[1] + p);
                Ug.load(Rg.base, Rg.lanes, min(lane, Rg.lanes - 1));
                Uu.load(Ru.base, Ru.lanes, min(lane, Ru.lanes - 1));
            }
            float term[TPUA];
            int isum[TPUA];
            unit_terms<TA, 1>(Ug, S, term, isum);
            if (lane < Rg.lanes) {
#pragma unroll
                for (int t = 0; t < TPUA; t++) strip[lane * TPUA + t] = term[t];
            }
            wave_sync();
            float g = 0.0f;
            if (lane < Rg.nrows) g = 0.0f + chain_sum(strip + lane * per_row, per_row);
            wave_sync();
            unit_terms<TA, 1>(Uu, S, term, isum);
            if (lane < Ru.lanes) {
#pragma unroll
                for (int t = 0; t < TPUA; t++) strip[lane * TPUA + t] = term[t];
            }
            wave_sync();
            if (lane < Ru.nrows) {
                const float u = 0.0f + chain_sum(strip + lane * per_row, per_row);
                const float sg = g / (1.0f + pi_expf(-g));
                h[Rg.row0 + lane] = sg * u;
            }
            wave_sync();
        }
        return;
    } else {
        // segment A (its first tile is requested before the prologue)
        const uint32_t firstA = gw;
        const TileRef R0 = tile_ref(SA, firstA < ntA ? firstA : ntA - 1);
        Unit<TA, 1> U0;
        U0.load(R0.base, R0.lanes, min(lane, R0.lanes - 1));
        pro_norm_q8<NEON>(x, nw, ne, eps, xs, red, A);
        Slice<TA, 1> S;
        S.load(reinterpret_cast<const int8_t *>(A.qw), A.d, A.s, lane % SA.upr);
        auto out = [&](uint32_t m, uint32_t row, float v) {
            SA.y[m][row] = v;
            if constexpr (EPI == PI_EPI_ARGMAX) amax_merge(best_v, best_i, v, row);
        };
        if (firstA < ntA) {
            // first tile from the registers loaded above, then the rest
            consume_tile<TA, 1>(SA, S, U0, R0, strip, out);
            run_tiles<TA, 1>(SA, S, firstA + nw_all, nw_all, strip, out);
        }
        if constexpr (TB != TA) {
            if (SB.n > 0) {
                Slice<TB, 1> SBs;
                SBs.load(reinterpret_cast<const int8_t *>(A.qw), A.d, A.s, lane % SB.upr);
                // segment B continues the wavefront numbering after segment A
                const uint32_t shift = ntA % nw_all;
                const uint32_t firstB = (gw + nw_all - shift) % nw_all;
                auto outB = [&](uint32_t m, uint32_t row, float v) { SB.y[m][row] = v; };
                run_tiles<TB, 1>(SB, SBs, firstB, nw_all, strip, outB);
            }
        }
    }
    if constexpr (EPI == PI_EPI_ARGMAX) {
#pragma unroll
        for (int off = 32; off; off >>= 1) {
            const float ov = __shfl_xor(best_v, off, 64);
            const uint32_t oi = __shfl_xor(best_i, off, 64);
            amax_merge(best_v, best_i, ov, oi);
        }
        __shared__ float sv[kThreads / 64];
        __shared__ uint32_t si[kThreads / 64];
        if (lane == 0) {
            sv[wave] = best_v;
            si[wave] = best_i;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            for (uint32_t w = 1; w < kThreads / 64; w++) amax_merge(best_v, best_i, sv[w], si[w]);
            pv[blockIdx.x] = best_v;
            pidx[blockIdx.x] = best_i;
        }
    }
}

// ---------------------------------------------------------------------------
// GEMV + residual on a Q8 activation: from HBM (PRO_GLOBAL: the attention
// output) or quantized here from an f32 vector (PRO_Q8: the SwiGLU output).
// x[row] = x[row] + (0 + acc) (model.rs:1095-1097, 1123-1125).
// ---------------------------------------------------------------------------
template <uint32_t T, int G, int PRO>
__global__ __launch_bounds__(kThreads) void k_gemv_res(const int8_t *__restrict__ aq, const float *__restrict__ ad,
                                                       const int32_t *__restrict__ as, const float *__restrict__ hx,
                                                       uint32_t k, MatSet S) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int TPU = QT<T>::TPB * G;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    float *strip = reinterpret_cast<float *>(smem) + wave * 64 * TPU;
    const uint32_t gw = blockIdx.x * (kThreads / 64) + wave, nw_all = gridDim.x * (kThreads / 64);
    const uint32_t nt = S.tile0[3];
    const TileRef R0 = tile_ref(S, gw < nt ? gw : nt - 1);
    Unit<T, G> U0;
    U0.load(R0.base, R0.lanes, min(lane, R0.lanes - 1));
    Slice<T, G> SL;
    if constexpr (PRO == PI_PRO_Q8) {
        ActLds A = carve_act(smem + (kThreads / 64) * 64 * TPU * 4, k);
        pro_q8(hx, k, A);
        SL.load(reinterpret_cast<const int8_t *>(A.qw), A.d, A.s, lane % S.upr);
    } else {
        SL.load(aq, ad, as, lane % S.upr);
    }
    auto out = [&](uint32_t m, uint32_t row, float v) { S.y[m][row] = S.y[m][row] + v; };
    if (gw >= nt) return;
    consume_tile<T, G>(S, SL, U0, R0, strip, out);
    run_tiles<T, G>(S, SL, gw + nw_all, nw_all, strip, out);
}

// ---------------------------------------------------------------------------
// Standalone GEMV on a Q8 activation in HBM (OpenClBackend::matvec twin, the
// device-pointer GEMV and the block-sum test hook).  One wavefront per
// workgroup so that small matrices still spread over every CU.
// ---------------------------------------------------------------------------
template <uint32_t T, int G, int MODE>
__global__ __launch_bounds__(kGemvThreads) void k_gemv(MatSet S, const int8_t *__restrict__ aq,
                                                       const float *__restrict__ ad, const int32_t *__restrict__ as,
                                                       int32_t *__restrict__ sums) {
    constexpr int TPU = QT<T>::TPB * G;
    constexpr uint32_t W = kGemvThreads / 64;
    __shared__ __align__(16) float strips[W * 64 * TPU + kChainPad];
    const uint32_t lane = threadIdx.x & 63u, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t gw = blockIdx.x * W + wave, nw = gridDim.x * W;
    float *strip = strips + wave * 64 * TPU;
    Slice<T, G> SL;
    SL.load(aq, ad, as, lane % S.upr);
    if constexpr (MODE == PI_GEMV_SUMS) {
        run_tiles_sums<T, G>(S, SL, gw, nw, sums);
    } else {
        auto out = [&](uint32_t m, uint32_t row, float v) {
            if constexpr (MODE == PI_GEMV_OUT) S.y[m][row] = v;
            else S.y[m][row] = S.y[m][row] + v;
        };
        run_tiles<T, G>(S, SL, gw, nw, strip, out);
    }
}

// Row bytes of the LDS copy of a Q8 activation of k elements: quant chunks
// in act_chunk order need whole 256-byte rows.
__host__ __device__ constexpr uint32_t act_q_bytes(uint32_t k) { return (k + 255u) & ~255u; }

// Standalone GEMV on an f32 x in HBM: every workgroup forms the Q8
// activation of x itself (Q8Act::prepare, quant_int.rs:17-56: the pair rule
// of q8_pair_core, bit-identical to the oracle) into LDS, so one launch does
// the whole job of quantize-then-multiply.  Each wavefront requests the
// weights of its first tile before it reads x, so that latency overlaps the
// quantization.  y[m][row] = sum of terms in the reference's order.
template <uint32_t T, int G>
__global__ __launch_bounds__(kGemvThreads) void k_gemv_x(MatSet S, const float *__restrict__ x, uint32_t k) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int TPU = QT<T>::TPB * G;
    constexpr uint32_t W = kGemvThreads / 64;
    float *strips = reinterpret_cast<float *>(smem);
    unsigned char *act = smem + ((W * 64 * TPU + kChainPad) * 4 + 15) / 16 * 16;
    uint32_t *qw = reinterpret_cast<uint32_t *>(act);
    float *ad = reinterpret_cast<float *>(act + act_q_bytes(k));
    int32_t *as = reinterpret_cast<int32_t *>(ad + k / 32);
    const uint32_t lane = threadIdx.x & 63u, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t gw = blockIdx.x * W + wave, nw = gridDim.x * W;
    const bool has = gw < S.tile0[3];
    Unit<T, G> UA;
    TileRef RA{};
    if (has) {
        RA = tile_ref(S, gw);
        UA.load(RA.base, RA.lanes, min(lane, RA.lanes - 1));
    }
    // 16 elements per lane, the two halves of a block in adjacent lanes
    for (uint32_t t = threadIdx.x; t < k / 16; t += kGemvThreads) {
        const float4 *x4 = reinterpret_cast<const float4 *>(x + 16 * (uint64_t)t);
        float v[16];
#pragma unroll
        for (int j4 = 0; j4 < 4; j4++) {
            const float4 q = x4[j4];
            v[4 * j4 + 0] = q.x;
            v[4 * j4 + 1] = q.y;
            v[4 * j4 + 2] = q.z;
            v[4 * j4 + 3] = q.w;
        }
        const uint32_t b = t >> 1, h = t & 1u;
        q8_pair(v, h, qw + 4 * act_chunk(2 * b + h), ad + b, as + b);
    }
    __syncthreads();
    if (!has) return;
    Slice<T, G> SL;
    SL.load_swz(reinterpret_cast<const int8_t *>(qw), ad, as, lane % S.upr);
    float *strip = strips + wave * 64 * TPU;
    auto out = [&](uint32_t m, uint32_t row, float v) { S.y[m][row] = v; };
    run_tiles_pre<T, G>(S, SL, UA, RA, gw, nw, strip, out);
}

// ---------------------------------------------------------------------------
// Attention of one head (model.rs:953-1087) for the token at st->pos.
// RoPE over adjacent pairs with the cached cos/sin, the K/V row write
// (the first query head of a KV group writes it; every head uses its own
// rotated copy for the current position), scores q.k_p * (1/sqrt(dh)) for
// p = 0..pos (NEON: simd::f32_dot's two 4-lane accumulators; else the scalar
// loop), max, e_p = exp(s_p - max), sum over p in order, o[d] accumulated over
// p in order skipping e_p == 0 (f32_axpy), o * (1/sum), then Q8 of o.
// Values are staged through LDS by wavefronts 1-3 while wavefront 0 (lane =
// dimension) runs the ordered accumulation.
// ---------------------------------------------------------------------------
constexpr uint32_t kVChunk = 128;  // V rows per LDS buffer

template <bool NEON>
__global__ __launch_bounds__(kThreads) void k_attn(const float *__restrict__ qv, const float *__restrict__ kv,
                                                   const float *__restrict__ vv, const float *__restrict__ cos_tab,
                                                   const float *__restrict__ sin_tab, const pi_state *__restrict__ st,
                                                   float *__restrict__ kc, float *__restrict__ vc, uint32_t group,
                                                   uint32_t n_ctx, uint32_t half, float scale,
                                                   int8_t *__restrict__ oq, float *__restrict__ od,
                                                   int32_t *__restrict__ os) {
    constexpr uint32_t DH = 64;
    extern __shared__ __align__(16) unsigned char smem[];
    float *qs = reinterpret_cast<float *>(smem);           // 64
    float *kcur = qs + DH;                                  // 64
    float *vcur = kcur + DH;                                // 64
    float *red = vcur + DH;                                 // 16
    float *vbuf = red + 16;                                 // 2 * kVChunk * 64
    float *sc = vbuf + 2 * kVChunk * DH;                    // n_ctx
    const uint32_t h = blockIdx.x, kvh = h / group, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
    const int pos = st->pos;
    const uint32_t n = (uint32_t)pos + 1;
    const float *cb = cos_tab + (uint64_t)pos * half, *sb = sin_tab + (uint64_t)pos * half;
    float *kbase = kc + (uint64_t)kvh * n_ctx * DH;
    float *vbase = vc + (uint64_t)kvh * n_ctx * DH;

    // RoPE (model.rs:953-979): pair i = (2i, 2i+1) for i < half
    if (tid < DH / 2) {
        const uint32_t i = tid;
        float x0 = qv[h * DH + 2 * i], x1 = qv[h * DH + 2 * i + 1];
        float y0 = kv[kvh * DH + 2 * i], y1 = kv[kvh * DH + 2 * i + 1];
        if (i < half) {
            const float c = cb[i], s = sb[i];
            const float r0 = x0 * c - x1 * s, r1 = x0 * s + x1 * c;
            const float k0 = y0 * c - y1 * s, k1 = y0 * s + y1 * c;
            x0 = r0; x1 = r1; y0 = k0; y1 = k1;
        }
        qs[2 * i] = x0;
        qs[2 * i + 1] = x1;
        kcur[2 * i] = y0;
        kcur[2 * i + 1] = y1;
    } else if (tid >= 64 && tid < 128) {
        vcur[tid - 64] = vv[kvh * DH + (tid - 64)];
    }
    __syncthreads();
    // KV write (model.rs:984-992)
    if (h % group == 0 && tid < DH) {
        kbase[(uint64_t)pos * DH + tid] = kcur[tid];
        vbase[(uint64_t)pos * DH + tid] = vcur[tid];
    }
    // scores, one position per thread per round
    float mx = -INFINITY;
    for (uint32_t p = tid; p < n; p += kThreads) {
        const float4 *kr4 = (p == (uint32_t)pos) ? reinterpret_cast<const float4 *>(kcur)
                                                 : reinterpret_cast<const float4 *>(kbase + (uint64_t)p * DH);
        float4 kr[16];
#pragma unroll
        for (int i = 0; i < 16; i++) kr[i] = kr4[i];
        const float4 *q4 = reinterpret_cast<const float4 *>(qs);
        float s;
        if constexpr (NEON) {
            float a0[4] = {0.f, 0.f, 0.f, 0.f}, a1[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 qa = q4[2 * i], qb = q4[2 * i + 1], ka = kr[2 * i], kb = kr[2 * i + 1];
                a0[0] = a0[0] + qa.x * ka.x; a0[1] = a0[1] + qa.y * ka.y;
                a0[2] = a0[2] + qa.z * ka.z; a0[3] = a0[3] + qa.w * ka.w;
                a1[0] = a1[0] + qb.x * kb.x; a1[1] = a1[1] + qb.y * kb.y;
                a1[2] = a1[2] + qb.z * kb.z; a1[3] = a1[3] + qb.w * kb.w;
            }
            s = (a0[0] + a0[1]) + (a0[2] + a0[3]);
            s += (a1[0] + a1[1]) + (a1[2] + a1[3]);
        } else {
            s = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float4 qa = q4[i], ka = kr[i];
                s += qa.x * ka.x;
                s += qa.y * ka.y;
                s += qa.z * ka.z;
                s += qa.w * ka.w;
            }
        }
        s = s * scale;
        sc[p] = s;
        mx = fmaxf(mx, s);
    }
#pragma unroll
    for (int off = 32; off; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (uint32_t p = tid; p < n; p += kThreads) sc[p] = pi_expf(sc[p] - mx);

    // values: wavefronts 1-3 stage chunks, wavefront 0 accumulates in order
    const uint32_t nchunk = (n + kVChunk - 1) / kVChunk;
    auto stage = [&](uint32_t c) {
        float4 *dst = reinterpret_cast<float4 *>(vbuf + (c & 1u) * kVChunk * DH);
        const uint32_t r0 = c * kVChunk, rows = min(kVChunk, n - r0);
        for (uint32_t i = tid - 64; i < rows * 16; i += kThreads - 64) {
            const uint32_t r = r0 + i / 16, c4 = i % 16;
            dst[i] = (r == (uint32_t)pos) ? reinterpret_cast<const float4 *>(vcur)[c4]
                                          : reinterpret_cast<const float4 *>(vbase + (uint64_t)r * DH)[c4];
        }
    };
    if (wave != 0) stage(0);
    __syncthreads();
    float acc = 0.0f, sum = 0.0f;
    for (uint32_t c = 0; c < nchunk; c++) {
        if (wave != 0) {
            if (c + 1 < nchunk) stage(c + 1);
        } else {
            const float *vb = vbuf + (c & 1u) * kVChunk * DH;
            const uint32_t r0 = c * kVChunk, rows = min(kVChunk, n - r0);
            for (uint32_t r = 0; r < rows; r++) {
                const float e = sc[r0 + r];
                sum += e;
                const float t = acc + e * vb[r * DH + lane];
                acc = (e != 0.0f) ? t : acc;
            }
        }
        __syncthreads();
    }
    if (wave == 0) {
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        const float o = acc * inv;
        const uint32_t blk = h * 2 + lane / 32;
        q8_block32(o, (int)(lane % 32), oq + blk * 32, od + blk, os + blk, true);
    }
}

// ---------------------------------------------------------------------------
// Step kernel (one workgroup).  MODE_ARGMAX: reduce the head's partials to the
// greedy id (sampler.rs:26-36, first index of the max, NaN never wins),
// record it, advance the position.  MODE_PROMPT: advance to the next prompt
// token.  MODE_EMBED: keep the state.  Then embed st->tok into x
// (dequant_row of token_embd, model.rs:857-869).
// ---------------------------------------------------------------------------
template <int MODE>
__global__ __launch_bounds__(kThreads) void k_step(const float *__restrict__ pv, const uint32_t *__restrict__ pidx,
                                                   uint32_t np, pi_state *__restrict__ st, uint32_t *__restrict__ ids,
                                                   const uint32_t *__restrict__ prompt, const uint8_t *__restrict__ E,
                                                   uint32_t etype, uint32_t ne, uint64_t row_bytes,
                                                   float *__restrict__ x) {
    __shared__ uint32_t tok_s;
    const uint32_t tid = threadIdx.x;
    if constexpr (MODE == PI_STEP_ARGMAX) {
        float bv = -INFINITY;
        uint32_t bi = 0xFFFFFFFFu;
        for (uint32_t i = tid; i < np; i += kThreads) amax_merge(bv, bi, pv[i], pidx[i]);
#pragma unroll
        for (int off = 32; off; off >>= 1) {
            const float ov = __shfl_xor(bv, off, 64);
            const uint32_t oi = __shfl_xor(bi, off, 64);
            amax_merge(bv, bi, ov, oi);
        }
        __shared__ float sv[kThreads / 64];
        __shared__ uint32_t si[kThreads / 64];
        if ((tid & 63u) == 0) {
            sv[tid >> 6] = bv;
            si[tid >> 6] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            for (uint32_t w = 1; w < kThreads / 64; w++) amax_merge(bv, bi, sv[w], si[w]);
            if (bi == 0xFFFFFFFFu) bi = 0;
            st->tok = bi;
            if (ids) ids[st->n_gen] = bi;
            st->n_gen += 1;
            st->pos += 1;
            tok_s = bi;
        }
    } else if constexpr (MODE == PI_STEP_PROMPT) {
        if (tid == 0) {
            st->pos += 1;
            st->i += 1;
            st->tok = prompt[st->i];
            tok_s = st->tok;
        }
    } else {
        if (tid == 0) tok_s = st->tok;
    }
    __syncthreads();
    const uint8_t *row = E + (uint64_t)tok_s * row_bytes;
    for (uint32_t e = tid; e < ne; e += kThreads) x[e] = embed_elem(row, etype, e);
}

MatSet to_set(const pi_matset &M) {
    MatSet S{};
    for (int i = 0; i < 3; i++) {
        S.w[i] = M.w[i];
        S.y[i] = M.y[i];
        S.rows[i] = M.rows[i];
    }
    for (int i = 0; i < 4; i++) S.tile0[i] = M.tile0[i];
    S.n = M.n;
    S.upr = M.L.upr;
    S.rpw = M.L.rpw;
    S.lpt = M.L.lpt;
    S.tile_bytes = M.L.tile_bytes;
    return S;
}

uint32_t strip_bytes(uint32_t tpu) { return ((kThreads / 64) * 64 * tpu + kChainPad) * 4; }

template <bool NEON, uint32_t TA, uint32_t TB, int EPI>
hipError_t launch_norm_gemv(const pi_norm_gemv_args &a, hipStream_t s) {
    constexpr uint32_t TPU = QT<TA>::TPB > QT<TB>::TPB ? QT<TA>::TPB : QT<TB>::TPB;
    const size_t shm = strip_bytes(TPU) + 16 * 4 + (size_t)xs_floats(a.ne) * 4 + act_lds_bytes(a.ne) + 16;
    auto kern = k_norm_gemv<NEON, TA, TB, EPI>;
    hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    hipLaunchKernelGGL(kern, dim3(a.blocks), dim3(kThreads), shm, s, a.x, a.nw, a.ne, a.eps, to_set(a.A), to_set(a.B),
                       a.h, a.pv, a.pidx);
    return hipGetLastError();
}

template <bool NEON, uint32_t TA, int EPI>
hipError_t launch_norm_gemv_tb(const pi_norm_gemv_args &a, hipStream_t s) {
    if (a.B.n == 0 || a.B.L.type == TA) return launch_norm_gemv<NEON, TA, TA, EPI>(a, s);
    if (a.B.L.type == PI_TYPE_Q6_K && TA == PI_TYPE_Q4_K) return launch_norm_gemv<NEON, TA, PI_TYPE_Q6_K, EPI>(a, s);
    if (a.B.L.type == PI_TYPE_Q4_K && TA == PI_TYPE_Q6_K) return launch_norm_gemv<NEON, TA, PI_TYPE_Q4_K, EPI>(a, s);
    return hipErrorInvalidValue;
}

template <bool NEON, int EPI>
hipError_t launch_norm_gemv_ta(const pi_norm_gemv_args &a, hipStream_t s) {
    if (a.A.L.type == PI_TYPE_Q4_K) return launch_norm_gemv_tb<NEON, PI_TYPE_Q4_K, EPI>(a, s);
    if (a.A.L.type == PI_TYPE_Q6_K) return launch_norm_gemv_tb<NEON, PI_TYPE_Q6_K, EPI>(a, s);
    return hipErrorInvalidValue;
}

template <uint32_t T, int G, int PRO>
hipError_t launch_gemv_res_g(const pi_gemv_res_args &a, hipStream_t s) {
    constexpr uint32_t TPU = QT<T>::TPB * G;
    const size_t shm = strip_bytes(TPU) + (PRO == PI_PRO_Q8 ? act_lds_bytes(a.k) : 0) + 16;
    auto kern = k_gemv_res<T, G, PRO>;
    hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    hipLaunchKernelGGL(kern, dim3(a.blocks), dim3(kThreads), shm, s, a.aq, a.ad, a.as, a.hx, a.k, to_set(a.M));
    return hipGetLastError();
}

template <uint32_t T, int PRO>
hipError_t launch_gemv_res_t(const pi_gemv_res_args &a, hipStream_t s) {
    if constexpr (T == PI_TYPE_Q4_K || T == PI_TYPE_Q6_K) {
        return a.M.L.g == 1 ? launch_gemv_res_g<T, 1, PRO>(a, s) : hipErrorInvalidValue;
    } else {
        switch (a.M.L.g) {
        case 1: return launch_gemv_res_g<T, 1, PRO>(a, s);
        case 2: return launch_gemv_res_g<T, 2, PRO>(a, s);
        case 3: return launch_gemv_res_g<T, 3, PRO>(a, s);
        case 4: return launch_gemv_res_g<T, 4, PRO>(a, s);
        case 6: return launch_gemv_res_g<T, 6, PRO>(a, s);
        case 8: return launch_gemv_res_g<T, 8, PRO>(a, s);
        default: return hipErrorInvalidValue;
        }
    }
}

template <uint32_t T, int G>
hipError_t launch_gemv_g(const pi_matset &M, const int8_t *aq, const float *ad, const int32_t *as, int32_t *sums,
                         int mode, uint32_t blocks, hipStream_t s) {
    const MatSet S = to_set(M);
    const dim3 grid((blocks + kGemvThreads / 64 - 1) / (kGemvThreads / 64)), blk(kGemvThreads);   // blocks: wavefronts
    if (mode == PI_GEMV_OUT) hipLaunchKernelGGL((k_gemv<T, G, PI_GEMV_OUT>), grid, blk, 0, s, S, aq, ad, as, sums);
    else if (mode == PI_GEMV_RESIDUAL)
        hipLaunchKernelGGL((k_gemv<T, G, PI_GEMV_RESIDUAL>), grid, blk, 0, s, S, aq, ad, as, sums);
    else hipLaunchKernelGGL((k_gemv<T, G, PI_GEMV_SUMS>), grid, blk, 0, s, S, aq, ad, as, sums);
    return hipGetLastError();
}

template <uint32_t T, int G>
hipError_t launch_gemv_x_g(const pi_matset &M, const float *x, uint32_t blocks, hipStream_t s) {
    const MatSet S = to_set(M);
    constexpr uint32_t TPU = QT<T>::TPB * G;
    const size_t shm = (((kGemvThreads / 64) * 64 * TPU + kChainPad) * 4 + 15) / 16 * 16 + act_q_bytes(M.L.k) +
                       (size_t)(M.L.k / 32) * 8;
    const dim3 grid((blocks + kGemvThreads / 64 - 1) / (kGemvThreads / 64)), blk(kGemvThreads);
    hipError_t e = hipFuncSetAttribute((const void *)k_gemv_x<T, G>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((k_gemv_x<T, G>), grid, blk, shm, s, S, x, M.L.k);
    return hipGetLastError();
}

template <uint32_t T>
hipError_t launch_gemv_x_t(const pi_matset &M, const float *x, uint32_t blocks, hipStream_t s) {
    if constexpr (T == PI_TYPE_Q4_K || T == PI_TYPE_Q6_K) {
        return M.L.g == 1 ? launch_gemv_x_g<T, 1>(M, x, blocks, s) : hipErrorInvalidValue;
    } else {
        switch (M.L.g) {
        case 1: return launch_gemv_x_g<T, 1>(M, x, blocks, s);
        case 2: return launch_gemv_x_g<T, 2>(M, x, blocks, s);
        case 3: return launch_gemv_x_g<T, 3>(M, x, blocks, s);
        case 4: return launch_gemv_x_g<T, 4>(M, x, blocks, s);
        case 6: return launch_gemv_x_g<T, 6>(M, x, blocks, s);
        case 8: return launch_gemv_x_g<T, 8>(M, x, blocks, s);
        default: return hipErrorInvalidValue;
        }
    }
}

template <uint32_t T>
hipError_t launch_gemv_t(const pi_matset &M, const int8_t *aq, const float *ad, const int32_t *as, int32_t *sums,
                         int mode, uint32_t blocks, hipStream_t s) {
    if constexpr (T == PI_TYPE_Q4_K || T == PI_TYPE_Q6_K) {
        return M.L.g == 1 ? launch_gemv_g<T, 1>(M, aq, ad, as, sums, mode, blocks, s) : hipErrorInvalidValue;
    } else {
        switch (M.L.g) {
        case 1: return launch_gemv_g<T, 1>(M, aq, ad, as, sums, mode, blocks, s);
        case 2: return launch_gemv_g<T, 2>(M, aq, ad, as, sums, mode, blocks, s);
        case 3: return launch_gemv_g<T, 3>(M, aq, ad, as, sums, mode, blocks, s);
        case 4: return launch_gemv_g<T, 4>(M, aq, ad, as, sums, mode, blocks, s);
        case 6: return launch_gemv_g<T, 6>(M, aq, ad, as, sums, mode, blocks, s);
        case 8: return launch_gemv_g<T, 8>(M, aq, ad, as, sums, mode, blocks, s);
        default: return hipErrorInvalidValue;
        }
    }
}

}  // namespace

hipError_t pi_launch_gemv_set(const pi_matset &M, const int8_t *aq, const float *ad, const int32_t *as, int32_t *sums,
                              int mode, uint32_t blocks, hipStream_t s) {
    if (M.n < 1 || M.n > 3 || blocks == 0) return hipErrorInvalidValue;
    if (mode == PI_GEMV_SUMS && M.n != 1) return hipErrorInvalidValue;
    switch (M.L.type) {
    case PI_TYPE_Q4_K: return launch_gemv_t<PI_TYPE_Q4_K>(M, aq, ad, as, sums, mode, blocks, s);
    case PI_TYPE_Q6_K: return launch_gemv_t<PI_TYPE_Q6_K>(M, aq, ad, as, sums, mode, blocks, s);
    case PI_TYPE_Q4_0: return launch_gemv_t<PI_TYPE_Q4_0>(M, aq, ad, as, sums, mode, blocks, s);
    case PI_TYPE_Q8_0: return launch_gemv_t<PI_TYPE_Q8_0>(M, aq, ad, as, sums, mode, blocks, s);
    default: return hipErrorInvalidValue;
    }
}

size_t pi_gemv_x_lds_bytes(uint32_t type, uint32_t g, uint32_t k) {
    const uint32_t tpu = (type == PI_TYPE_Q4_K ? 8u : type == PI_TYPE_Q6_K ? 16u : 1u) * g;
    return (((kGemvThreads / 64) * 64 * tpu + kChainPad) * 4 + 15) / 16 * 16 + act_q_bytes(k) + (size_t)(k / 32) * 8;
}

hipError_t pi_launch_gemv_x(const pi_matset &M, const float *x, uint32_t blocks, hipStream_t s) {
    if (M.n < 1 || M.n > 3 || blocks == 0 || !x || M.L.k % 32) return hipErrorInvalidValue;
    switch (M.L.type) {
    case PI_TYPE_Q4_K: return launch_gemv_x_t<PI_TYPE_Q4_K>(M, x, blocks, s);
    case PI_TYPE_Q6_K: return launch_gemv_x_t<PI_TYPE_Q6_K>(M, x, blocks, s);
    case PI_TYPE_Q4_0: return launch_gemv_x_t<PI_TYPE_Q4_0>(M, x, blocks, s);
    case PI_TYPE_Q8_0: return launch_gemv_x_t<PI_TYPE_Q8_0>(M, x, blocks, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t pi_launch_norm_gemv(const pi_norm_gemv_args &a, bool neon, hipStream_t s) {
    if (a.A.n < 1 || a.blocks == 0 || a.ne % 32 || a.ne == 0) return hipErrorInvalidValue;
    if (a.A.L.g != 1 || (a.B.n && a.B.L.g != 1) || (a.B.n && a.B.L.upr != a.A.L.upr)) return hipErrorInvalidValue;
    if (a.epi == PI_EPI_SWIGLU) {
        if (a.A.n != 2 || a.B.n != 0 || a.A.tile0[1] * 2 != a.A.tile0[2] || a.A.rows[0] != a.A.rows[1] || !a.h)
            return hipErrorInvalidValue;
        if (a.A.L.type != PI_TYPE_Q4_K && a.A.L.type != PI_TYPE_Q6_K) return hipErrorInvalidValue;
        return neon ? (a.A.L.type == PI_TYPE_Q4_K ? launch_norm_gemv<true, PI_TYPE_Q4_K, PI_TYPE_Q4_K, PI_EPI_SWIGLU>(a, s)
                                                  : launch_norm_gemv<true, PI_TYPE_Q6_K, PI_TYPE_Q6_K, PI_EPI_SWIGLU>(a, s))
                    : (a.A.L.type == PI_TYPE_Q4_K ? launch_norm_gemv<false, PI_TYPE_Q4_K, PI_TYPE_Q4_K, PI_EPI_SWIGLU>(a, s)
                                                  : launch_norm_gemv<false, PI_TYPE_Q6_K, PI_TYPE_Q6_K, PI_EPI_SWIGLU>(a, s));
    }
    if (a.epi == PI_EPI_ARGMAX) {
        if (a.A.n != 1 || a.B.n != 0 || !a.pv || !a.pidx) return hipErrorInvalidValue;
        return neon ? launch_norm_gemv_ta<true, PI_EPI_ARGMAX>(a, s) : launch_norm_gemv_ta<false, PI_EPI_ARGMAX>(a, s);
    }
    return neon ? launch_norm_gemv_ta<true, PI_EPI_OUT>(a, s) : launch_norm_gemv_ta<false, PI_EPI_OUT>(a, s);
}

hipError_t pi_launch_gemv_res(const pi_gemv_res_args &a, hipStream_t s) {
    if (a.M.n < 1 || a.blocks == 0) return hipErrorInvalidValue;
    if (a.pro == PI_PRO_Q8 && (!a.hx || a.k % 32 || a.k != a.M.L.k)) return hipErrorInvalidValue;
    if (a.pro == PI_PRO_GLOBAL && (!a.aq || !a.ad || !a.as)) return hipErrorInvalidValue;
    switch (a.M.L.type) {
    case PI_TYPE_Q4_K: return a.pro == PI_PRO_Q8 ? launch_gemv_res_t<PI_TYPE_Q4_K, PI_PRO_Q8>(a, s) : launch_gemv_res_t<PI_TYPE_Q4_K, PI_PRO_GLOBAL>(a, s);
    case PI_TYPE_Q6_K: return a.pro == PI_PRO_Q8 ? launch_gemv_res_t<PI_TYPE_Q6_K, PI_PRO_Q8>(a, s) : launch_gemv_res_t<PI_TYPE_Q6_K, PI_PRO_GLOBAL>(a, s);
    case PI_TYPE_Q4_0: return a.pro == PI_PRO_Q8 ? launch_gemv_res_t<PI_TYPE_Q4_0, PI_PRO_Q8>(a, s) : launch_gemv_res_t<PI_TYPE_Q4_0, PI_PRO_GLOBAL>(a, s);
    case PI_TYPE_Q8_0: return a.pro == PI_PRO_Q8 ? launch_gemv_res_t<PI_TYPE_Q8_0, PI_PRO_Q8>(a, s) : launch_gemv_res_t<PI_TYPE_Q8_0, PI_PRO_GLOBAL>(a, s);
    default: return hipErrorInvalidValue;
    }
}

size_t pi_attn_lds_bytes(uint32_t n_ctx) { return (size_t)(64 * 3 + 16 + 2 * kVChunk * 64 + n_ctx) * 4 + 16; }

hipError_t pi_launch_attn(const pi_attn_args &a, bool neon, hipStream_t s) {
    if (a.dh != 64 || a.n_head == 0 || a.n_kv == 0 || a.n_head % a.n_kv) return hipErrorInvalidValue;
    const size_t shm = pi_attn_lds_bytes(a.n_ctx);
    const uint32_t group = a.n_head / a.n_kv;
    if (neon) {
        hipFuncSetAttribute((const void *)k_attn<true>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
        hipLaunchKernelGGL(k_attn<true>, dim3(a.n_head), dim3(kThreads), shm, s, a.q, a.k, a.v, a.cos_tab, a.sin_tab,
                           a.st, a.kc, a.vc, group, a.n_ctx, a.half, a.scale, a.oq, a.od, a.os);
    } else {
        hipFuncSetAttribute((const void *)k_attn<false>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
        hipLaunchKernelGGL(k_attn<false>, dim3(a.n_head), dim3(kThreads), shm, s, a.q, a.k, a.v, a.cos_tab, a.sin_tab,
                           a.st, a.kc, a.vc, group, a.n_ctx, a.half, a.scale, a.oq, a.od, a.os);
    }
    return hipGetLastError();
}

hipError_t pi_launch_step(int mode, const float *pv, const uint32_t *pidx, uint32_t np, pi_state *st, uint32_t *ids,
                          const uint32_t *prompt, const uint8_t *E, uint32_t etype, uint32_t ne, uint64_t row_bytes,
                          float *x, hipStream_t s) {
    if (mode == PI_STEP_ARGMAX)
        hipLaunchKernelGGL(k_step<PI_STEP_ARGMAX>, dim3(1), dim3(kThreads), 0, s, pv, pidx, np, st, ids, prompt, E,
                           etype, ne, row_bytes, x);
    else if (mode == PI_STEP_PROMPT)
        hipLaunchKernelGGL(k_step<PI_STEP_PROMPT>, dim3(1), dim3(kThreads), 0, s, pv, pidx, np, st, ids, prompt, E,
                           etype, ne, row_bytes, x);
    else
        hipLaunchKernelGGL(k_step<PI_STEP_EMBED>, dim3(1), dim3(kThreads), 0, s, pv, pidx, np, st, ids, prompt, E,
                           etype, ne, row_bytes, x);
    return hipGetLastError();
}
